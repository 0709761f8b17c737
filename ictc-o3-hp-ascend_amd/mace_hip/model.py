"""MACE-style ICTC model (the baseline route of the reference's PureCartesianICTDFix)
running its equivariant operators on the HIP kernels of ``ictc_o3``.

Architecture (reference ``mace_ictc/models/pure_cartesian_ictd_fix.py``; factory
``mace_ictc/hp/runtime.py:7-81`` with ``freeze_conv_tp_weight=True``, Bessel basis of 8,
``radial_sqrt_num_basis=False``, polynomial cutoff p = 5):

  h_0 = node_embedding[species]                                   (:3008-3011)
  for t in 0..T-1:
    interaction_t (:1452-2055):
      x1    = linear_up(h_t)                     per-l C x C, identity init
      gates = fc(bessel(r))                      8 -> 64 -> 64 -> 64 -> P*C, normalised SiLU
      m     = sum_{e -> n} mask_e TP(x1[src_e], Y_e, gates_e)   (fused message, HIP)
      msg   = message_linear(m) / avg_num_neighbors             (per-l, path-preserving)
      sc    = self_connection(h_t l=0 block, species)           (element-conditioned)
    product_t (:1145-1195):  h_{t+1} = Linear(SC(msg, species)) + sc   (SC on HIP)
    energy  += readout_t(h_{t+1})                                (:3095-3101)
  layer 0 has input degree 0 (paths (0,l,l)); the last product targets l = 0.

Dense layers (radial MLP, channel linears, readouts) go through ``mace_hip.linear`` (one GEMM
per layer and degree; weight gradients reduced in row blocks).  The edge directions and the
Bessel x cutoff embedding come from ``mace_hip.embedding`` (one HIP kernel per derivative order).

Layouts.  Node features between blocks are the reference's flat mul_ir layout
``[N, C*(L+1)^2]`` (degree blocks ``[C, 2l+1]``), which the symmetric-contraction
kernels read directly.  ``linear_up`` writes the channel-contiguous ir_mul layout the
message kernels read (the transpose is folded into its GEMM), and ``message_linear``
reads the message kernel's packed ir_mul output and writes mul_ir (again folded).
The product's symmetric contraction is the bridge-U module (``ICTDBridgeUProductBasisBlockSO3``,
the reference's default ``ictd-bridge-u`` backend, :1145-1195); the surrounding ``o3.Linear`` is
restated as a per-degree C x C map with weights ~ N(0, 1) scaled by 1/sqrt(C) (e3nn's element
normalisation for one path).  Every sum over atoms or edges has a fixed order (HIP kernels over
CSR rows, GEMMs against indicator rows), so energies, forces and training gradients are
bit-identical from run to run.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from ictc_o3.backends.hip.degree_linear import (DegreeLinearPlan, degree_linear, degree_linear_adjoint,
                                                 degree_linear_mul_ir)
from ictc_o3.backends.hip.graph_message import message_bonds, packed_graph_message
from ictc_o3.backends.hip.harmonics import direction_harmonics_packed
from ictc_o3.backends.hip.radial_message import fold_projection, packed_radial_graph_message
from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
from ictc_o3.ops.symmetric_contraction import ICTDBridgeUSymmetricContractionSO3

from . import radial_mlp, species_linear
from .readout import readout, supported as readout_supported
from .activation import silu
from .embedding import edge_embedding
from .geometry import edge_vectors, one_hot_rows
from .linear import Linear, linear
from .radial import bessel_embedding

SILU_SCALE = 1.6791767923989418   # _Normalize2MomSiLU (pure_cartesian_ictd_fix.py:610-619)


def tp_paths(input_lmax: int, edge_lmax: int, target_lmax: int):
    """_tp_allowed_paths_from_target_lmax (pure_cartesian_ictd_fix.py:298-319)."""
    return [(a, b, c) for a in range(input_lmax + 1) for b in range(edge_lmax + 1)
            for c in range(abs(a - b), a + b + 1) if c <= target_lmax and (a + b + c) % 2 == 0]


class NormalizedSiLU(nn.Module):
    def forward(self, x):
        return F.silu(x) * SILU_SCALE


def _mace_linear(fan_in: int, fan_out: int) -> Linear:
    lin = Linear(fan_in, fan_out)
    nn.init.normal_(lin.weight, mean=0.0, std=1.0 / math.sqrt(fan_in))
    return lin


class ChannelLinear(nn.Module):
    """EquivariantChannelLinearSO3 (ictd_irreps.py:187-207): per-degree C x C, identity init."""

    def __init__(self, channels: int, lmax: int):
        super().__init__()
        self.channels, self.lmax = channels, lmax
        self.weights = nn.ParameterList([nn.Parameter(torch.eye(channels)) for _ in range(lmax + 1)])
        self.plan = DegreeLinearPlan([1] * (lmax + 1), channels, channels)

    def to_ir_mul(self, x: torch.Tensor) -> torch.Tensor:
        """mul_ir [N, C(L+1)^2] -> ir_mul [N, sum_l (2l+1) C]: out[n, m, o] = sum_c W[o,c] x[n,c,m],
        one fp32-MFMA launch over every degree (the message linear's adjoint kernel with the
        weights transposed; the layout change folded into its tile loads and stores)."""
        width = self.channels * (self.lmax + 1) ** 2
        if x.shape[1] != width:
            x = x[:, :width]
        return degree_linear_adjoint(x, [w.t() for w in self.weights], self.plan)


class MessageLinear(nn.Module):
    """PathPreservingLinearSO3 (pure_cartesian_ictd_fix.py:629-661) reading the packed ir_mul
    message (per degree: [count_l paths][2l+1][C]) and writing mul_ir [N, C(L+1)^2]: one
    fp32-MFMA launch over every degree (degree_linear), the layout changes folded into its tile
    loads and stores and the 1/avg_num_neighbors scale passed as its alpha."""

    def __init__(self, counts: Dict[int, int], channels: int, lmax: int):
        super().__init__()
        self.channels, self.lmax = channels, lmax
        self.counts = [int(counts.get(l, 0)) for l in range(lmax + 1)]
        self.plan = DegreeLinearPlan(self.counts, channels, channels)
        self.weights = nn.ParameterList()
        for l in range(lmax + 1):
            fan_in = channels * self.counts[l]
            w = torch.empty(channels, fan_in)
            if fan_in:
                nn.init.normal_(w, mean=0.0, std=1.0 / math.sqrt(fan_in))
            self.weights.append(nn.Parameter(w))

    def forward(self, m: torch.Tensor, alpha: float = 1.0) -> torch.Tensor:
        if m.shape[1] != self.plan.in_width:
            raise ValueError(f"message width {m.shape[1]} differs from the linear's {self.plan.in_width}")
        return degree_linear(m, list(self.weights), self.plan, alpha)


class SpeciesLinear(nn.Module):
    """ElementConditionedLinearSO3 on a scalar block [N, C] (identity init,
    pure_cartesian_ictd_fix.py:335-390, 140-158): out[n] = W[s_n] x[n]."""

    def __init__(self, num_elements: int, channels: int):
        super().__init__()
        self.num_elements, self.channels = num_elements, channels
        self.weight = nn.Parameter(torch.eye(channels).unsqueeze(0).repeat(num_elements, 1, 1))

    def forward(self, x: torch.Tensor, species: torch.Tensor) -> torch.Tensor:
        s, c = self.num_elements, self.channels
        if species_linear.supported(x, self.weight, species):
            # a frozen weight: one kernel per node block (and its transpose as the adjoint)
            return species_linear.species_linear(x, self.weight, species)
        # all species at once (one GEMM), then pick each node's own block
        y = linear(x, self.weight.reshape(s * c, c)).reshape(-1, s, c)
        return y.gather(1, species.view(-1, 1, 1).expand(-1, 1, c)).squeeze(1)


class IrrepsLinear(nn.Module):
    """e3nn o3.Linear on C x (0..L): per degree out = W x / sqrt(C), W ~ N(0, 1)."""

    def __init__(self, channels: int, lmax: int):
        super().__init__()
        self.channels, self.lmax = channels, lmax
        self.weights = nn.ParameterList([nn.Parameter(torch.randn(channels, channels)) for _ in range(lmax + 1)])
        self.plan = DegreeLinearPlan([1] * (lmax + 1), channels, channels)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """One fp32-MFMA launch over every degree, mul_ir in and out, 1/sqrt(C) as its alpha."""
        return degree_linear_mul_ir(x, list(self.weights), self.plan, 1.0 / math.sqrt(self.channels))


class Interaction(nn.Module):
    def __init__(self, *, channels: int, input_lmax: int, edge_lmax: int, num_elements: int, num_basis: int,
                 avg_num_neighbors: float):
        super().__init__()
        self.channels, self.input_lmax, self.edge_lmax = channels, input_lmax, edge_lmax
        self.avg_num_neighbors = float(avg_num_neighbors)
        self.linear_up = ChannelLinear(channels, input_lmax)
        self.tp = EdgeWeightedPathPreservingTensorProduct(channels, edge_lmax,
                                                          allowed_paths=tp_paths(input_lmax, edge_lmax, edge_lmax))
        with torch.no_grad():
            self.tp.weight.fill_(1.0)          # _init_path_tp_weight_to_one_, then frozen
        self.tp.weight.requires_grad_(False)
        self.fc = nn.Sequential(_mace_linear(num_basis, 64), NormalizedSiLU(), _mace_linear(64, 64),
                                NormalizedSiLU(), _mace_linear(64, 64), NormalizedSiLU(),
                                _mace_linear(64, self.tp.num_paths * channels))
        self.message_linear = MessageLinear(self.tp.path_counts_by_l, channels, edge_lmax)
        # None: the gates are one [E, P*C] tensor; an int: radial streaming over receiver ranges of
        # at most that many edges (the reference's _ascend_edge_chunk_size)
        self.edge_chunk_size: Optional[int] = None
        self._gate_weight = None   # (weights' identity and version, folded last-layer weight) when frozen
        self.self_connection = SpeciesLinear(num_elements, channels)

    def radial_hidden(self, edge_feats):
        """self.fc up to its last Linear: (the last layer's input [E, 64], its weight [P*C, 64]),
        each normalised SiLU's constant folded into the next layer's weight instead of scaling
        the [E, 64] activations.  On the GPU the three layers and their activations run as one
        kernel per derivative order (mace_hip.radial_mlp)."""
        return self._hidden(edge_feats), self.fc[-1].weight * SILU_SCALE

    def _hidden(self, edge_feats):
        layers = [m for m in self.fc if isinstance(m, nn.Linear)]
        w = [lin.weight for lin in layers]
        if len(layers) == 4 and radial_mlp.supported(edge_feats, *w[:3]):
            return radial_mlp.radial_hidden(edge_feats, *w[:3], SILU_SCALE)
        h = layers[0](edge_feats)
        for lin in layers[1:-1]:
            h = linear(silu(h), lin.weight * SILU_SCALE)
        return silu(h)

    def radial_mlp(self, edge_feats):
        """self.fc on the edge features: the gates [E, P*C]."""
        hidden, weight = self.radial_hidden(edge_feats)
        return linear(hidden, weight)

    def message_gates(self, edge_feats):
        """The gates times the TP's frozen path weight (the reference's gates * weight,
        ``backends/ascend/packed_tensor_product.py:163-164``), folded into the rows of the radial
        MLP's last weight ([P*C, 64]) rather than applied to the [E, P*C] gates.  With no gradient
        to either weight the folded [P*C, 64] weight is kept until one of them is replaced or
        modified in place."""
        hidden = self._hidden(edge_feats)
        last = self.fc[-1].weight
        if torch.is_grad_enabled() and (last.requires_grad or self.tp.weight.requires_grad):
            return linear(hidden, last * SILU_SCALE * self.tp.weight.reshape(-1, 1))
        key = tuple((id(t), t.data_ptr(), t._version) for t in (last, self.tp.weight))
        if self._gate_weight is None or self._gate_weight[0] != key:
            self._gate_weight = (key, last * SILU_SCALE * self.tp.weight.reshape(-1, 1))
        return linear(hidden, self._gate_weight[1])

    def message_bonds(self, harmonics):
        """The bond rows the message forward derives from the harmonics (see forward's bonds)."""
        return message_bonds(self.tp.hip_plan(self.input_lmax, self.edge_lmax), harmonics)

    def forward(self, h, harmonics, edge_feats, src, dst, mask, species, scalars=None, gates=None, bonds=None):
        """mask: the reference multiplies the gates by (r <= r_max) (:1801-1808).  The radial
        features carry the cutoff envelope, exactly 0 from r_max on, and fc has no biases, so
        the gates are already exactly 0 wherever the mask is 0: the product is an identity and
        is skipped (mask is accepted for the signature).  scalars: h's l = 0 block as its own
        tensor when the caller has it (the previous product's), so the self connection does not
        slice h (a slice's backward zero-fills a gradient of h's full width).  gates: this
        interaction's message gates, and bonds the bond rows of the harmonics, when the caller has
        produced them already (on a side stream)."""
        n = h.shape[0]
        x1 = self.linear_up.to_ir_mul(h)
        plan = self.tp.hip_plan(self.input_lmax, self.edge_lmax)
        if self.edge_chunk_size is None:
            if gates is None:
                gates = self.message_gates(edge_feats)
            m = packed_graph_message(plan, x1, harmonics, gates, src, dst, nodes_dst=n, bonds=bonds)
        else:
            # the radial MLP's last layer produced one receiver range at a time inside the message
            # (reference capacity mode, capacity_message.py:109-179): no [E, P*C] gate tensor
            hidden, weight = self.radial_hidden(edge_feats)
            weight, _ = fold_projection(self.tp, plan, weight, None)
            m = packed_radial_graph_message(plan, x1, harmonics, hidden, weight, None, src, dst, nodes_dst=n,
                                            edge_chunk_size=self.edge_chunk_size)
        message = self.message_linear(m, 1.0 / max(self.avg_num_neighbors, 1e-8))
        sc = self.self_connection(h[:, :self.channels] if scalars is None else scalars, species)
        return message, sc


class Product(nn.Module):
    def __init__(self, *, channels: int, lmax: int, target_lmax: int, correlation: int, num_elements: int):
        super().__init__()
        self.channels, self.target_lmax = channels, target_lmax
        # ICTDBridgeUProductBasisBlockSO3 (:1145-1195): the bridge-U contraction the reference ships
        self.symmetric_contractions = ICTDBridgeUSymmetricContractionSO3(
            num_elements=num_elements, channels=channels, lmax=lmax, target_lmax=target_lmax,
            correlation=correlation)
        self.linear = IrrepsLinear(channels, target_lmax)

    def forward(self, message, sc, species):
        """(node features, their l = 0 block): the block is returned as the tensor the features
        are concatenated from, so its users need no slice of them."""
        out = self.linear(self.symmetric_contractions(message, node_type_idx=species))
        # _add_product_self_connection (:94-118): an l = 0 skip lands on the scalar block
        scalar, rest = out.split([self.channels, out.shape[1] - self.channels], dim=-1)
        scalar = scalar + sc
        return (torch.cat([scalar, rest], dim=-1) if rest.shape[1] else scalar), scalar


_SIDE_STREAMS: Dict[int, torch.cuda.Stream] = {}


def _side_stream(device: torch.device) -> "torch.cuda.Stream":
    """One default-priority side stream per device, created once."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    stream = _SIDE_STREAMS.get(index)
    if stream is None:
        stream = torch.cuda.Stream(device=index)
        _SIDE_STREAMS[index] = stream
    return stream


class MaceICTC(nn.Module):
    def __init__(self, *, channels: int = 128, lmax: int = 3, num_interactions: int = 2, correlation: int = 3,
                 atomic_numbers=tuple(range(1, 11)), cutoff: float = 5.0, avg_num_neighbors: float = 50.0,
                 num_basis: int = 8, cutoff_p: int = 5, readout_hidden: int = 16):
        super().__init__()
        self.channels, self.lmax, self.cutoff = int(channels), int(lmax), float(cutoff)
        self.num_basis, self.cutoff_p = int(num_basis), int(cutoff_p)
        # radial MLPs and gates on a second stream beside the interactions (GPU, whole gates)
        self.overlap_radial = True
        self.atomic_numbers = [int(z) for z in atomic_numbers]
        self.num_elements = len(self.atomic_numbers)
        table = torch.full((max(self.atomic_numbers) + 1,), -1, dtype=torch.int64)
        for i, z in enumerate(self.atomic_numbers):
            table[z] = i
        self.register_buffer("atomic_number_to_index", table, persistent=False)
        self.node_embedding = nn.Linear(self.num_elements, self.channels, bias=False)
        targets = [self.lmax if t < num_interactions - 1 else 0 for t in range(num_interactions)]
        self.interactions = nn.ModuleList()
        self.products = nn.ModuleList()
        for t, target in enumerate(targets):
            self.interactions.append(Interaction(channels=self.channels, input_lmax=0 if t == 0 else self.lmax,
                                                 edge_lmax=self.lmax, num_elements=self.num_elements,
                                                 num_basis=self.num_basis, avg_num_neighbors=avg_num_neighbors))
            self.products.append(Product(channels=self.channels, lmax=self.lmax, target_lmax=target,
                                         correlation=correlation, num_elements=self.num_elements))
        # EquivariantScalarReadoutSO3 (pure_cartesian_ictd_layers.py:46-70) per inner layer and the
        # MACE-style MLP readout (pure_cartesian_ictd_fix.py:1434-1449) after the last one
        self.layer_readouts = nn.ModuleList([_mace_linear(self.channels, 1) for _ in range(num_interactions - 1)])
        self.last_readout = nn.Sequential(_mace_linear(self.channels, readout_hidden), NormalizedSiLU(),
                                          _mace_linear(readout_hidden, 1))

    def set_message_streaming(self, edge_chunk_size: Optional[int]) -> None:
        """Radial streaming in every interaction (receiver ranges of at most ``edge_chunk_size``
        edges), or None for whole gate tensors."""
        if edge_chunk_size is not None and (not isinstance(edge_chunk_size, int) or edge_chunk_size < 1):
            raise ValueError("Edge chunk size must be a positive integer or None")
        for interaction in self.interactions:
            interaction.edge_chunk_size = edge_chunk_size

    def species_index(self, atomic_numbers: torch.Tensor) -> torch.Tensor:
        a = atomic_numbers.long()
        if int(a.max()) >= self.atomic_number_to_index.numel() or int(a.min()) < 0:
            raise ValueError(f"atomic numbers outside the configured set {self.atomic_numbers}")
        idx = self.atomic_number_to_index[a]
        if bool((idx < 0).any()):
            raise ValueError(f"atomic numbers outside the configured set {self.atomic_numbers}")
        return idx

    def forward(self, pos, atomic_numbers, batch, edge_src, edge_dst, edge_shifts, cell, species=None):
        """Atomic energies [N] (reference forward :2879-3106, baseline route)."""
        # shift_e @ cell_e as three multiply-adds per edge (not a batched GEMM of 3 x 3 matrices)
        # index_select rather than advanced indexing (cheaper to issue; same gather)
        # (one structure: its cell broadcast over the edges, no per-edge gather of it)
        edge_cell = (cell[0] if cell.shape[0] == 1 else cell.index_select(0, batch.index_select(0, edge_src))).to(pos.dtype)
        shift_vecs = (edge_shifts.to(pos.dtype).unsqueeze(-1) * edge_cell).sum(1)
        # pos[dst] - pos[src] with a fixed-order (atomic-free) adjoint: forces are reproducible
        vec = edge_vectors(pos, edge_src, edge_dst) + shift_vecs
        if vec.dtype == torch.float32 and self.cutoff_p is not None:
            # directions and the radial embedding in one kernel per derivative order; the interaction
            # takes no cutoff mask (its gates are exactly zero from r_max on, see Interaction.forward)
            directions, edge_feats = edge_embedding(vec, r_max=self.cutoff, num_basis=self.num_basis,
                                                    cutoff_p=self.cutoff_p)
            mask = None
        else:
            length = vec.norm(dim=1)
            directions = vec / length.clamp(min=1e-8).unsqueeze(-1)
            mask = (length <= self.cutoff).to(pos.dtype)
            edge_feats = bessel_embedding(length, r_max=self.cutoff, num_basis=self.num_basis,
                                          cutoff_p=self.cutoff_p)
        harmonics = direction_harmonics_packed(directions, self.lmax)
        if species is None:
            species = self.species_index(atomic_numbers)
        # the embedding as the product one_hot(species) @ W^T (the reference's node_embedding on
        # one-hot attributes): its weight gradient is a GEMM, not an atomic index_add; a frozen
        # embedding (inference) is the same rows picked directly
        if self.node_embedding.weight.requires_grad and torch.is_grad_enabled():
            h = linear(one_hot_rows(species, self.num_elements), self.node_embedding.weight)
        else:
            h = self.node_embedding.weight.t().index_select(0, species)
        side = self._side_work(edge_feats, harmonics)
        energy = None
        scalars = h
        last = len(self.interactions) - 1
        deferred = None   # the second-to-last layer's scalars, read out with the last layer's
        for t, (interaction, product) in enumerate(zip(self.interactions, self.products)):
            gates = bonds = None
            if side is not None:
                gates, bonds, ready = side[t]
                torch.cuda.current_stream(pos.device).wait_event(ready)
            message, sc = interaction(h, harmonics, edge_feats, edge_src, edge_dst, mask, species, scalars,
                                      gates, bonds)
            h, scalars = product(message, sc, species)
            if t == last - 1 and self._fused_readout(scalars, h):
                deferred = scalars
                continue
            if t < last:
                e = self.layer_readouts[t](scalars)
            elif deferred is not None:
                lin1, _, lin2 = self.last_readout
                e = readout(deferred, h, self.layer_readouts[t - 1].weight, lin1.weight, lin2.weight, SILU_SCALE)
            else:
                e = self.last_readout(h)
            energy = e if energy is None else energy + e
        if side is not None:   # join the side stream (nothing left on it unwaited, also under capture)
            torch.cuda.current_stream(pos.device).wait_stream(_side_stream(pos.device))
        return energy.reshape(-1)

    def _fused_readout(self, scalars, h):
        """Whether the second-to-last layer's readout and the last layer's run as one kernel
        (mace_hip.readout: frozen fp32 GPU weights, the last readout Linear -> SiLU -> Linear)."""
        if len(self.interactions) < 2 or len(self.last_readout) != 3:
            return False
        lin1, act, lin2 = self.last_readout
        if not isinstance(act, NormalizedSiLU) or lin2.weight.shape[0] != 1:
            return False
        w_lin = self.layer_readouts[len(self.interactions) - 2].weight
        return w_lin.shape[0] == 1 and readout_supported(scalars, scalars, w_lin, lin1.weight, lin2.weight)

    def _side_work(self, edge_feats, harmonics):
        """Each interaction's message gates (radial MLP and its [E, P*C] last layer) and bond rows,
        issued on a second stream: they depend only on the edge features and harmonics, so
        interaction t+1's run beside interaction t's message, contraction and linears, and the
        autograd engine runs their adjoints on that stream too (beside the other interaction's
        backward).  Returns [(gates, bonds, ready event)] per interaction, or None where this does
        not apply (CPU, radial streaming)."""
        if not (self.overlap_radial and edge_feats.is_cuda
                and all(i.edge_chunk_size is None for i in self.interactions)):
            return None
        main = torch.cuda.current_stream(edge_feats.device)
        side = _side_stream(edge_feats.device)
        side.wait_stream(main)
        out = []
        with torch.cuda.stream(side):
            for interaction in self.interactions:
                gates = interaction.message_gates(edge_feats)
                bonds = interaction.message_bonds(harmonics)
                ev = torch.cuda.Event()
                ev.record(side)
                out.append((gates, bonds, ev))
        for gates, bonds, _ in out:   # used on the main stream: not reusable by side allocations before
            gates.record_stream(main)
            if bonds is not None:
                bonds.record_stream(main)
        for t in (edge_feats, harmonics):   # read on the side stream: not reusable on the main one before
            t.record_stream(side)
        return out
