"""CPU float64 restatement of the MACE-style ICTC energy model (test infrastructure only).

Follows the reference's baseline route (``mace_ictc/models/pure_cartesian_ictd_fix.py``):
edge geometry and masks (:2914-2937), ICTC direction harmonics (``ictd_irreps.py:1113-1168``),
Bessel x polynomial-cutoff radial features (``radial_basis.py:11-92``), the interaction
block (:1762-2055: linear_up, radial MLP ``fc`` :1545-1553, gather -> TP -> mask ->
index_add message, path-preserving message linear / avg_num_neighbors, element-conditioned
self connection), the product block (:1145-1195 with the module's bridge-U contraction, o3.Linear,
``_add_product_self_connection`` :94-118) and the readouts (:1434-1449,
``pure_cartesian_ictd_layers.py:46-70``); energy and forces as ``hp/runtime.py:84-119``.

Every equivariant operation goes through this package's own oracles (TensorProductOracle,
SymmetricContractionOracle, ictc_basis.direction_harmonics_all); the parameters are read by
name from a state dict, so the oracle evaluates exactly the function the GPU model holds.
"""
from __future__ import annotations

import math
from typing import Dict

import torch
import torch.nn.functional as F

from . import ictc_basis as basis
from .symmetric_contraction import SymmetricContractionOracle
from .tensor_product import TensorProductOracle

SILU_SCALE = 1.6791767923989418


def polynomial_cutoff(r, r_max, p):
    x = r / r_max
    env = (1.0 - (p + 1.0) * (p + 2.0) / 2.0 * x ** p + p * (p + 2.0) * x ** (p + 1)
           - p * (p + 1.0) / 2.0 * x ** (p + 2))
    return env * (r < r_max).to(r.dtype)


def bessel_features(r, r_max, num_basis, p):
    n = torch.arange(1, num_basis + 1, dtype=r.dtype)
    e = math.sqrt(2.0 / r_max) * torch.sin(n * math.pi * r[:, None] / r_max) / r.clamp_min(1e-12)[:, None]
    return e * polynomial_cutoff(r, r_max, p)[:, None]


def _silu(x):
    return F.silu(x) * SILU_SCALE


def _paths(input_lmax, edge_lmax, target_lmax):
    return [(a, b, c) for a in range(input_lmax + 1) for b in range(edge_lmax + 1)
            for c in range(abs(a - b), a + b + 1) if c <= target_lmax and (a + b + c) % 2 == 0]


def _blocks(x, c, lmax):
    out, off = {}, 0
    for l in range(lmax + 1):
        out[l] = x[:, off:off + c * (2 * l + 1)].reshape(-1, c, 2 * l + 1)
        off += c * (2 * l + 1)
    return out


def _flat(blocks):
    return torch.cat([blocks[l].reshape(blocks[l].shape[0], -1) for l in sorted(blocks)], -1)


class MaceOracle:
    def __init__(self, params: Dict[str, torch.Tensor], *, channels, lmax, num_interactions, correlation,
                 num_elements, cutoff, avg_num_neighbors, num_basis=8, cutoff_p=5):
        self.p = params
        self.C, self.L, self.T = channels, lmax, num_interactions
        self.corr, self.S = correlation, num_elements
        self.cutoff, self.avg = float(cutoff), float(avg_num_neighbors)
        self.num_basis, self.cutoff_p = num_basis, cutoff_p
        self.tps, self.scs = [], []
        for t in range(num_interactions):
            lin = 0 if t == 0 else lmax
            target = lmax if t < num_interactions - 1 else 0
            self.tps.append(TensorProductOracle(channels, lin, lmax, lmax, paths=_paths(lin, lmax, lmax),
                                                weight=params[f"interactions.{t}.tp.weight"]))
            self.scs.append(SymmetricContractionOracle(num_elements, channels, lmax, target, correlation, seed=0))

    def _sc_weights(self, t, target):
        """Weights and U buffers of product t's bridge-U contraction, read by name; the oracle
        contracts with the module's own U (``ops/symmetric_contraction.py:92-206``)."""
        w = {}
        for l in range(target + 1):
            pre = f"products.{t}.symmetric_contractions.symmetric_contractions.contractions.{l}"
            w[(l, self.corr)] = self.p[f"{pre}.weights_max"]
            for i, nu in enumerate(range(self.corr - 1, 0, -1)):
                w[(l, nu)] = self.p[f"{pre}.weights.{i}"]
            for nu in range(1, self.corr + 1):
                self.scs[t].u[(l, nu)] = self.p[f"{pre}.U_matrix_{nu}"].to(torch.float64)
        return w

    def atomic_energies(self, pos, species, src, dst, shifts, cell, batch):
        p, C, L = self.p, self.C, self.L
        vec = pos[dst] - pos[src] + torch.einsum("ni,nij->nj", shifts, cell[batch[src]])
        r = vec.norm(dim=1)
        n = vec / r.clamp(min=1e-8)[:, None]
        mask = (r <= self.cutoff).to(pos.dtype)
        y = basis.direction_harmonics_all(n, L)
        harm = {l: y[l].unsqueeze(1) for l in range(L + 1)}
        feats = bessel_features(r, self.cutoff, self.num_basis, self.cutoff_p)
        h = p["node_embedding.weight"].t()[species]
        energy = 0.0
        for t in range(self.T):
            pre = f"interactions.{t}"
            lin = 0 if t == 0 else L
            target = L if t < self.T - 1 else 0
            hb = _blocks(h, C, lin)
            x1 = {l: torch.einsum("oc,ncm->nom", p[f"{pre}.linear_up.weights.{l}"], hb[l]) for l in hb}
            g = feats
            for k in (0, 2, 4):
                g = _silu(g @ p[f"{pre}.fc.{k}.weight"].t())
            gates = g @ p[f"{pre}.fc.6.weight"].t()
            m = self.tps[t].graph_message_blocks(x1, harm, gates, src, dst, mask, nodes=pos.shape[0])
            msg = {l: torch.einsum("oc,ncm->nom", p[f"{pre}.message_linear.weights.{l}"], m[l]) / self.avg
                   for l in range(L + 1)}
            sc = torch.einsum("noc,nc->no", p[f"{pre}.self_connection.weight"][species], h[:, :C])
            out = self.scs[t].forward(_flat(msg), species, self._sc_weights(t, target))
            ob = _blocks(out, C, target)
            ob = {l: torch.einsum("oc,ncm->nom", p[f"products.{t}.linear.weights.{l}"], ob[l]) / math.sqrt(C)
                  for l in ob}
            ob[0] = ob[0] + sc[:, :, None]
            h = _flat(ob)
            if t < self.T - 1:
                e = h[:, :C] @ p[f"layer_readouts.{t}.weight"].t()
            else:
                e = _silu(h @ p["last_readout.0.weight"].t()) @ p["last_readout.2.weight"].t()
            energy = energy + e
        return energy.reshape(-1)

    def energy_and_forces(self, pos, species, src, dst, shifts, cell, batch, *, create_graph=False):
        pos = pos.detach().requires_grad_(True)
        atomic = self.atomic_energies(pos, species, src, dst, shifts, cell, batch)
        energy = atomic.new_zeros(cell.shape[0]).index_add(0, batch, atomic)
        forces = -torch.autograd.grad(energy.sum(), pos, create_graph=create_graph)[0]
        return energy, forces, atomic
