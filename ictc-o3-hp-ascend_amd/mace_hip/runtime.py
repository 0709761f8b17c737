"""Model construction, energy + force evaluation and one force-loss training step.

Mirrors reference ``mace_ictc/hp/runtime.py``: ``create_model`` (:7-81; channels, lmax,
num_interactions, correlation 1-3, atomic_numbers, cutoff, avg_num_neighbors) and
``energy_and_forces`` (:84-119; forces = -dE/dpos through autograd, ``create_graph``
when training, detached results otherwise, zero-edge graphs keep the coordinate
dependency).  ``check_model`` / ``configure_model`` (:123-145) report and select the HIP
operators.  ``training_step`` is the pattern of ``examples/model.py:35-41``: energy and
forces with ``training=True``, loss = mean((E/N)^2) + mean(F^2), backward, AdamW step.

``CapturedEnergyAndForces`` / ``CapturedTrainingStep`` record one fixed-shape step into a
HIP graph and replay it (the reference runs eager only: its graph capture is not qualified,
``mace_ictc/ascend/runtime.py:28-29``).  Every operator of the step launches on the current
stream, allocates through torch and performs no host synchronisation once its per-graph
checks are cached, which the warmup calls do.
"""
from __future__ import annotations

import torch

from ictc_o3.backends.hip.graph_message import pin_graphs
from ictc_o3.backends.hip.runtime import require_gpu_fp32, strict_fp32

from .geometry import one_hot_rows
from .linear import mm
from .model import MaceICTC


def create_model(*, channels=64, lmax=3, edge_lmax=None, num_interactions=2, correlation=3,
                 atomic_numbers=(1, 6, 8), cutoff=5.0, avg_num_neighbors=50.0, device="cuda",
                 dtype=torch.float32, seed=None) -> MaceICTC:
    if dtype != torch.float32:
        raise ValueError("the HIP operators compute in float32")
    if not isinstance(num_interactions, int) or isinstance(num_interactions, bool) or num_interactions < 1:
        raise ValueError("num_interactions must be a positive integer")
    if correlation not in (1, 2, 3):
        raise ValueError("correlation must be 1, 2 or 3")
    if not isinstance(channels, int) or channels < 1:
        raise ValueError("channels must be a positive integer")
    if not isinstance(lmax, int) or not 0 <= lmax <= 3:
        raise ValueError("lmax must be an integer in [0, 3]")
    if edge_lmax is not None and edge_lmax != lmax:
        raise ValueError("edge_lmax must equal lmax for the compiled kernels")
    if seed is not None:
        torch.manual_seed(int(seed))
    model = MaceICTC(channels=channels, lmax=lmax, num_interactions=num_interactions, correlation=correlation,
                     atomic_numbers=atomic_numbers, cutoff=cutoff, avg_num_neighbors=avg_num_neighbors)
    return model.to(device=device, dtype=dtype)


_ONE_BLOCK_SUM = 65536   # atoms of one structure summed by a plain reduction (see energy_and_forces)


def energy_and_forces(model, positions, atomic_numbers, batch, edge_src, edge_dst, edge_shifts, cell, *,
                      training=False, species=None):
    """-> {"energy": [B], "forces": [N,3], "atomic_energy": [N]}; cell [B,3,3], shifts in lattice
    coordinates."""
    if torch.is_inference_mode_enabled():
        raise ValueError("forces require autograd; use no_grad instead of inference_mode")
    if positions.ndim != 2 or positions.shape[1] != 3 or cell.ndim != 3 or cell.shape[1:] != (3, 3):
        raise ValueError("expected positions [N,3] and cell [B,3,3]")
    n = positions.shape[0]
    if atomic_numbers.shape != (n,) or batch.shape != (n,):
        raise ValueError("atomic numbers and batch must have shape [N]")
    require_gpu_fp32(positions)
    _validate_batch(batch, cell.shape[0])
    with torch.enable_grad():
        pos = positions if positions.requires_grad else positions.detach().requires_grad_(True)
        atomic = model(pos, atomic_numbers, batch, edge_src, edge_dst, edge_shifts, cell, species=species)
        if cell.shape[0] == 1 and n <= _ONE_BLOCK_SUM:
            # one structure: its energy is the sum of every atomic energy, one reduction kernel
            # whose adjoint is a broadcast (at this size torch reduces in one workgroup, with no
            # cross-block staging to clear: the step stays capturable into a HIP graph)
            energy = atomic.sum(0, keepdim=True)
            total = energy.reshape(())
        else:
            # per-structure sums as one_hot(batch)^T @ atomic: a fixed summation order
            energy = mm(one_hot_rows(batch, cell.shape[0]).t(), atomic.unsqueeze(1)).squeeze(1)
            total = energy.sum()
        if edge_src.numel() == 0:
            # keep the coordinate dependency of a graph without edges (a 3-element sum: no
            # multi-block reduction, so the step stays capturable into a HIP graph)
            total = total + pos[:1].sum() * 0.0
        force = -torch.autograd.grad(total, pos, create_graph=training, retain_graph=training)[0]
    result = {"energy": energy, "forces": force, "atomic_energy": atomic}
    return result if training else {k: v.detach() for k, v in result.items()}


def _validate_batch(batch: torch.Tensor, structures: int) -> None:
    """Per-structure energies are one_hot(batch)^T @ atomic energies, which would silently drop an
    atom whose batch index is outside [0, structures) (an index_add would raise): check the range
    once per batch tensor (one host read), cached on its identity, address and version."""
    key = (id(batch), batch.data_ptr(), batch._version, int(structures))
    if _validate_batch.last == key:
        return
    if batch.numel() and (int(batch.min()) < 0 or int(batch.max()) >= structures):
        raise ValueError(f"batch indices must lie in [0, {structures}) (one per cell)")
    _validate_batch.last = key


_validate_batch.last = None


def force_loss(prediction, atoms: int):
    return (prediction["energy"] / atoms).square().mean() + prediction["forces"].square().mean()


def backward_to_parameters(loss: torch.Tensor, model, positions: torch.Tensor = None) -> None:
    """loss.backward() restricted to the model's trainable parameters (and to ``positions`` when
    the caller passes positions that require a gradient, so their ``.grad`` fills as with
    loss.backward()).  For positions without a gradient, energy_and_forces differentiates through
    a private copy whose loss gradient is never read; leaving it out of the backward's inputs lets
    every adjoint that only leads there (the harmonics and edge-geometry terms of the message VJPs
    and of their double backward, the radial MLP's input adjoints) be skipped.  The parameters'
    gradients are the same as those of loss.backward()."""
    inputs = [p for p in model.parameters() if p.requires_grad]
    if positions is not None and positions.requires_grad:
        inputs.append(positions)
    loss.backward(inputs=inputs)


def training_step(model, optimizer, graph: dict, *, species=None):
    """One force-loss step; returns the loss (a device tensor, not synchronised)."""
    prediction = energy_and_forces(model, **graph, training=True, species=species)
    loss = force_loss(prediction, graph["positions"].shape[0])
    backward_to_parameters(loss, model, graph["positions"])
    optimizer.step()
    optimizer.zero_grad(set_to_none=True)
    return loss.detach()


def check_model(model, *, training=False, capture=False) -> dict:
    """Coverage of the HIP operators for this model, without modifying it (reference
    ``hp/runtime.py:123-130`` and its backend check ``mace_ictc/ascend/runtime.py:10-39``):
    {"supported": bool, "backend": "hip", "reasons": [...]}.  Training (force-loss second
    derivatives) and HIP-graph capture (``CapturedEnergyAndForces``, ``CapturedTrainingStep``)
    are both covered, so ``training`` and ``capture`` add no reasons."""
    if not isinstance(model, MaceICTC):
        return {"supported": False, "backend": "hip", "reasons": ["Expected the MACE-ICTC model (mace_hip.MaceICTC)"]}
    reasons = []
    if any(p.device.type != "cuda" or p.dtype != torch.float32 for p in model.parameters()):
        reasons.append("All model parameters must already be ROCm GPU FP32")
    try:
        from ictc_o3 import _lib
        _lib.lib()
    except (OSError, RuntimeError) as exc:
        reasons.append(f"The HIP operator library is unavailable: {exc}")
    if not 0 <= model.lmax <= 3:
        reasons.append("The message tangent kernels and the symmetric contraction are compiled for lmax <= 3")
    for product in model.products:
        if product.symmetric_contractions.correlation not in (1, 2, 3):
            reasons.append("The symmetric contraction supports correlation 1, 2 and 3")
    for interaction in model.interactions:
        if interaction.tp.internal_compute_dtype != torch.float32:
            reasons.append("Tensor-product internal compute dtype must be FP32")
    return {"supported": not reasons, "backend": "hip", "reasons": reasons}


def configure_model(model, *, training=False, policy="auto", layout="packed", capture=False,
                    message_chunk_edges=None, electrostatics_backend="auto") -> dict:
    """Select the HIP operators for a model (reference ``hp/runtime.py:133-145`` and
    ``mace_ictc/ascend/runtime.py:42-89``; same arguments).  ``message_chunk_edges`` switches
    radial streaming on (receiver ranges of at most that many edges; the reference's
    ``edge_chunk_size``) or off (None).  There is no reference backend to fall back to (no CPU
    path in this build), so ``policy="reference"`` and an unsupported model raise."""
    if layout not in ("packed", "fused_pack"):
        raise ValueError("layout must be packed or fused_pack")
    if policy not in ("auto", "generated", "reference"):
        raise ValueError("policy must be auto, generated or reference")
    if message_chunk_edges is not None and (not isinstance(message_chunk_edges, int)
                                            or isinstance(message_chunk_edges, bool) or message_chunk_edges < 1):
        raise ValueError("edge_chunk_size must be a positive integer or None for automatic sizing")
    if electrostatics_backend not in ("auto", "none"):
        raise ValueError("electrostatics is not part of this model; electrostatics_backend must be auto or none")
    if policy == "reference":
        raise ValueError("this build has no reference (CPU) backend; use policy='auto' or 'generated'")
    coverage = check_model(model, training=training, capture=capture)
    if not coverage["supported"]:
        raise ValueError("HIP HP unavailable: " + "; ".join(coverage["reasons"]))
    strict_fp32()
    model.set_message_streaming(message_chunk_edges)
    return {"requested": policy, "selected": "generated", "backend": "hip", "reasons": [],
            "electrostatics": None, "arithmetic": "strict FP32; TF32 and autocast disabled",
            "edge_chunk_size": message_chunk_edges, "kernel_backend": "hip",
            "tensor_product_adjoint": "analytic",
            "counts": {"interactions": len(model.interactions)}}


def _warm_up(fn, calls: int, device) -> None:
    """Run fn on a side stream (default priority) before capture, as graph capture requires."""
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for _ in range(calls):
            fn()
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize(device)


class CapturedEnergyAndForces:
    """energy_and_forces of one fixed structure graph, captured once and replayed.

    Atomic numbers, batch, edges and shifts are fixed at capture; each call copies new
    positions (and optionally a new cell) into the captured input buffers and replays.
    The returned tensors are the graph's own output buffers, overwritten by the next call
    (clone them to keep them).  A different edge count needs a new capture."""

    def __init__(self, model, positions, atomic_numbers, batch, edge_src, edge_dst, edge_shifts, cell, *,
                 species=None, warmup: int = 3):
        self.model = model
        self._pos = positions.detach().clone()
        self._cell = cell.detach().clone()
        self._fixed = dict(atomic_numbers=atomic_numbers, batch=batch, edge_src=edge_src, edge_dst=edge_dst,
                           edge_shifts=edge_shifts)
        self._species = model.species_index(atomic_numbers) if species is None else species
        dev = positions.device
        _warm_up(self._step, warmup, dev)
        self.graph = torch.cuda.CUDAGraph()
        # the capture records the addresses of the cached message-graph CSR tensors: hold them
        with pin_graphs() as self._message_graphs, torch.cuda.graph(self.graph):
            self._out = self._step()

    def _step(self):
        return energy_and_forces(self.model, positions=self._pos, cell=self._cell, species=self._species,
                                 **self._fixed)

    def __call__(self, positions: torch.Tensor, cell=None) -> dict:
        if positions.shape != self._pos.shape:
            raise ValueError("positions must keep the captured shape")
        self._pos.copy_(positions)
        if cell is not None:
            self._cell.copy_(cell)
        self.graph.replay()
        return self._out


class CapturedTrainingStep:
    """One force-loss training step (energy + forces with create_graph, loss backward, optimizer
    step) captured once and replayed on new positions.  The optimizer must keep its state on
    the device (``torch.optim.AdamW(..., capturable=True)``, which may also be ``fused=True``: one
    update kernel for all parameters, 0.3 ms less per cfg-4 step); gradients are released before
    capture so that backward writes them into the graph's own buffers on every replay."""

    def __init__(self, model, optimizer, graph: dict, *, species=None, warmup: int = 3):
        if not all(group.get("capturable", False) for group in optimizer.param_groups):
            raise ValueError("the optimizer must be created with capturable=True")
        self.model, self.optimizer = model, optimizer
        self._graph = {k: (v.detach().clone() if k in ("positions", "cell") else v) for k, v in graph.items()}
        self._species = model.species_index(graph["atomic_numbers"]) if species is None else species
        dev = self._graph["positions"].device
        _warm_up(lambda: training_step(model, optimizer, self._graph, species=self._species), warmup, dev)
        optimizer.zero_grad(set_to_none=True)
        self.graph = torch.cuda.CUDAGraph()
        with pin_graphs() as self._message_graphs, torch.cuda.graph(self.graph):
            prediction = energy_and_forces(model, **self._graph, training=True, species=self._species)
            self._loss = force_loss(prediction, self._graph["positions"].shape[0])
            backward_to_parameters(self._loss, model, self._graph["positions"])
            optimizer.step()

    def __call__(self, positions: torch.Tensor, cell=None) -> torch.Tensor:
        """Replays the step on these positions; returns the loss buffer (device, not synchronised)."""
        if positions.shape != self._graph["positions"].shape:
            raise ValueError("positions must keep the captured shape")
        self._graph["positions"].copy_(positions)
        if cell is not None:
            self._graph["cell"].copy_(cell)
        self.graph.replay()
        return self._loss
