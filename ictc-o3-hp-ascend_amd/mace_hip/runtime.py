"""Model construction, energy + force evaluation and one force-loss training step.

Mirrors reference ``mace_ictc/hp/runtime.py``: ``create_model`` (:7-81; channels, lmax,
num_interactions, correlation 1-3, atomic_numbers, cutoff, avg_num_neighbors) and
``energy_and_forces`` (:84-119; forces = -dE/dpos through autograd, ``create_graph``
when training, detached results otherwise, zero-edge graphs keep the coordinate
dependency).  ``training_step`` is the pattern of ``examples/model.py:35-41``: energy and
forces with ``training=True``, loss = mean((E/N)^2) + mean(F^2), backward, AdamW step.
"""
from __future__ import annotations

import torch

from ictc_o3.backends.hip.runtime import require_gpu_fp32

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
    with torch.enable_grad():
        pos = positions if positions.requires_grad else positions.detach().requires_grad_(True)
        atomic = model(pos, atomic_numbers, batch, edge_src, edge_dst, edge_shifts, cell, species=species)
        energy = atomic.new_zeros(cell.shape[0]).index_add(0, batch, atomic)
        force = -torch.autograd.grad(energy.sum() + pos.sum() * 0.0, pos, create_graph=training,
                                     retain_graph=training)[0]
    result = {"energy": energy, "forces": force, "atomic_energy": atomic}
    return result if training else {k: v.detach() for k, v in result.items()}


def force_loss(prediction, atoms: int):
    return (prediction["energy"] / atoms).square().mean() + prediction["forces"].square().mean()


def training_step(model, optimizer, graph: dict, *, species=None):
    """One force-loss step; returns the loss (a device tensor, not synchronised)."""
    prediction = energy_and_forces(model, **graph, training=True, species=species)
    loss = force_loss(prediction, graph["positions"].shape[0])
    loss.backward()
    optimizer.step()
    optimizer.zero_grad(set_to_none=True)
    return loss.detach()
