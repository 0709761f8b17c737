"""HIP-graph capture of the MACE step (mace_hip.runtime.CapturedEnergyAndForces /
CapturedTrainingStep) against eager execution of the same step.

Each captured graph is replayed several times on new positions, with the program's own
eager work and device synchronisations between replays, and every replay is compared with
the eager result on the same inputs (the graph must not keep stale values from its capture
or an earlier replay).  The eager step itself is pinned to the float64 oracle in
test_mace_gpu.py.
"""
import pytest
import torch

from conftest import assert_rel
from test_mace_gpu import _setup

pytestmark = pytest.mark.gpu


def _positions(graph, step, gpu):
    g = torch.Generator(device=gpu).manual_seed(100 + step)
    return graph["positions"] + 0.05 * torch.randn(graph["positions"].shape, device=gpu, generator=g)


def test_captured_inference_replays_match_eager(gpu):
    from mace_hip import CapturedEnergyAndForces, energy_and_forces
    model, graph, _, _ = _setup(gpu, atoms=96)
    model.eval().requires_grad_(False)
    captured = CapturedEnergyAndForces(model, **graph)
    fixed = {k: v for k, v in graph.items() if k != "positions"}
    for step in range(4):
        pos = _positions(graph, step, gpu)
        eager = energy_and_forces(model, positions=pos, **fixed)
        torch.cuda.synchronize(gpu)
        got = captured(pos)
        torch.cuda.synchronize(gpu)
        for key in ("atomic_energy", "energy", "forces"):
            assert_rel(got[key], eager[key], rtol=1e-5, what=f"replay {step} {key}")


def test_captured_training_step_replays_match_eager(gpu):
    from mace_hip import CapturedTrainingStep, training_step
    model_a, graph, _, _ = _setup(gpu, atoms=96)
    model_b, _, _, _ = _setup(gpu, atoms=96)
    for (na, pa), (nb, pb) in zip(model_a.named_parameters(), model_b.named_parameters()):
        assert na == nb and torch.equal(pa, pb)
    opt_a = torch.optim.AdamW(model_a.parameters(), lr=1e-3, capturable=True)
    opt_b = torch.optim.AdamW(model_b.parameters(), lr=1e-3, capturable=True)
    # warm-up steps inside the capture helper advance model_b; advance model_a identically
    warm = dict(graph)
    for _ in range(3):
        training_step(model_a, opt_a, warm)
    captured = CapturedTrainingStep(model_b, opt_b, graph, warmup=3)
    for step in range(3):
        pos = _positions(graph, step, gpu)
        loss_a = training_step(model_a, opt_a, dict(graph, positions=pos))
        torch.cuda.synchronize(gpu)
        loss_b = captured(pos)
        torch.cuda.synchronize(gpu)
        assert_rel(loss_b, loss_a, rtol=1e-4, what=f"replay {step} loss")
        for (name, pa), (_, pb) in zip(model_a.named_parameters(), model_b.named_parameters()):
            if pa.requires_grad:
                assert_rel(pb, pa, rtol=1e-4, what=f"replay {step} parameter {name}")
