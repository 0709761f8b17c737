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


@pytest.mark.parametrize("fused", [False, True])
def test_captured_training_step_replays_match_eager(gpu, fused):
    from mace_hip import CapturedTrainingStep, training_step
    model_a, graph, _, _ = _setup(gpu, atoms=96)
    model_b, _, _, _ = _setup(gpu, atoms=96)
    for (na, pa), (nb, pb) in zip(model_a.named_parameters(), model_b.named_parameters()):
        assert na == nb and torch.equal(pa, pb)
    opt_a = torch.optim.AdamW(model_a.parameters(), lr=1e-3, capturable=True, fused=fused)
    opt_b = torch.optim.AdamW(model_b.parameters(), lr=1e-3, capturable=True, fused=fused)
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


def test_captured_replay_after_message_graph_cache_eviction(gpu):
    """The captured step keeps its message-graph CSR tensors alive after the CSR cache has been
    cycled and cleared and their memory would otherwise have been reused."""
    import gc
    from ictc_o3.backends.hip import graph_message as gm
    from mace_hip import CapturedEnergyAndForces, energy_and_forces
    model, graph, _, _ = _setup(gpu, atoms=96)
    model.eval().requires_grad_(False)
    captured = CapturedEnergyAndForces(model, **graph)
    n = graph["positions"].shape[0]
    for seed in range(12):
        g = torch.Generator(device=gpu).manual_seed(seed)
        gm.message_graph(torch.randint(0, n, (4000,), device=gpu, generator=g),
                         torch.randint(0, n, (4000,), device=gpu, generator=g), n, n)
    gm._GRAPH_CACHE.clear()
    gc.collect()
    junk = [torch.full((1 << 16,), -1, dtype=torch.int64, device=gpu) for _ in range(64)]
    fixed = {k: v for k, v in graph.items() if k != "positions"}
    pos = _positions(graph, 7, gpu)
    eager = energy_and_forces(model, positions=pos, **fixed)
    torch.cuda.synchronize(gpu)
    got = captured(pos)
    torch.cuda.synchronize(gpu)
    del junk
    for key in ("atomic_energy", "energy", "forces"):
        assert_rel(got[key], eager[key], rtol=1e-5, what=f"replay after eviction {key}")
