"""MACE-style energy + force model on the HIP operators against the float64 oracle
restatement (oracle/mace.py) on the same parameters and graph.

* energies (rel 1e-5) and forces (rel 1e-4) on a small periodic structure, at C = 32 and at
  cfg 4's C = 128;
* force-loss training gradients of every trainable parameter (rel 1e-4): the loss
  depends on the forces, so this exercises the mixed second derivatives of the graph
  message, the symmetric contraction and the direction harmonics end to end;
* at the cfg-4 size (C=128, lmax 3, 2,048 atoms, ~107k edges): invariance of the
  energy and covariance of the forces under a rigid rotation of the cell, and
  one AdamW training step.
"""
import math

import pytest
import torch

from conftest import RTOL_FORCE, assert_rel
from oracle import ictc_basis as B
from oracle.mace import MaceOracle

pytestmark = pytest.mark.gpu

ZS = (1, 6, 8)


def _setup(gpu, *, channels=32, atoms=48, density=0.05, cutoff=4.0, seed=3):
    from mace_hip import create_model, radius_graph, sequential_insertion
    model = create_model(channels=channels, lmax=3, num_interactions=2, correlation=3, atomic_numbers=ZS,
                         cutoff=cutoff, avg_num_neighbors=12.0, device=gpu, seed=seed)
    with torch.no_grad():                       # move off the identity init so every weight matters
        g = torch.Generator(device=gpu).manual_seed(seed + 1)
        for name, p in model.named_parameters():
            if p.requires_grad and ("linear_up" in name or "self_connection" in name):
                p.add_(torch.randn(p.shape, device=gpu, generator=g) * 0.1)
    st = sequential_insertion(atoms, density, min_separation=1.2, num_species=len(ZS), seed=seed)
    src, dst, shifts = radius_graph(st.positions, st.cell, cutoff)
    z = torch.tensor(ZS)[st.species]
    graph = dict(positions=st.positions.to(gpu), atomic_numbers=z.to(gpu),
                 batch=torch.zeros(atoms, dtype=torch.int64, device=gpu), edge_src=src.to(gpu),
                 edge_dst=dst.to(gpu), edge_shifts=shifts.to(gpu), cell=st.cell[None].to(gpu))
    state = [*model.named_parameters(), *model.named_buffers()]      # buffers: the contractions' U
    oracle = MaceOracle({k: v.detach().double().cpu() for k, v in state},
                        channels=channels, lmax=3, num_interactions=2, correlation=3, num_elements=len(ZS),
                        cutoff=cutoff, avg_num_neighbors=12.0)
    cpu = dict(pos=st.positions.double(), species=st.species, src=src, dst=dst, shifts=shifts.double(),
               cell=st.cell[None].double(), batch=torch.zeros(atoms, dtype=torch.int64))
    return model, graph, oracle, cpu


@pytest.mark.parametrize("channels", [32, 128])
def test_energy_and_forces_match_oracle(gpu, channels):
    from mace_hip import energy_and_forces
    model, graph, oracle, cpu = _setup(gpu, channels=channels)
    assert graph["edge_src"].numel() > 300
    got = energy_and_forces(model, **graph)
    e, f, atomic = oracle.energy_and_forces(**cpu)
    assert_rel(got["atomic_energy"], atomic, what="atomic energies")
    assert_rel(got["energy"], e, what="energy")
    assert_rel(got["forces"], f, rtol=RTOL_FORCE, what="forces")


@pytest.mark.parametrize("channels", [32, 128])
@pytest.mark.parametrize("to_parameters", [False, True], ids=["backward", "backward_to_parameters"])
def test_force_loss_gradients_match_oracle(gpu, channels, to_parameters):
    """Both the plain loss.backward() and the parameter-restricted backward of training_step
    (which skips every adjoint that only leads to the positions) against the oracle."""
    from mace_hip import energy_and_forces, force_loss
    from mace_hip.runtime import backward_to_parameters
    model, graph, oracle, cpu = _setup(gpu, channels=channels, seed=5)
    atoms = graph["positions"].shape[0]
    pred = energy_and_forces(model, **graph, training=True)
    loss = force_loss(pred, atoms)
    if to_parameters:
        backward_to_parameters(loss, model)
    else:
        loss.backward()
    names = [n for n, p in model.named_parameters() if p.requires_grad]
    for n in names:
        oracle.p[n].requires_grad_(True)
    e, f, _ = oracle.energy_and_forces(**cpu, create_graph=True)
    eloss = (e / atoms).square().mean() + f.square().mean()
    grads = torch.autograd.grad(eloss, [oracle.p[n] for n in names])
    assert_rel(loss.detach(), eloss.detach(), rtol=RTOL_FORCE, what="force loss")
    params = dict(model.named_parameters())
    for n, g in zip(names, grads):
        assert_rel(params[n].grad, g, rtol=RTOL_FORCE, what=f"d loss / d {n}")


def test_backward_to_parameters_equals_full_backward(gpu):
    """The parameter-restricted backward gives the parameters the gradients of loss.backward()."""
    from mace_hip import energy_and_forces, force_loss
    from mace_hip.runtime import backward_to_parameters
    grads = []
    for restricted in (False, True):
        model, graph, _, _ = _setup(gpu, channels=64, seed=7)
        loss = force_loss(energy_and_forces(model, **graph, training=True), graph["positions"].shape[0])
        if restricted:
            backward_to_parameters(loss, model)
        else:
            loss.backward()
        grads.append({n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None})
    assert grads[0].keys() == grads[1].keys()
    for n in grads[0]:
        assert_rel(grads[1][n], grads[0][n], rtol=1e-6, what=f"d loss / d {n}")


def _rotation(om):
    k = torch.zeros(3, 3, dtype=torch.float64)
    k[0, 1], k[0, 2], k[1, 2] = -om[2], om[1], -om[0]
    k = k - k.T
    return torch.linalg.matrix_exp(k)


def test_full_size_rotation_and_training_step(gpu):
    """cfg 4: C128/lmax 3, 2 interactions, correlation 3, 10 species, r_c 5 A, 2,048 atoms."""
    from mace_hip import create_model, energy_and_forces, radius_graph, sequential_insertion, training_step
    zs = tuple(range(1, 11))
    model = create_model(channels=128, lmax=3, num_interactions=2, correlation=3, atomic_numbers=zs, cutoff=5.0,
                         device=gpu, seed=0)
    st = sequential_insertion(2048, 0.1, min_separation=1.5, num_species=10, seed=4)
    src, dst, shifts = radius_graph(st.positions.to(gpu), st.cell.to(gpu), 5.0)
    assert 95_000 < src.numel() < 120_000
    z = torch.tensor(zs, device=gpu)[st.species.to(gpu)]
    batch = torch.zeros(2048, dtype=torch.int64, device=gpu)
    base = dict(atomic_numbers=z, batch=batch, edge_src=src, edge_dst=dst, edge_shifts=shifts)
    out = energy_and_forces(model, positions=st.positions.to(gpu), cell=st.cell[None].to(gpu), **base)
    rot = _rotation(torch.tensor([0.3, -1.1, 0.7])).float().to(gpu)
    # rotate positions and lattice vectors together and translate: same graph, same shifts
    pos_r = st.positions.to(gpu) @ rot.T + torch.tensor([0.4, -2.0, 1.3], device=gpu)
    out_r = energy_and_forces(model, positions=pos_r, cell=(st.cell.to(gpu) @ rot.T)[None], **base)
    assert_rel(out_r["energy"], out["energy"], rtol=2e-5, what="energy invariance")
    assert_rel(out_r["atomic_energy"], out["atomic_energy"], rtol=2e-5, what="atomic energy invariance")
    assert_rel(out_r["forces"], out["forces"] @ rot.T, rtol=RTOL_FORCE, what="force covariance")
    assert math.isfinite(float(out["energy"]))
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
    before = {n: p.detach().clone() for n, p in model.named_parameters() if p.requires_grad}
    loss = training_step(model, opt, dict(positions=st.positions.to(gpu), cell=st.cell[None].to(gpu), **base))
    assert math.isfinite(float(loss))
    moved = [n for n, p in model.named_parameters() if p.requires_grad and not torch.equal(p, before[n])]
    assert len(moved) == len(before)


def test_configure_model_selects_hip_and_streaming(gpu):
    """configure_model (reference hp/runtime.py:133-145) on a GPU model: supported, the message
    chunk size switches radial streaming on and off, and the configured model still matches the
    oracle; positions that require a gradient get it from the restricted training backward."""
    from mace_hip import check_model, configure_model, energy_and_forces, force_loss
    from mace_hip.runtime import backward_to_parameters
    model, graph, oracle, cpu = _setup(gpu)
    assert check_model(model, training=True, capture=True) == {"supported": True, "backend": "hip", "reasons": []}
    info = configure_model(model, training=True, message_chunk_edges=64)
    assert info["selected"] == "generated" and info["edge_chunk_size"] == 64
    assert all(i.edge_chunk_size == 64 for i in model.interactions)
    got = energy_and_forces(model, **graph)
    e, f, _ = oracle.energy_and_forces(**cpu)
    assert_rel(got["energy"], e, what="streamed energy")
    assert_rel(got["forces"], f, rtol=RTOL_FORCE, what="streamed forces")
    configure_model(model)
    assert all(i.edge_chunk_size is None for i in model.interactions)
    pos = graph["positions"].clone().requires_grad_()
    pred = energy_and_forces(model, **{**graph, "positions": pos}, training=True)
    backward_to_parameters(force_loss(pred, pos.shape[0]), model, pos)
    assert pos.grad is not None and torch.isfinite(pos.grad).all()


def test_gate_gradient_handover(gpu, monkeypatch):
    """Force-loss backward: the force path's gate gradient (the message VJP's double backward) is
    handed to the energy path's message VJP, whose edge kernel adds its own gate gradient into it,
    instead of the engine adding two [E, P*C] tensors.  The parameter gradients are bit-identical
    to those of the engine's sum (a float add is commutative), and the hand-over is taken."""
    import ictc_o3.backends.hip.graph_message as GM
    from mace_hip import energy_and_forces, force_loss
    from mace_hip.runtime import backward_to_parameters
    accumulated = []
    raw = GM._backward_raw

    def spy(*args, dg_into=None, **kw):
        accumulated.append(dg_into is not None)
        return raw(*args, dg_into=dg_into, **kw)

    monkeypatch.setattr(GM, "_backward_raw", spy)
    grads = []
    for handover in (False, True):
        monkeypatch.setattr(GM, "GATE_GRAD_HANDOVER", handover)
        accumulated.clear()
        model, graph, _, _ = _setup(gpu, channels=64, seed=9)
        loss = force_loss(energy_and_forces(model, **graph, training=True), graph["positions"].shape[0])
        backward_to_parameters(loss, model, graph["positions"])
        grads.append({n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None})
        print(f"handover={handover}: accumulate-mode edge kernels {sum(accumulated)}", flush=True)
        assert sum(accumulated) == (len(model.interactions) if handover else 0)
    assert grads[0].keys() == grads[1].keys()
    for n in grads[0]:
        assert torch.equal(grads[1][n], grads[0][n]), n
