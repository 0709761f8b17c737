"""Radial-streaming message (reference ``capacity_message.py:109-179``,
``capacity_adjoint.py:5-148``): the gates are the radial MLP's last Linear, produced one receiver
range at a time inside the message (``ictc_o3/backends/hip/radial_message.py``).

* the hook ``radial_graph_message(owner, features, harmonics, radial, edge_features, src, dst,
  mask, edge_chunk_size=)`` against the float64 oracle (gather -> TP -> mask -> index_add with the
  gates of the same radial MLP): values, first derivatives (features, harmonics, edge features,
  every radial parameter) and second derivatives, with ranges smaller than a receiver's row,
  unsorted edges, a mask and a live (non-unit) owner weight;
* its None returns (not handled): empty graph, a radial module that does not end in a Linear,
  a mask that needs a gradient;
* the packed form at C=128 / lmax 3 (bond rows from the harmonics) equals the whole-gate message;
* the MACE model with streaming on: energies, forces and force-loss gradients equal the whole-
  gate model's, and at the cfg-4 size the inference peak memory drops by at least the gate tensor.
"""
import math

import pytest
import torch

from conftest import RTOL_FORCE, assert_rel
from oracle import ictc_basis as B
from oracle.tensor_product import TensorProductOracle

pytestmark = pytest.mark.gpu


def _owner(gpu, channels, lmax, weight):
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    tp = EdgeWeightedPathPreservingTensorProduct(channels, lmax, internal_compute_dtype=torch.float32).to(gpu)
    with torch.no_grad():
        tp.weight.copy_(weight.reshape(tp.weight.shape))
    return tp


def _radial(width, hidden, basis, gen):
    torch.manual_seed(int(torch.randint(0, 1 << 30, (1,), generator=gen)))
    return torch.nn.Sequential(torch.nn.Linear(basis, hidden), torch.nn.SiLU(), torch.nn.Linear(hidden, width))


def _case(gpu, seed, c=16, lmax=2, nodes=25, edges=240, sort=False):
    gen = torch.Generator().manual_seed(seed)
    ref = TensorProductOracle(c, lmax, lmax, lmax)
    weight = 1.0 + 0.2 * torch.randn(ref.num_paths, c, generator=gen, dtype=torch.float64)
    ref.weight = weight
    owner = _owner(gpu, c, lmax, weight.float())
    radial64 = _radial(ref.num_paths * c, 12, 6, gen).double()
    radial = _radial(ref.num_paths * c, 12, 6, gen).to(gpu)
    with torch.no_grad():
        for a, b in zip(radial.parameters(), radial64.parameters()):
            a.copy_(b.float())
    x = {l: torch.randn(nodes, c, 2 * l + 1, generator=gen, dtype=torch.float64) for l in range(lmax + 1)}
    n = torch.nn.functional.normalize(torch.randn(edges, 3, generator=gen, dtype=torch.float64), dim=-1)
    yp = B.direction_harmonics_packed(n, lmax)
    y = {l: yp[:, l * l:(l + 1) ** 2].unsqueeze(1) for l in range(lmax + 1)}
    feats = torch.randn(edges, 6, generator=gen, dtype=torch.float64)
    src = torch.randint(0, nodes, (edges,), generator=gen)
    dst = torch.randint(0, nodes - 1, (edges,), generator=gen)
    dst[:40] = 3                                        # one receiver with a long row
    if sort:
        order = torch.argsort(dst * nodes + src, stable=True)
        src, dst, feats = src[order], dst[order], feats[order]
        y = {l: v[order] for l, v in y.items()}
    mask = (torch.rand(edges, generator=gen) > 0.15).double()
    return ref, owner, radial64, radial, x, y, feats, src, dst, mask


def _dev(d, gpu, grad=False):
    return {l: v.float().to(gpu).requires_grad_(grad) for l, v in d.items()}


@pytest.mark.parametrize("sort,chunk", [(False, 17), (True, 64), (True, 100000)])
def test_hook_values_and_first_derivatives(gpu, sort, chunk):
    from ictc_o3.backends.hip.radial_message import radial_graph_message
    ref, owner, radial64, radial, x, y, feats, src, dst, mask = _case(gpu, 3 + chunk, sort=sort)
    xs, ys = _dev(x, gpu, True), _dev(y, gpu, True)
    fs = feats.float().to(gpu).requires_grad_()
    got = radial_graph_message(owner, xs, ys, radial, fs, src.to(gpu), dst.to(gpu), mask.float().to(gpu),
                               edge_chunk_size=chunk)
    xc = {l: v.clone().requires_grad_() for l, v in x.items()}
    yc = {l: v.clone().requires_grad_() for l, v in y.items()}
    fc = feats.clone().requires_grad_()
    expect = ref.graph_message_blocks(xc, yc, radial64(fc), src, dst, mask)
    for l in expect:
        assert_rel(got[l], expect[l], what=f"radial message l={l}")
    gen = torch.Generator().manual_seed(5)
    cots = {l: torch.randn(v.shape, generator=gen, dtype=torch.float64) for l, v in expect.items()}
    leaves = [*xs.values(), *ys.values(), fs, *radial.parameters()]
    eleaves = [*xc.values(), *yc.values(), fc, *radial64.parameters()]
    grads = torch.autograd.grad([got[l] for l in cots], leaves, [cots[l].float().to(gpu) for l in cots])
    egrads = torch.autograd.grad([expect[l] for l in cots], eleaves, [cots[l] for l in cots])
    for i, (a, b) in enumerate(zip(grads, egrads)):
        assert_rel(a, b, what=f"radial message first derivative {i}")


def test_hook_second_derivatives(gpu):
    """d/d(features, harmonics, edge features, radial parameters) of <a, d<cot, out>/d features>
    + <b, d<cot, out>/d edge features> (the force-training pattern)."""
    from ictc_o3.backends.hip.radial_message import radial_graph_message
    ref, owner, radial64, radial, x, y, feats, src, dst, mask = _case(gpu, 21, sort=True)
    gen = torch.Generator().manual_seed(6)

    def run(fn, xs, ys, fs, params, to):
        out = fn(xs, ys, fs)
        cots = {l: to(torch.randn(v.shape, generator=torch.Generator().manual_seed(7 + l), dtype=torch.float64))
                for l, v in out.items()}
        leaves = [*xs.values(), fs]
        first = torch.autograd.grad([out[l] for l in cots], leaves, [cots[l] for l in cots], create_graph=True)
        a = [to(torch.randn(t.shape, generator=torch.Generator().manual_seed(30 + i), dtype=torch.float64))
             for i, t in enumerate(first)]
        loss = sum((f * w).sum() for f, w in zip(first, a))
        return torch.autograd.grad(loss, [*xs.values(), *ys.values(), fs, *params], allow_unused=True)
    xs, ys = _dev(x, gpu, True), _dev(y, gpu, True)
    fs = feats.float().to(gpu).requires_grad_()
    got = run(lambda a, b, f: radial_graph_message(owner, a, b, radial, f, src.to(gpu), dst.to(gpu),
                                                   mask.float().to(gpu), edge_chunk_size=31),
              xs, ys, fs, list(radial.parameters()), lambda t: t.float().to(gpu))
    xc = {l: v.clone().requires_grad_() for l, v in x.items()}
    yc = {l: v.clone().requires_grad_() for l, v in y.items()}
    fc = feats.clone().requires_grad_()
    want = run(lambda a, b, f: ref.graph_message_blocks(a, b, radial64(f), src, dst, mask), xc, yc, fc,
               list(radial64.parameters()), lambda t: t)
    for i, (a, b) in enumerate(zip(got, want)):
        if b is None:
            assert a is None or float(a.abs().max()) == 0.0
            continue
        assert_rel(a, b, rtol=RTOL_FORCE, what=f"radial message second derivative {i}")


def test_hook_not_handled_cases(gpu):
    from ictc_o3.backends.hip.radial_message import radial_graph_message
    ref, owner, radial64, radial, x, y, feats, src, dst, mask = _case(gpu, 8)
    xs, ys, fs = _dev(x, gpu), _dev(y, gpu), feats.float().to(gpu)
    s, d = src.to(gpu), dst.to(gpu)
    assert radial_graph_message(owner, xs, {l: v[:0] for l, v in ys.items()}, radial, fs[:0], s[:0], d[:0]) is None
    odd = torch.nn.Sequential(radial[0], radial[1])
    assert radial_graph_message(owner, xs, ys, odd, fs, s, d) is None
    live = mask.float().to(gpu).requires_grad_()
    assert radial_graph_message(owner, xs, ys, radial, fs, s, d, live) is None
    with pytest.raises(ValueError):
        radial_graph_message(owner, xs, ys, radial, fs, s, d, edge_chunk_size=0)


def test_packed_lmax3_equals_whole_gates(gpu):
    """C=128, lmax 3 (bond rows from the harmonics), unsorted edges, ranges of 300 edges."""
    from ictc_o3.backends.hip.graph_message import packed_graph_message
    from ictc_o3.backends.hip.radial_message import packed_radial_graph_message
    from ictc_o3.backends.hip.tensor_product import TensorProductPlan
    from ictc_o3.basis.ictd_irreps import triangle_paths
    plan = TensorProductPlan(triangle_paths(3, 3, 3), 128, 3, 3)
    gen = torch.Generator(device=gpu).manual_seed(2)
    nodes, edges, hid = 200, 3000, 64
    x = torch.randn(nodes, plan.x_width, device=gpu, generator=gen).requires_grad_()
    n = torch.nn.functional.normalize(torch.randn(edges, 3, device=gpu, generator=gen), dim=-1)
    from ictc_o3.backends.hip.harmonics import direction_harmonics_packed
    y = direction_harmonics_packed(n, 3).detach().requires_grad_()
    h = torch.randn(edges, hid, device=gpu, generator=gen).requires_grad_()
    w = (torch.randn(plan.full_gate_width, hid, device=gpu, generator=gen) / 8).requires_grad_()
    src = torch.randint(0, nodes, (edges,), device=gpu, generator=gen)
    dst = torch.randint(0, nodes, (edges,), device=gpu, generator=gen)
    got = packed_radial_graph_message(plan, x, y, h, w, None, src, dst, edge_chunk_size=300)
    expect = packed_graph_message(plan, x, y, h @ w.t(), src, dst)
    assert_rel(got, expect, rtol=2e-6, what="streamed vs whole gates")
    go = torch.randn_like(got)
    a = torch.autograd.grad(got, (x, y, h, w), go)
    b = torch.autograd.grad(expect, (x, y, h, w), go)
    # the weight gradient sums over every edge, range by range here and in one product there
    for name, u, v in zip(("x", "Y", "hidden", "weight"), a, b):
        assert_rel(u, v, what=f"streamed vs whole gates grad {name}")


def _mace(gpu, channels, atoms, seed):
    from mace_hip import create_model, radius_graph, sequential_insertion
    zs = (1, 6, 8)
    model = create_model(channels=channels, lmax=3, num_interactions=2, correlation=3, atomic_numbers=zs,
                         cutoff=5.0 if atoms > 500 else 4.0, avg_num_neighbors=12.0, device=gpu, seed=seed)
    st = sequential_insertion(atoms, 0.1 if atoms > 500 else 0.05, min_separation=1.2, num_species=3, seed=seed)
    src, dst, shifts = radius_graph(st.positions, st.cell, 5.0 if atoms > 500 else 4.0)
    graph = dict(positions=st.positions.to(gpu), atomic_numbers=torch.tensor(zs)[st.species].to(gpu),
                 batch=torch.zeros(atoms, dtype=torch.int64, device=gpu), edge_src=src.to(gpu),
                 edge_dst=dst.to(gpu), edge_shifts=shifts.to(gpu), cell=st.cell[None].to(gpu))
    return model, graph


def test_mace_streaming_matches_whole_gates(gpu):
    from mace_hip import energy_and_forces, force_loss
    model, graph = _mace(gpu, 64, 80, 4)
    params = [p for p in model.parameters() if p.requires_grad]
    base = energy_and_forces(model, **graph, training=True)
    gbase = torch.autograd.grad(force_loss(base, 80), params)
    model.set_message_streaming(97)
    got = energy_and_forces(model, **graph, training=True)
    ggot = torch.autograd.grad(force_loss(got, 80), params)
    assert_rel(got["energy"], base["energy"], what="streamed energy")
    assert_rel(got["forces"], base["forces"], what="streamed forces")
    for a, b in zip(ggot, gbase):
        assert_rel(a, b, rtol=RTOL_FORCE, what="streamed training gradient")
    inf = energy_and_forces(model, **graph)
    model.set_message_streaming(None)
    ref = energy_and_forces(model, **graph)
    assert_rel(inf["forces"], ref["forces"], what="streamed inference forces")


def test_mace_streaming_peak_memory_at_cfg4_size(gpu):
    """C=128, lmax 3, 2,048 atoms at 0.1 A^-3, r_c 5 A (~107k edges): inference (energy + forces)
    peak memory with 16,384-edge ranges is lower than with whole gates by at least the
    [E, P*C] gate tensor of the second interaction."""
    from mace_hip import energy_and_forces
    model, graph = _mace(gpu, 128, 2048, 1)
    edges = graph["edge_src"].numel()
    peaks = {}
    for chunk in (None, 16384):
        model.set_message_streaming(chunk)
        energy_and_forces(model, **graph)                  # warm caches (plans, CSR, ranges)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(gpu)
        base = torch.cuda.memory_allocated(gpu)
        out = energy_and_forces(model, **graph)
        torch.cuda.synchronize()
        peaks[chunk] = torch.cuda.max_memory_allocated(gpu) - base
        del out
    gate_bytes = edges * 23 * 128 * 4
    assert peaks[None] - peaks[16384] >= gate_bytes, (peaks, gate_bytes)


def test_mace_streaming_is_deterministic(gpu):
    """Two receiver ranges run on two streams; every sum still has a fixed order, so streamed
    energies and forces (frozen model) and training gradients are bit-identical run to run, with
    several ranges in flight (47-edge ranges)."""
    from mace_hip import energy_and_forces, force_loss
    model, graph = _mace(gpu, 64, 80, 5)
    model.set_message_streaming(47)
    params = [p for p in model.parameters() if p.requires_grad]
    first = energy_and_forces(model, **graph, training=True)
    g1 = torch.autograd.grad(force_loss(first, 80), params)
    second = energy_and_forces(model, **graph, training=True)
    g2 = torch.autograd.grad(force_loss(second, 80), params)
    assert torch.equal(first["forces"], second["forces"]) and torch.equal(first["energy"], second["energy"])
    assert all(torch.equal(a, b) for a, b in zip(g1, g2))
    model.eval().requires_grad_(False)
    a = energy_and_forces(model, **graph)
    b = energy_and_forces(model, **graph)
    assert torch.equal(a["forces"], b["forces"]) and torch.equal(a["energy"], b["energy"])
