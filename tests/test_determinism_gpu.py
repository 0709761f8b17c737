"""Run-to-run determinism and edge-order behaviour of the HIP operators (no atomics in the
message or contraction kernels: every sum has a fixed order).

* the graph message (forward and all three gradients), the symmetric contraction (forward,
  feature VJP, weight gradients) and the MACE energy + forces and force-loss gradients are
  bit-identical when run twice on the same inputs;
* the message under a random permutation of its edge list: node outputs and node-feature
  gradients agree to float32 rounding (the per-receiver sums run in another order), the
  per-edge gradients are the same rows permuted; after the stable re-sort of the shuffled
  edges by (dst, src) every output is bit-identical to the sorted original's.
"""
import math

import pytest
import torch

from conftest import assert_rel

pytestmark = pytest.mark.gpu


def _message_inputs(gpu, c=128, lmax=3, nodes=1500, per=24, seed=5):
    """Edges with unique (dst, src) pairs, sorted by (dst, src)."""
    g = torch.Generator().manual_seed(seed)
    src = torch.stack([torch.randperm(nodes, generator=g)[:per] for _ in range(nodes)]).reshape(-1)
    dst = torch.arange(nodes).repeat_interleave(per)
    order = torch.argsort(dst * nodes + src, stable=True)
    src, dst = src[order], dst[order]
    edges = src.numel()
    npath = {2: 11, 3: 23}[lmax]
    x = torch.randn(nodes, c * (lmax + 1) ** 2, generator=g)
    n = torch.nn.functional.normalize(torch.randn(edges, 3, generator=g), dim=-1)
    gates = torch.randn(edges, npath * c, generator=g) / math.sqrt(npath)
    return [t.to(gpu) for t in (src, dst, x, n, gates)]


def _message(gpu, c, lmax):
    from ictc_o3 import PackedGraphMessage
    return PackedGraphMessage.create(channels=c, input_lmax=lmax, edge_lmax=lmax, output_lmax=lmax, device=gpu)


def _run_message(op, src, dst, x, n, gates, go, lmax):
    from ictc_o3.backends.hip.harmonics import direction_harmonics_packed
    y = direction_harmonics_packed(n, lmax).detach()
    leaves = [t.detach().clone().requires_grad_() for t in (x, y, gates)]
    out = op(*leaves, src, dst)
    grads = torch.autograd.grad(out, leaves, go)
    return [out.detach(), *grads]


@pytest.mark.parametrize("c,lmax", [(128, 3), (64, 2)])
def test_message_bit_identical_twice_and_under_edge_shuffle(gpu, c, lmax):
    op = _message(gpu, c, lmax)
    src, dst, x, n, gates = _message_inputs(gpu, c, lmax)
    go = torch.randn(x.shape[0], op.output_width, generator=torch.Generator(device=gpu).manual_seed(3),
                     device=gpu)
    first = _run_message(op, src, dst, x, n, gates, go, lmax)
    second = _run_message(op, src, dst, x, n, gates, go, lmax)
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    # a random permutation of the edge list
    perm = torch.randperm(src.numel(), generator=torch.Generator().manual_seed(9)).to(gpu)
    shuffled = _run_message(op, src[perm], dst[perm], x, n[perm], gates[perm], go, lmax)
    assert_rel(shuffled[0], first[0], rtol=2e-6, what="shuffled node outputs")
    assert_rel(shuffled[1], first[1], rtol=2e-6, what="shuffled node-feature gradient")
    assert_rel(shuffled[2], first[2][perm], rtol=2e-6, what="shuffled harmonics gradient")
    assert_rel(shuffled[3], first[3][perm], rtol=2e-6, what="shuffled gate gradient")
    # the stable re-sort by (dst, src) restores the original order and with it every bit
    s2, d2 = src[perm], dst[perm]
    back = torch.argsort(d2 * x.shape[0] + s2, stable=True)
    resorted = _run_message(op, s2[back], d2[back], x, n[perm][back], gates[perm][back], go, lmax)
    for a, b in zip(resorted, first):
        assert torch.equal(a, b)


def test_symmetric_contraction_bit_identical_twice(gpu):
    from ictc_o3 import create_symmetric_contraction
    torch.manual_seed(2)
    mod = create_symmetric_contraction(num_elements=10, lmax=3, target_lmax=1, channels=128, correlation=3,
                                       device=gpu)
    gen = torch.Generator(device=gpu).manual_seed(4)
    x = torch.randn(4096, 128 * 16, device=gpu, generator=gen) * 0.5
    species = torch.randint(0, 10, (4096,), device=gpu, generator=gen)
    go = torch.randn(4096, 128 * 4, device=gpu, generator=gen)
    params = [p for con in mod.symmetric_contractions.contractions for p in con.columns()]

    def run():
        xd = x.clone().requires_grad_()
        out = mod(xd, node_type_idx=species)
        return [out.detach(), *torch.autograd.grad(out, [xd, *params], go)]
    for a, b in zip(run(), run()):
        assert torch.equal(a, b)


def test_mace_energy_forces_and_training_gradients_bit_identical_twice(gpu):
    from mace_hip import create_model, energy_and_forces, force_loss, radius_graph, sequential_insertion
    zs = (1, 6, 8)
    model = create_model(channels=64, lmax=3, num_interactions=2, correlation=3, atomic_numbers=zs, cutoff=4.0,
                         avg_num_neighbors=12.0, device=gpu, seed=7)
    st = sequential_insertion(96, 0.05, min_separation=1.2, num_species=3, seed=7)
    src, dst, shifts = radius_graph(st.positions, st.cell, 4.0)
    graph = dict(positions=st.positions.to(gpu), atomic_numbers=torch.tensor(zs)[st.species].to(gpu),
                 batch=torch.zeros(96, dtype=torch.int64, device=gpu), edge_src=src.to(gpu), edge_dst=dst.to(gpu),
                 edge_shifts=shifts.to(gpu), cell=st.cell[None].to(gpu))
    params = [p for p in model.parameters() if p.requires_grad]

    def run():
        pred = energy_and_forces(model, **graph, training=True)
        grads = torch.autograd.grad(force_loss(pred, 96), params)
        return [pred["energy"].detach(), pred["forces"].detach(), *grads]
    for a, b in zip(run(), run()):
        assert torch.equal(a, b)
