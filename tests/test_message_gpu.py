"""GPU parity of the fused graph message (gather -> TP -> receiver segmented sum)
against the oracle's chunked ``index_select -> TP -> index_add`` restatement
(reference backends/ascend/tensor_product.py:189-218), through the C ABI.

Covers unsorted and sorted edge lists, repeated edges, isolated nodes, masks (with
gradient), owned-destination counts below the source count, path subsets, the dict
interface, the empty graph, index validation, mixed second derivatives, and a
full-size (cfg 2 shape) comparison of the fused kernels with the plain TP kernel
followed by a scatter-sum.
"""
import math

import pytest
import torch

from conftest import assert_rel
from oracle import ictc_basis as B
from oracle.tensor_product import TensorProductOracle, enumerate_paths

pytestmark = pytest.mark.gpu


def _graph(nodes, edges, seed, sort=False):
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, nodes, (edges,), generator=g)
    dst = torch.randint(0, nodes - 2, (edges,), generator=g)   # last two nodes receive nothing
    if sort:
        key = dst * nodes + src
        order = torch.argsort(key, stable=True)
        src, dst = src[order], dst[order]
    return src, dst


def _edge_inputs(ref, nodes, edges, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(nodes, ref.input_width, generator=g)
    n = torch.nn.functional.normalize(torch.randn(edges, 3, generator=g, dtype=torch.float64), dim=-1)
    y = B.direction_harmonics_packed(n, ref.edge_lmax).float()
    gates = torch.randn(edges, ref.gate_width, generator=g) / math.sqrt(ref.num_paths)
    return x, y, gates


def _op(c, lin, le, lout, device, layout="ir_mul", paths=None):
    from ictc_o3 import PackedGraphMessage
    if paths is None:
        return PackedGraphMessage.create(channels=c, input_lmax=lin, edge_lmax=le, output_lmax=lout,
                                         layout=layout, device=device)
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    tp = EdgeWeightedPathPreservingTensorProduct(c, max(lin, le, lout), allowed_paths=paths,
                                                 internal_compute_dtype=torch.float32).to(device)
    with torch.no_grad():
        tp.weight.fill_(1.)
    tp.weight.requires_grad_(False)
    return PackedGraphMessage(tp, input_lmax=lin, edge_lmax=le, layout=layout)


# the last two have input degrees without any path (l1 > L_e + L_out): their feature-gradient rows
# are zero
CASES = [(64, 2, 2, 2, False), (128, 3, 3, 3, True), (48, 3, 3, 3, False), (96, 1, 2, 2, True),
         (128, 0, 3, 3, False), (64, 3, 0, 1, True), (32, 2, 1, 0, False), (192, 3, 3, 3, False)]


@pytest.mark.parametrize("c,lin,le,lout,sort", CASES)
def test_forward_and_vjp(gpu, c, lin, le, lout, sort):
    op = _op(c, lin, le, lout, gpu)
    ref = TensorProductOracle(c, lin, le, lout)
    nodes, edges = 30, 211
    src, dst = _graph(nodes, edges, c + lin, sort)
    x, y, g = _edge_inputs(ref, nodes, edges, 7)
    go = torch.randn(nodes, ref.output_width, generator=torch.Generator().manual_seed(8))
    dev = [t.to(gpu).requires_grad_() for t in (x, y, g)]
    out = op(*dev, src.to(gpu), dst.to(gpu))
    cpu = [t.double().requires_grad_() for t in (x, y, g)]
    expect = ref.graph_message(*cpu, src, dst, edge_chunk_size=64)
    assert_rel(out, expect, what="message forward")
    assert out[-2:].abs().max() == 0            # nodes without in-edges
    grads = torch.autograd.grad(out, dev, go.to(gpu))
    egrads = torch.autograd.grad(expect, cpu, go.double())
    for name, a, b in zip(("features", "harmonics", "gates"), grads, egrads):
        assert_rel(a, b, what=f"message grad {name}")


def test_mask_destinations_and_mul_ir(gpu):
    c, lin, le, lout = 64, 2, 2, 2
    op = _op(c, lin, le, lout, gpu, layout="mul_ir")
    ref = TensorProductOracle(c, lin, le, lout, layout="mul_ir")
    nodes, edges = 25, 150
    src, dst = _graph(nodes, edges, 3)
    dst = dst % 20                                   # owned destinations: the first 20 nodes
    op.tp._destination_nodes = 20
    x, y, g = _edge_inputs(ref, nodes, edges, 9)
    mask = (torch.rand(edges, generator=torch.Generator().manual_seed(4)) > 0.25).float()
    mask = mask * torch.rand(edges, generator=torch.Generator().manual_seed(5))
    dev = [t.to(gpu).requires_grad_() for t in (x, y, g, mask)]
    out = op(*dev[:3], src.to(gpu), dst.to(gpu), dev[3])
    cpu = [t.double().requires_grad_() for t in (x, y, g, mask)]
    expect = ref.graph_message(*cpu[:3], src, dst, cpu[3], nodes=20)
    assert out.shape == (20, ref.output_width)
    assert_rel(out, expect, what="masked message")
    go = torch.randn(20, ref.output_width, generator=torch.Generator().manual_seed(6))
    grads = torch.autograd.grad(out, dev, go.to(gpu))
    egrads = torch.autograd.grad(expect, cpu, go.double())
    for name, a, b in zip(("x", "Y", "g", "mask"), grads, egrads):
        assert_rel(a, b, what=f"masked grad {name}")


@pytest.mark.parametrize("c,lin,le,lout", [(64, 2, 2, 2), (128, 3, 3, 3), (48, 3, 3, 3), (96, 0, 3, 3),
                                           (64, 1, 2, 1), (192, 3, 3, 3)])
@pytest.mark.parametrize("fused", [True, False], ids=["tangent_kernels", "substitution"])
def test_mixed_second_derivatives(gpu, c, lin, le, lout, fused, monkeypatch):
    """Second derivatives of <dout, message> contracted with (hx, hY, hg), against the float64
    oracle: once through the fused tangent kernels (the final backward records nothing, so
    the message's double backward uses them) and once through the differentiable
    one-argument substitutions."""
    from ictc_o3.backends.hip import graph_message as gm
    monkeypatch.setattr(gm, "FUSED_SECOND_ORDER", fused)
    op = _op(c, lin, le, lout, gpu)
    ref = TensorProductOracle(c, lin, le, lout)
    nodes, edges = 12, 60
    src, dst = _graph(nodes, edges, 11)
    x, y, g = _edge_inputs(ref, nodes, edges, 12)
    gen = torch.Generator().manual_seed(13)
    go = torch.randn(nodes, ref.output_width, generator=gen)
    hs = [torch.randn(*t.shape, generator=gen) for t in (x, y, g)]

    def second(fwd, tensors, dev, s, d):
        leaves = [t.to(dev).requires_grad_() for t in tensors]
        first = torch.autograd.grad(fwd(*leaves[:3], s.to(dev), d.to(dev)), leaves[:3], leaves[3],
                                    create_graph=True)
        total = sum((f * h.to(dev)).sum() for f, h in zip(first, hs))
        return torch.autograd.grad(total, leaves)

    got = second(op, (x, y, g, go), gpu, src, dst)
    expect = second(lambda a, b, cc, s, d: ref.graph_message(a, b, cc, s, d), [t.double() for t in (x, y, g, go)],
                    "cpu", src, dst)
    for name, a, b in zip(("x", "Y", "g", "go"), got, expect):
        assert_rel(a, b, what=f"message mixed second derivative {name}")


def test_mixed_second_derivatives_masked_destinations_mul_ir(gpu):
    """The tangent-kernel double backward with a mask (with gradient), owned destinations
    below the source count, unsorted edges (receiver permutation) and the mul_ir layout."""
    c, lin, le, lout = 96, 3, 3, 3
    op = _op(c, lin, le, lout, gpu, layout="mul_ir")
    ref = TensorProductOracle(c, lin, le, lout, layout="mul_ir")
    nodes, edges = 21, 120
    src, dst = _graph(nodes, edges, 21)
    dst = dst % 15
    op.tp._destination_nodes = 15
    x, y, g = _edge_inputs(ref, nodes, edges, 22)
    gen = torch.Generator().manual_seed(23)
    mask = (torch.rand(edges, generator=gen) > 0.3).float() * torch.rand(edges, generator=gen)
    go = torch.randn(15, ref.output_width, generator=gen)
    hs = [torch.randn(*t.shape, generator=gen) for t in (x, y, g, mask)]

    def second(fwd, tensors, dev):
        leaves = [t.to(dev).requires_grad_() for t in tensors]
        first = torch.autograd.grad(fwd(*leaves[:4]), leaves[:4], leaves[4], create_graph=True)
        total = sum((f * h.to(dev)).sum() for f, h in zip(first, hs))
        return torch.autograd.grad(total, leaves)

    got = second(lambda a, b, cc, m: op(a, b, cc, src.to(gpu), dst.to(gpu), m), (x, y, g, mask, go), gpu)
    expect = second(lambda a, b, cc, m: ref.graph_message(a, b, cc, src, dst, m, nodes=15),
                    [t.double() for t in (x, y, g, mask, go)], "cpu")
    for name, a, b in zip(("x", "Y", "g", "mask", "go"), got, expect):
        assert_rel(a, b, what=f"masked message mixed second derivative {name}")


def test_dict_interface_subset_and_empty(gpu):
    from ictc_o3 import GraphMessage
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    c = 32
    paths = [p for p in enumerate_paths(2, 2, 2) if p != (1, 1, 1) and p != (2, 2, 0)]
    tp = EdgeWeightedPathPreservingTensorProduct(c, 2, allowed_paths=paths,
                                                 internal_compute_dtype=torch.float32).to(gpu)
    op = GraphMessage(tp, input_lmax=2, edge_lmax=2)
    ref = TensorProductOracle(c, 2, 2, 2, paths=paths, weight=tp.weight.detach().cpu().double())
    nodes, edges = 14, 70
    src, dst = _graph(nodes, edges, 21)
    x, y, g = _edge_inputs(ref, nodes, edges, 22)
    xb, yb = ref.blocks(x), ref.harmonics(y)
    out = op({l: v.to(gpu) for l, v in xb.items()}, {l: v.to(gpu) for l, v in yb.items()}, g.to(gpu),
             src.to(gpu), dst.to(gpu))
    expect = ref.graph_message_blocks({l: v.double() for l, v in xb.items()},
                                      {l: v.double() for l, v in yb.items()}, g.double(), src, dst)
    for l in expect:
        assert_rel(out[l], expect[l], what=f"dict block {l}")
    # empty graph: zeros, still differentiable
    xe = x.to(gpu).requires_grad_()
    empty = _op(c, 2, 2, 2, gpu)(xe, y[:0].to(gpu), torch.zeros(0, 11 * c, device=gpu),
                                 src[:0].to(gpu), dst[:0].to(gpu))
    assert empty.shape == (nodes, 35 * c)
    assert empty.abs().max() == 0
    (dx,) = torch.autograd.grad(empty.sum(), xe)
    assert dx.abs().max() == 0


def test_index_validation(gpu):
    op = _op(32, 1, 1, 1, gpu)
    x = torch.zeros(5, 32 * 4, device=gpu)
    y = torch.zeros(3, 4, device=gpu)
    g = torch.zeros(3, op.gate_width, device=gpu)
    good = torch.tensor([0, 1, 2], device=gpu)
    with pytest.raises(ValueError):
        op(x, y, g, torch.tensor([0, 1, 5], device=gpu), good)
    with pytest.raises(ValueError):
        op(x, y, g, good, torch.tensor([0, -1, 2], device=gpu))
    with pytest.raises(ValueError):
        op(x, y, g, good.int(), good)


def test_full_size_matches_tp_plus_scatter(gpu):
    """cfg 2 shape (16,384 nodes, ~52 in-edges per node, C64/L2): the fused receiver-CSR
    kernels equal the standalone TP kernel followed by a scatter-sum (forward and all
    three gradients), i.e. the fusion changes nothing but the summation order."""
    from ictc_o3 import EdgeTensorProduct
    c, nodes, per = 64, 16384, 52
    edges = nodes * per
    gen = torch.Generator(device=gpu).manual_seed(31)
    msg = _op(c, 2, 2, 2, gpu)
    tp = EdgeTensorProduct(msg.tp, input_lmax=2, edge_lmax=2)
    src = torch.randint(0, nodes, (edges,), device=gpu, generator=gen)
    dst = torch.arange(nodes, device=gpu).repeat_interleave(per)
    x = torch.randn(nodes, 9 * c, device=gpu, generator=gen).requires_grad_()
    n = torch.nn.functional.normalize(torch.randn(edges, 3, device=gpu, generator=gen), dim=-1)
    from ictc_o3.backends.hip.harmonics import direction_harmonics_packed
    y = direction_harmonics_packed(n, 2).detach().requires_grad_()
    g = (torch.randn(edges, 11 * c, device=gpu, generator=gen) / math.sqrt(11)).requires_grad_()
    out = msg(x, y, g, src, dst)
    ref = torch.zeros_like(out).index_add(0, dst, tp(x[src], y, g))
    assert_rel(out, ref, what="fused vs TP+scatter forward")
    go = torch.randn_like(out)
    a = torch.autograd.grad(out, (x, y, g), go)
    b = torch.autograd.grad(ref, (x, y, g), go)
    for name, u, v in zip(("x", "Y", "g"), a, b):
        assert_rel(u, v, what=f"fused vs TP+scatter grad {name}")


@pytest.mark.parametrize("layout", ["ir_mul", "mul_ir"])
def test_frozen_weight_written_through_data(gpu, layout):
    """A frozen path weight changed through ``weight.data`` (no version bump) after a first call:
    the TP folds it into the gates and the message applies it to the receiver rows, both on
    every call (reference gates * weight, packed_tensor_product.py:163-164); values and all
    three gradients against the oracle with that weight, also for the dict hook."""
    from ictc_o3 import EdgeTensorProduct, GraphMessage
    c, lin, le, lout = 64, 2, 2, 2
    paths = [p for i, p in enumerate(enumerate_paths(lin, le, lout)) if i != 3]
    op = _op(c, lin, le, lout, gpu, layout=layout, paths=paths)
    nodes, edges = 20, 160
    src, dst = _graph(nodes, edges, 11)
    plain = TensorProductOracle(c, lin, le, lout, layout=layout, paths=paths)
    x, y, g = _edge_inputs(plain, nodes, edges, 12)
    dev = [t.to(gpu) for t in (x, y, g)]
    op(*dev, src.to(gpu), dst.to(gpu))                       # a first call with the unit weight
    w = torch.randn(plain.num_paths, c, generator=torch.Generator().manual_seed(13))
    op.tp.weight.data.copy_(w.to(gpu))                       # invisible to the version counter
    ref = TensorProductOracle(c, lin, le, lout, layout=layout, paths=paths, weight=w.double())
    go = torch.randn(nodes, ref.output_width, generator=torch.Generator().manual_seed(14))
    cpu = [t.double().requires_grad_() for t in (x, y, g)]
    expect = ref.graph_message(*cpu, src, dst)
    egrads = torch.autograd.grad(expect, cpu, go.double())
    leaves = [t.clone().requires_grad_() for t in dev]
    out = op(*leaves, src.to(gpu), dst.to(gpu))
    assert_rel(out, expect, what="weighted message")
    for name, a, b in zip(("x", "Y", "g"), torch.autograd.grad(out, leaves, go.to(gpu)), egrads):
        assert_rel(a, b, what=f"weighted message grad {name}")
    hook = GraphMessage(op.tp, input_lmax=lin, edge_lmax=le, layout=layout)
    blocks = hook(plain.blocks(dev[0]), plain.harmonics(dev[1]), dev[2], src.to(gpu), dst.to(gpu))
    for l, v in ref.unpack_output(expect.detach()).items():
        assert_rel(blocks[l], v, what=f"weighted dict message l={l}")
    tp = EdgeTensorProduct(op.tp, input_lmax=lin, edge_lmax=le, layout=layout)
    xe = x[src]
    assert_rel(tp(xe.to(gpu), dev[1], dev[2]), ref.forward(xe.double(), y.double(), g.double()),
               what="weighted TP")


@pytest.mark.parametrize("c,lin,le,lout", [(64, 2, 2, 2), (128, 3, 3, 3), (96, 0, 3, 3)])
def test_edge_grad_accumulate_mode(gpu, c, lin, le, lout):
    """ictc_hip_message_edge_grad with accumulate_gates = 1 through the C ABI: grad_gates ends as
    its prior contents plus the gate gradient (bit-identical to adding them afterwards); the
    other outputs are those of the overwriting call."""
    import ctypes
    from ictc_o3 import _lib
    from ictc_o3.backends.hip.graph_message import message_graph
    from ictc_o3.backends.hip.tensor_product import TensorProductPlan
    from ictc_o3.basis.ictd_irreps import triangle_paths
    plan = TensorProductPlan(triangle_paths(lin, le, lout), c, lin, le)
    lib = _lib.lib()
    nodes, edges = 40, 700
    src, dst = _graph(nodes, edges, c + lin)
    g = torch.Generator().manual_seed(21)
    x = torch.randn(nodes, plan.x_width, generator=g).to(gpu)
    n = torch.nn.functional.normalize(torch.randn(edges, 3, generator=g, dtype=torch.float64), dim=-1)
    y = B.direction_harmonics_packed(n, le).float().to(gpu)
    gates = torch.randn(edges, plan.full_gate_width, generator=g).to(gpu)
    go = torch.randn(nodes, plan.full_out_width, generator=g).to(gpu)
    prior = torch.randn(edges, plan.full_gate_width, generator=g).to(gpu)
    graph = message_graph(src.to(gpu), dst.to(gpu), nodes, nodes)
    chunks = lib.ictc_hip_message_chunks(c)
    outs = []
    for acc in (0, 1):
        dyp = torch.empty(edges, chunks, plan.y_width, device=gpu)
        dg = prior.clone() if acc else torch.empty_like(prior)
        dxe = torch.empty(edges, plan.x_width, device=gpu)
        print(f"edge grad accumulate={acc}: C={c} degrees={(lin, le, lout)}", flush=True)
        _lib.check(lib.ictc_hip_message_edge_grad(
            ctypes.byref(plan.desc), x.data_ptr(), y.data_ptr(), gates.data_ptr(), go.data_ptr(),
            graph.src.data_ptr(), graph.rowptr_dst.data_ptr(), _lib.ptr(graph.perm_dst), dyp.data_ptr(),
            dg.data_ptr(), dxe.data_ptr(), nodes, nodes, edges, acc, _lib.stream_of(gpu)), "edge_grad")
        outs.append((dyp, dg, dxe))
    torch.cuda.synchronize()
    assert torch.equal(outs[1][1], outs[0][1] + prior)
    assert torch.equal(outs[1][0], outs[0][0]) and torch.equal(outs[1][2], outs[0][2])
