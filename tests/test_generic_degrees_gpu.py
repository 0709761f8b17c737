"""GPU parity of the degree sets with a degree of 4 to 6 against the float64 oracle, through the
C ABI: the degree-generic kernels (path tables and CG tensors read at run time), and for the TP
entry points at (4, 4, 4) the compiled per-degree forward and the wide VJP: tensor product forward / VJP / mixed second derivatives, graph message forward / VJP /
mixed second derivatives (the substitution route: these degrees have no fused tangent
kernels), the message VJP through the allocation-free entry point, and size-independent
properties at a larger size (rotation equivariance, the adjoint identity, message over the
identity graph = tensor product, run-to-run determinism).

The oracle's CG tensors for every triple up to degree 6 are pinned by the Gaunt closed form
and equivariance (tests/test_oracle_basis.py).
"""
import ctypes
import math

import pytest
import torch

from conftest import RTOL, assert_rel
from oracle import ictc_basis as B
from oracle.tensor_product import TensorProductOracle

pytestmark = pytest.mark.gpu

# (C, input_lmax, edge_lmax, output_lmax): C = 70 covers a partial second channel chunk; (4, 2, 1)
# has an input degree without any path (4 > 2 + 1), whose feature-gradient rows are zero.  The
# (4, 4, 4) cases run the compiled kernels: C = 32 a partial first chunk, C = 70 a partial second
# chunk of the wide VJP, C = 128 the two-channels-per-lane forward.
TP_CASES = [(32, 4, 4, 4, "ir_mul"), (70, 4, 4, 4, "mul_ir"), (128, 4, 4, 4, "ir_mul"), (16, 6, 6, 6, "ir_mul"),
            (70, 5, 3, 6, "mul_ir"), (24, 4, 2, 1, "ir_mul"), (8, 0, 5, 5, "ir_mul")]
MSG_CASES = [(32, 4, 4, 4, False), (70, 5, 2, 4, True), (16, 6, 6, 6, False), (24, 4, 2, 1, True)]


def _tp(c, lin, le, lout, layout, device):
    from ictc_o3 import EdgeTensorProduct
    return EdgeTensorProduct.create(channels=c, input_lmax=lin, edge_lmax=le, output_lmax=lout, layout=layout,
                                    device=device)


def _inputs(ref, rows, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, ref.input_width, generator=g)
    n = torch.nn.functional.normalize(torch.randn(rows, 3, generator=g, dtype=torch.float64), dim=-1)
    y = B.direction_harmonics_packed(n, ref.edge_lmax).float()
    gates = torch.randn(rows, ref.gate_width, generator=g) / math.sqrt(ref.num_paths)
    return x, y, gates


def test_plans_use_generic_kernels():
    from ictc_o3.backends.hip.tensor_product import TensorProductPlan
    from ictc_o3.basis.ictd_irreps import triangle_paths
    assert TensorProductPlan(triangle_paths(4, 4, 4), 8, 4, 4).generic
    assert not TensorProductPlan(triangle_paths(3, 3, 3), 8, 3, 3).generic
    with pytest.raises(ValueError):
        TensorProductPlan(triangle_paths(7, 1, 6), 8, 7, 1)


@pytest.mark.parametrize("c,lin,le,lout,layout", TP_CASES)
def test_tp_forward_and_vjp(gpu, c, lin, le, lout, layout):
    op = _tp(c, lin, le, lout, layout, gpu)
    assert op.plan.generic
    ref = TensorProductOracle(c, lin, le, lout, layout=layout)
    rows = 19
    x, y, g = _inputs(ref, rows, 40 + lin)
    go = torch.randn(rows, ref.output_width, generator=torch.Generator().manual_seed(41))
    dev = [t.to(gpu).requires_grad_() for t in (x, y, g)]
    out = op(*dev)
    cpu = [t.double().requires_grad_() for t in (x, y, g)]
    expect = ref.forward(*cpu)
    assert_rel(out, expect, what="generic forward")
    grads = torch.autograd.grad(out, dev, go.to(gpu))
    egrads = torch.autograd.grad(expect, cpu, go.double())
    for name, a, b in zip(("features", "harmonics", "gates"), grads, egrads):
        assert_rel(a, b, what=f"generic grad {name}")


def test_tp_mixed_second_derivatives(gpu):
    c, lin, le, lout = 24, 4, 4, 4
    op = _tp(c, lin, le, lout, "ir_mul", gpu)
    ref = TensorProductOracle(c, lin, le, lout)
    rows = 9
    x, y, g = _inputs(ref, rows, 51)
    gen = torch.Generator().manual_seed(52)
    go = torch.randn(rows, ref.output_width, generator=gen)
    hs = [torch.randn(*t.shape, generator=gen) for t in (x, y, g)]

    def second(fwd, tensors, dev):
        leaves = [t.to(dev).requires_grad_() for t in tensors]
        first = torch.autograd.grad(fwd(*leaves[:3]), leaves[:3], leaves[3], create_graph=True)
        return torch.autograd.grad(sum((f * h.to(dev)).sum() for f, h in zip(first, hs)), leaves)

    got = second(op, (x, y, g, go), gpu)
    expect = second(ref.forward, [t.double() for t in (x, y, g, go)], "cpu")
    for name, a, b in zip(("x", "Y", "g", "go"), got, expect):
        assert_rel(a, b, what=f"generic mixed second derivative wrt {name}")


def _msg(c, lin, le, lout, device):
    from ictc_o3 import PackedGraphMessage
    return PackedGraphMessage.create(channels=c, input_lmax=lin, edge_lmax=le, output_lmax=lout, device=device)


def _graph(nodes, edges, seed, sort):
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, nodes, (edges,), generator=g)
    dst = torch.randint(0, nodes - 2, (edges,), generator=g)   # the last two nodes receive nothing
    if sort:
        order = torch.argsort(dst * nodes + src, stable=True)
        src, dst = src[order], dst[order]
    return src, dst


@pytest.mark.parametrize("c,lin,le,lout,sort", MSG_CASES)
def test_message_forward_and_vjp(gpu, c, lin, le, lout, sort):
    op = _msg(c, lin, le, lout, gpu)
    ref = TensorProductOracle(c, lin, le, lout)
    nodes, edges = 14, 67
    src, dst = _graph(nodes, edges, c + lin, sort)
    g0 = torch.Generator().manual_seed(61)
    x = torch.randn(nodes, ref.input_width, generator=g0)
    _, y, g = _inputs(ref, edges, 62)
    go = torch.randn(nodes, ref.output_width, generator=g0)
    dev = [t.to(gpu).requires_grad_() for t in (x, y, g)]
    out = op(*dev, src.to(gpu), dst.to(gpu))
    cpu = [t.double().requires_grad_() for t in (x, y, g)]
    expect = ref.graph_message(*cpu, src, dst, edge_chunk_size=16)
    assert_rel(out, expect, what="generic message forward")
    assert out[-2:].abs().max() == 0
    grads = torch.autograd.grad(out, dev, go.to(gpu))
    egrads = torch.autograd.grad(expect, cpu, go.double())
    for name, a, b in zip(("features", "harmonics", "gates"), grads, egrads):
        assert_rel(a, b, what=f"generic message grad {name}")


@pytest.mark.parametrize("fused", [True, False], ids=["fused_requested", "substitution"])
def test_message_mixed_second_derivatives(gpu, fused, monkeypatch):
    """With the fused tangent route requested, generic degrees still take the substitutions."""
    from ictc_o3.backends.hip import graph_message as gm
    monkeypatch.setattr(gm, "FUSED_SECOND_ORDER", fused)
    c, lin, le, lout = 16, 4, 3, 4
    op = _msg(c, lin, le, lout, gpu)
    ref = TensorProductOracle(c, lin, le, lout)
    nodes, edges = 9, 40
    src, dst = _graph(nodes, edges, 71, False)
    g0 = torch.Generator().manual_seed(72)
    x = torch.randn(nodes, ref.input_width, generator=g0)
    _, y, g = _inputs(ref, edges, 73)
    go = torch.randn(nodes, ref.output_width, generator=g0)
    hs = [torch.randn(*t.shape, generator=g0) for t in (x, y, g)]

    def second(fwd, tensors, dev):
        leaves = [t.to(dev).requires_grad_() for t in tensors]
        first = torch.autograd.grad(fwd(*leaves[:3], src.to(dev), dst.to(dev)), leaves[:3], leaves[3],
                                    create_graph=True)
        return torch.autograd.grad(sum((f * h.to(dev)).sum() for f, h in zip(first, hs)), leaves)

    got = second(op, (x, y, g, go), gpu)
    expect = second(lambda a, b, cc, s, d: ref.graph_message(a, b, cc, s, d), [t.double() for t in (x, y, g, go)],
                    "cpu")
    for name, a, b in zip(("x", "Y", "g", "go"), got, expect):
        assert_rel(a, b, what=f"generic message mixed second derivative {name}")


def test_message_vjp_allocation_free_entry_point(gpu):
    """ictc_hip_message_edge_grad_static (harmonics gradient summed in the library) matches the
    partial-sum entry point for a generic degree set, on two calls in a row."""
    from ictc_o3 import _lib
    from ictc_o3.backends.hip.graph_message import message_graph
    c, lin, le, lout = 130, 4, 2, 3          # three channel chunks
    op = _msg(c, lin, le, lout, gpu)
    plan = op.plan
    lib = _lib.lib()
    for nodes, edges, seed in ((20, 150, 81), (7, 23, 82)):
        src, dst = (t.to(gpu) for t in _graph(nodes, edges, seed, False))
        graph = message_graph(src, dst, nodes, nodes)
        gen = torch.Generator(device=gpu).manual_seed(seed)
        x = torch.randn(nodes, plan.x_width, device=gpu, generator=gen)
        y = torch.randn(edges, plan.y_width, device=gpu, generator=gen)
        g = torch.randn(edges, plan.full_gate_width, device=gpu, generator=gen)
        go = torch.randn(nodes, plan.full_out_width, device=gpu, generator=gen)
        nch = lib.ictc_hip_message_chunks(c)
        dyp = torch.empty(edges, nch, plan.y_width, device=gpu)
        dg1, dg2 = (torch.empty(edges, plan.full_gate_width, device=gpu) for _ in range(2))
        dx1, dx2 = (torch.empty(edges, plan.x_width, device=gpu) for _ in range(2))
        dy2 = torch.empty(edges, plan.y_width, device=gpu)
        perm = None if graph.perm_dst is None else graph.perm_dst.data_ptr()
        common = (x.data_ptr(), y.data_ptr(), g.data_ptr(), go.data_ptr(), graph.src.data_ptr(),
                  graph.rowptr_dst.data_ptr(), perm)
        stream = _lib.stream_of(gpu)
        _lib.check(lib.ictc_hip_message_edge_grad(ctypes.byref(plan.desc), *common, dyp.data_ptr(), dg1.data_ptr(),
                                                  dx1.data_ptr(), nodes, nodes, edges, 0, stream), "edge_grad")
        _lib.check(lib.ictc_hip_message_edge_grad_static(ctypes.byref(plan.desc), *common, dy2.data_ptr(),
                                                         dg2.data_ptr(), dx2.data_ptr(), nodes, nodes, edges, stream),
                   "edge_grad_static")
        torch.cuda.synchronize()
        assert torch.equal(dyp.sum(1), dy2)
        assert torch.equal(dg1, dg2) and torch.equal(dx1, dx2)


def _rotate_blocks(t, widths_l, channels, d):
    """Rotate an ir_mul packed tensor [rows, sum (2l+1) C] whose blocks have degrees widths_l."""
    out, off, rows = [], 0, t.shape[0]
    for l in widths_l:
        n = (2 * l + 1) * channels
        blk = t[:, off:off + n].reshape(rows, 2 * l + 1, channels)
        out.append(torch.einsum("ab,rbc->rac", d[l], blk).reshape(rows, n))
        off += n
    return torch.cat(out, 1)


def test_full_size_properties(gpu):
    """20,000 rows at C = 64, degrees (4, 4, 4): rotation equivariance of the forward, the
    adjoint identity <F(x,Y,g), o> = <x, Gx> = <Y, GY> = <g, Gg>, the message over the identity
    graph equals the TP (two different kernels), and bit-identical repeat runs."""
    from ictc_o3.backends.hip.graph_message import packed_graph_message
    from ictc_o3.backends.hip.tensor_product import packed_tensor_product, vjp
    c, lin, le, lout = 64, 4, 4, 4
    op = _tp(c, lin, le, lout, "ir_mul", gpu)
    plan = op.plan
    ref = TensorProductOracle(c, lin, le, lout)
    rows = 20000
    gen = torch.Generator(device=gpu).manual_seed(91)
    x = torch.randn(rows, plan.x_width, device=gpu, generator=gen)
    nrm = torch.nn.functional.normalize(torch.randn(rows, 3, dtype=torch.float64, generator=torch.Generator()
                                                    .manual_seed(92)), dim=-1)
    y = B.direction_harmonics_packed(nrm, le).float().to(gpu)
    g = torch.randn(rows, plan.gate_width, device=gpu, generator=gen)
    o = torch.randn(rows, plan.out_width, device=gpu, generator=gen)
    out = packed_tensor_product(plan, x, y, g)
    assert torch.equal(out, packed_tensor_product(plan, x, y, g))
    # equivariance: F(D x, D Y, g) = D F(x, Y, g)
    omega = torch.tensor([0.3, -1.1, 0.7], dtype=torch.float64)
    d = {l: B.wigner_d(l, omega).float().to(gpu) for l in range(max(lin, le, lout) + 1)}
    rx = _rotate_blocks(x, range(lin + 1), c, d)
    ry = _rotate_blocks(y, range(le + 1), 1, d)
    out_l = [p[2] for p in sorted(ref.paths, key=lambda p: p[2])]
    rout = packed_tensor_product(plan, rx, ry, g)
    assert_rel(rout, _rotate_blocks(out, out_l, c, d), rtol=20 * RTOL, what="equivariance")
    # adjoint identity
    dx, dy, dg = vjp(plan, (True, True, True), x, y, g, o)
    inner = (out.double() * o.double()).sum(1)
    for name, lhs in (("x", (x.double() * dx.double()).sum(1)), ("Y", (y.double() * dy.double()).sum(1)),
                      ("g", (g.double() * dg.double()).sum(1))):
        err = ((lhs - inner).abs().max() / inner.abs().max()).item()
        assert err < 20 * RTOL, f"adjoint identity for {name}: {err:.2e}"
    # identity graph: node n receives exactly edge n
    idx = torch.arange(rows, device=gpu)
    msg = packed_graph_message(plan, x, y, g, idx, idx)
    assert_rel(msg, out, rtol=RTOL, what="identity-graph message")
