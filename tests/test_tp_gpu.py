"""GPU parity of the HIP tensor product (through the C ABI) against the CPU oracle.

Every case feeds identical seeded fp32 bytes to the HIP path and to the float64
oracle (reference CPU path: ``_forward_index_add`` + autograd) and checks the
relative error at the fp32 bar (1e-5).  Covered: forward, VJP to features /
harmonics / gates, mixed second derivatives (gradients of a VJP contraction)
and a third-order derivative, ir_mul and mul_ir layouts, path subsets, live
path weights, channel counts that do not fill a wave, empty inputs, and
size-independent properties at the full benchmark size.
"""
import math

import pytest
import torch

from conftest import RTOL, assert_rel
from oracle import ictc_basis as B
from oracle.tensor_product import TensorProductOracle, enumerate_paths

pytestmark = pytest.mark.gpu


def _inputs(c, lin, le, num_paths, rows, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, c * (lin + 1) ** 2, generator=g)
    n = torch.nn.functional.normalize(torch.randn(rows, 3, generator=g, dtype=torch.float64), dim=-1)
    y = B.direction_harmonics_packed(n, le).float()
    gates = torch.randn(rows, num_paths * c, generator=g) / math.sqrt(num_paths)
    return x, y, gates


def _op(c, lin, le, lout, layout, device, paths=None):
    from ictc_o3 import EdgeTensorProduct
    if paths is None:
        return EdgeTensorProduct.create(channels=c, input_lmax=lin, edge_lmax=le, output_lmax=lout,
                                        layout=layout, device=device)
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    tp = EdgeWeightedPathPreservingTensorProduct(c, max(lin, le, lout), allowed_paths=paths,
                                                 internal_compute_dtype=torch.float32).to(device)
    with torch.no_grad():
        tp.weight.fill_(1.)
    tp.weight.requires_grad_(False)
    return EdgeTensorProduct(tp, input_lmax=lin, edge_lmax=le, layout=layout)


CASES = [
    (64, 2, 2, 2, "ir_mul"),
    (128, 3, 3, 3, "ir_mul"),
    (128, 0, 3, 3, "ir_mul"),
    (96, 2, 2, 2, "ir_mul"),     # NV=1 path, 1.5 waves of channels
    (48, 3, 3, 3, "mul_ir"),     # partial wave, mul_ir layout
    (256, 1, 2, 3, "ir_mul"),
    (32, 3, 1, 0, "ir_mul"),
    (64, 0, 0, 0, "ir_mul"),     # one path: fewer paths than the VJP's prefetch distance
    (16, 1, 1, 1, "mul_ir"),     # fewer channels than lanes
]


@pytest.mark.parametrize("c,lin,le,lout,layout", CASES)
def test_forward_parity(gpu, c, lin, le, lout, layout):
    op = _op(c, lin, le, lout, layout, gpu)
    ref = TensorProductOracle(c, lin, le, lout, layout=layout)
    x, y, g = _inputs(c, lin, le, ref.num_paths, 37, 11)
    out = op(x.to(gpu), y.to(gpu), g.to(gpu))
    expect = ref.forward(x.double(), y.double(), g.double())
    assert out.shape == expect.shape
    assert_rel(out, expect, what="forward")


@pytest.mark.parametrize("c,lin,le,lout,layout", CASES)
def test_vjp_parity(gpu, c, lin, le, lout, layout):
    op = _op(c, lin, le, lout, layout, gpu)
    ref = TensorProductOracle(c, lin, le, lout, layout=layout)
    x, y, g = _inputs(c, lin, le, ref.num_paths, 29, 12)
    go = torch.randn(29, ref.output_width, generator=torch.Generator().manual_seed(13))
    dev = [t.to(gpu).requires_grad_() for t in (x, y, g)]
    grads = torch.autograd.grad(op(*dev), dev, go.to(gpu))
    cpu = [t.double().requires_grad_() for t in (x, y, g)]
    expect = torch.autograd.grad(ref.forward(*cpu), cpu, go.double())
    for name, a, b in zip(("features", "harmonics", "gates"), grads, expect):
        assert_rel(a, b, what=f"grad {name}")


@pytest.mark.parametrize("c,lin,le,lout", [(64, 2, 2, 2), (128, 3, 3, 3), (48, 1, 2, 2)])
def test_mixed_second_derivatives(gpu, c, lin, le, lout):
    """d/d(x,Y,g,go) of <h, VJP(x,Y,g;go)>: exercises every bilinear-substitution term."""
    op = _op(c, lin, le, lout, "ir_mul", gpu)
    ref = TensorProductOracle(c, lin, le, lout)
    rows = 17
    x, y, g = _inputs(c, lin, le, ref.num_paths, rows, 21)
    gen = torch.Generator().manual_seed(22)
    go = torch.randn(rows, ref.output_width, generator=gen)
    hs = [torch.randn(rows, w, generator=gen) for w in (x.shape[1], y.shape[1], g.shape[1])]

    def second(fwd, tensors, dev):
        leaves = [t.to(dev).requires_grad_() for t in tensors]
        first = torch.autograd.grad(fwd(*leaves[:3]), leaves[:3], leaves[3], create_graph=True)
        total = sum((f * h.to(dev)).sum() for f, h in zip(first, hs))
        return torch.autograd.grad(total, leaves)

    dtype_cpu = [t.double() for t in (x, y, g, go)]
    got = second(op, (x, y, g, go), gpu)
    expect = second(ref.forward, dtype_cpu, "cpu")
    for name, a, b in zip(("x", "Y", "g", "go"), got, expect):
        assert_rel(a, b, what=f"mixed second derivative wrt {name}")


def test_third_order(gpu):
    """Third derivatives of a scalar cubic in the TP output (chains the Functions three deep):
    s = sum(w * F^3); d1 = ds/dY, d2 = d<d1,v>/d(Y,x), d3 = d<d2,u>/d(Y,g)."""
    c, lin, le = 64, 2, 2
    op = _op(c, lin, le, 2, "ir_mul", gpu)
    ref = TensorProductOracle(c, lin, le, 2)
    rows = 5
    x, y, g = _inputs(c, lin, le, ref.num_paths, rows, 31)
    gen = torch.Generator().manual_seed(32)
    w = torch.randn(rows, ref.output_width, generator=gen)
    v = torch.randn(rows, y.shape[1], generator=gen)
    u = torch.randn(rows, y.shape[1], generator=gen)

    def third(fwd, xx, yy, gg, ww, vv, uu):
        xx, yy, gg = (t.clone().requires_grad_() for t in (xx, yy, gg))
        s = (fwd(xx, yy, gg) ** 3 * ww).sum()
        (d1,) = torch.autograd.grad(s, yy, create_graph=True)
        d2y, d2x = torch.autograd.grad((d1 * vv).sum(), (yy, xx), create_graph=True)
        d3y, d3g = torch.autograd.grad((d2y * uu).sum() + (d2x ** 2).sum(), (yy, gg))
        return d1, d2y, d2x, d3y, d3g

    got = third(op, *(t.to(gpu) for t in (x, y, g, w, v, u)))
    expect = third(ref.forward, *(t.double() for t in (x, y, g, w, v, u)))
    for name, a, b in zip(("d1", "d2y", "d2x", "d3y", "d3g"), got, expect):
        assert_rel(a, b, rtol=1e-4, what=f"third order {name}")


def test_path_subset_and_live_weight(gpu):
    from ictc_o3 import EdgeTensorProduct
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    paths = [p for p in enumerate_paths(3, 3, 3) if p[0] + p[1] + p[2] != 6]
    c = 64
    tp = EdgeWeightedPathPreservingTensorProduct(c, 3, allowed_paths=paths,
                                                 internal_compute_dtype=torch.float32).to(gpu)
    op = EdgeTensorProduct(tp, input_lmax=3, edge_lmax=3)
    w = tp.weight.detach().cpu().double()
    ref = TensorProductOracle(c, 3, 3, 3, paths=paths, weight=w)
    assert list(op.paths) == ref.paths
    x, y, g = _inputs(c, 3, 3, ref.num_paths, 23, 41)
    out = op(x.to(gpu), y.to(gpu), g.to(gpu))
    assert_rel(out, ref.forward(x.double(), y.double(), g.double()), what="subset forward")
    (dw,) = torch.autograd.grad(out, tp.weight, torch.ones_like(out))
    wr = w.clone().requires_grad_()
    ref.weight = wr
    (dw_ref,) = torch.autograd.grad(ref.forward(x.double(), y.double(), g.double()).sum(), wr)
    assert_rel(dw, dw_ref, what="weight grad")


def test_empty_rows(gpu):
    op = _op(64, 2, 2, 2, "ir_mul", gpu)
    x = torch.zeros(0, 64 * 9, device=gpu, requires_grad=True)
    y = torch.zeros(0, 9, device=gpu)
    g = torch.zeros(0, op.gate_width, device=gpu)
    out = op(x, y, g)
    assert out.shape == (0, op.output_width)
    (dx,) = torch.autograd.grad(out.sum(), x)
    assert dx.shape == x.shape


def test_owner_dict_interface(gpu):
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    c = 32
    paths = enumerate_paths(2, 2, 2)
    tp = EdgeWeightedPathPreservingTensorProduct(c, 2, allowed_paths=paths,
                                                 internal_compute_dtype=torch.float32).to(gpu)
    ref = TensorProductOracle(c, 2, 2, 2, weight=tp.weight.detach().cpu().double())
    x, y, g = _inputs(c, 2, 2, ref.num_paths, 9, 51)
    xb, yb = ref.blocks(x), ref.harmonics(y)
    out = tp({l: v.to(gpu) for l, v in xb.items()}, {l: v.to(gpu) for l, v in yb.items()},
             g.to(gpu).reshape(9, ref.num_paths, c))
    expect = ref.forward_blocks({l: v.double() for l, v in xb.items()},
                                {l: v.double() for l, v in yb.items()}, g.double())
    for l in expect:
        assert_rel(out[l], expect[l], what=f"owner block {l}")


def test_full_size_properties(gpu):
    """At the benchmark size (C128/L3, 131,072 instances): trilinearity of the forward
    and the adjoint identity <F(x,Y,g), o> = <x, Gx> = <g, Gg> = <Y, GY>."""
    from ictc_o3.backends.hip.tensor_product import packed_tensor_product as tensor_product, vjp
    op = _op(128, 3, 3, 3, "ir_mul", gpu)
    plan = op.plan
    rows = 131072
    gen = torch.Generator(device=gpu).manual_seed(61)
    x = torch.randn(rows, plan.x_width, device=gpu, generator=gen)
    n = torch.nn.functional.normalize(torch.randn(rows, 3, device=gpu, generator=gen), dim=-1)
    y = B.direction_harmonics_packed(n.cpu().double(), 3).float().to(gpu)
    g = torch.randn(rows, plan.gate_width, device=gpu, generator=gen)
    o = torch.randn(rows, plan.out_width, device=gpu, generator=gen)
    out = tensor_product(plan, x, y, g)
    out2 = tensor_product(plan, 2.0 * x, y, g)
    assert torch.equal(out2, 2.0 * out)   # power-of-two scaling is exact in fp32
    dx, dy, dg = vjp(plan, (True, True, True), x, y, g, o)
    inner = (out.double() * o.double()).sum(1)
    for name, lhs in (("x", (x.double() * dx.double()).sum(1)), ("Y", (y.double() * dy.double()).sum(1)),
                      ("g", (g.double() * dg.double()).sum(1))):
        err = ((lhs - inner).abs().max() / inner.abs().max()).item()
        assert err < 20 * RTOL, f"adjoint identity for {name}: {err:.2e}"
