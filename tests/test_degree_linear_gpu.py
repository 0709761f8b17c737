"""The fp32-MFMA per-degree channel linear (``csrc/linear_api.hip``,
``ictc_o3/backends/hip/degree_linear.py``): the path-preserving message linear of reference
``pure_cartesian_ictd_fix.py:629-661`` applied to the message kernels' packed output, against a
float64 torch restatement of the same map (blocks rearranged and multiplied per degree):
values, first derivatives (features and every weight) and second derivatives, at the cfg-4
shapes (C = 128, lmax 3, path counts 4/6/7/6), odd channel counts and row counts that do not
fill a tile, and a degree without path blocks (zero output rows); and the adjoint map used as an
operator of its own (the interaction's linear_up, mul_ir -> ir_mul, reference
``ictd_irreps.py:187-207``), against the same restatement's transpose.
"""
import pytest
import torch

from conftest import assert_rel

pytestmark = pytest.mark.gpu


def _reference(x, weights, counts, c, o, alpha):
    n = x.shape[0]
    out, off = [], 0
    for l, k in enumerate(counts):
        d = 2 * l + 1
        blk = x[:, off:off + k * d * c].reshape(n, k, d, c)
        off += k * d * c
        if k == 0:
            out.append(x.new_zeros(n, o * d))
            continue
        rows = blk.transpose(1, 2).reshape(n * d, k * c)
        y = (rows @ weights[l].t()) * alpha
        out.append(y.reshape(n, d, o).transpose(1, 2).reshape(n, o * d))
    return torch.cat(out, -1)


# the vector path (C a multiple of 32) at the cfg-4 shape, with column counts that end inside a
# 128-column tile (32, 96, 64: the clamped weight runs), with a degree without path blocks, and
# with O not a multiple of 32 (its input adjoint on the element-wise path); the element-wise path
# with odd C and O; rows of a degree split over several 512-row ranges of the weight adjoint
# (the last one partial) and O past one 128-row tile
CASES = [((4, 6, 7, 6), 128, 128, 2048, 1 / 50.0), ((3, 4, 4), 64, 64, 77, 0.3), ((1, 3, 2), 32, 64, 45, 0.7),
         ((3, 0, 2), 64, 96, 70, 1.5), ((1, 1), 96, 40, 29, 1.0), ((2, 0, 3), 40, 24, 33, 1.0),
         ((1,), 16, 8, 5, 2.0), ((2, 3, 1), 64, 160, 600, 0.5)]


@pytest.mark.parametrize("counts,c,o,nodes,alpha", CASES)
def test_values_and_derivatives(gpu, counts, c, o, nodes, alpha):
    from ictc_o3.backends.hip.degree_linear import DegreeLinearPlan, degree_linear
    g = torch.Generator().manual_seed(len(counts) * 100 + c)
    plan = DegreeLinearPlan(counts, c, o)
    x = torch.randn(nodes, plan.in_width, generator=g, dtype=torch.float64)
    ws = [torch.randn(o, k * c, generator=g, dtype=torch.float64) / max(1, k * c) ** 0.5 for k in counts]
    xd = x.float().to(gpu).requires_grad_()
    wd = [w.float().to(gpu).requires_grad_() for w in ws]
    xc = x.clone().requires_grad_()
    wc = [w.clone().requires_grad_() for w in ws]
    got = degree_linear(xd, wd, plan, alpha)
    want = _reference(xc, wc, counts, c, o, alpha)
    assert got.shape == want.shape == (nodes, o * len(counts) ** 2)
    assert_rel(got, want, what="degree linear forward")
    gy = torch.randn(want.shape, generator=g, dtype=torch.float64)
    live_w = [w for w, k in zip(wd, counts) if k]
    live_wc = [w for w, k in zip(wc, counts) if k]
    first = torch.autograd.grad(got, [xd, *live_w], gy.float().to(gpu), create_graph=True)
    efirst = torch.autograd.grad(want, [xc, *live_wc], gy.clone().requires_grad_(), create_graph=True)
    for i, (a, b) in enumerate(zip(first, efirst)):
        assert_rel(a, b, what=f"degree linear first derivative {i}")
    # second derivatives: d/d(x, W) of <h, dL/dx> + sum <v_l, dL/dW_l>
    hs = [torch.randn(t.shape, generator=g, dtype=torch.float64) for t in efirst]
    loss = sum((a * h.float().to(gpu)).sum() for a, h in zip(first, hs))
    eloss = sum((a * h).sum() for a, h in zip(efirst, hs))
    second = torch.autograd.grad(loss, [xd, *live_w], allow_unused=True)
    esecond = torch.autograd.grad(eloss, [xc, *live_wc], allow_unused=True)
    for i, (a, b) in enumerate(zip(second, esecond)):
        if b is None:
            assert a is None or float(a.abs().max()) == 0.0
            continue
        assert_rel(a, b, what=f"degree linear second derivative {i}")


def test_bit_identical_twice_and_validation(gpu):
    from ictc_o3.backends.hip.degree_linear import DegreeLinearPlan, degree_linear
    plan = DegreeLinearPlan((4, 6, 7, 6), 128, 128)
    gen = torch.Generator(device=gpu).manual_seed(1)
    x = torch.randn(300, plan.in_width, device=gpu, generator=gen)
    ws = [torch.randn(128, k * 128, device=gpu, generator=gen) for k in plan.counts]
    assert torch.equal(degree_linear(x, ws, plan, 0.02), degree_linear(x, ws, plan, 0.02))
    with pytest.raises(ValueError):
        degree_linear(x[:, 1:], ws, plan)
    with pytest.raises(ValueError):
        degree_linear(x, ws[:3], plan)


@pytest.mark.parametrize("lmax,c,nodes", [(3, 128, 2048), (2, 64, 91), (3, 48, 37), (0, 32, 10)])
def test_channel_linear_up(gpu, lmax, c, nodes):
    """y[n, l][m][o] = sum_c W_l[o, c] x[n, l][c][m]: mul_ir in, ir_mul out, values and first and
    second derivatives (features and every weight) against float64 torch."""
    from ictc_o3.backends.hip.degree_linear import DegreeLinearPlan, degree_linear_adjoint
    g = torch.Generator().manual_seed(lmax * 1000 + c)
    plan = DegreeLinearPlan([1] * (lmax + 1), c, c)
    x = torch.randn(nodes, c * (lmax + 1) ** 2, generator=g, dtype=torch.float64)
    ws = [torch.randn(c, c, generator=g, dtype=torch.float64) / c ** 0.5 for _ in range(lmax + 1)]

    def reference(x, ws):
        out, off = [], 0
        for l, w in enumerate(ws):
            d = 2 * l + 1
            blk = x[:, off:off + c * d].reshape(-1, c, d)
            off += c * d
            out.append(torch.einsum("oc,ncm->nmo", w, blk).reshape(x.shape[0], -1))
        return torch.cat(out, -1)
    xd = x.float().to(gpu).requires_grad_()
    wd = [w.float().to(gpu).requires_grad_() for w in ws]
    xc = x.clone().requires_grad_()
    wc = [w.clone().requires_grad_() for w in ws]
    got = degree_linear_adjoint(xd, [w.t() for w in wd], plan)
    want = reference(xc, wc)
    assert got.shape == want.shape
    assert_rel(got, want, what="linear_up forward")
    gy = torch.randn(want.shape, generator=g, dtype=torch.float64)
    first = torch.autograd.grad(got, [xd, *wd], gy.float().to(gpu), create_graph=True)
    efirst = torch.autograd.grad(want, [xc, *wc], gy, create_graph=True)
    for i, (a, b) in enumerate(zip(first, efirst)):
        assert_rel(a, b, what=f"linear_up first derivative {i}")
    hs = [torch.randn(t.shape, generator=g, dtype=torch.float64) for t in efirst]
    loss = sum((a * h.float().to(gpu)).sum() for a, h in zip(first, hs))
    eloss = sum((a * h).sum() for a, h in zip(efirst, hs))
    second = torch.autograd.grad(loss, [xd, *wd], allow_unused=True)
    esecond = torch.autograd.grad(eloss, [xc, *wc], allow_unused=True)
    for i, (a, b) in enumerate(zip(second, esecond)):
        if b is None:
            assert a is None or float(a.abs().max()) == 0.0
            continue
        assert_rel(a, b, what=f"linear_up second derivative {i}")


@pytest.mark.parametrize("lmax,c,o,nodes", [(3, 128, 128, 2048), (2, 64, 32, 91), (1, 48, 40, 37), (1, 64, 136, 700)])
def test_mul_ir_map(gpu, lmax, c, o, nodes):
    """y[n, l][o][m] = alpha sum_c W_l[o, c] x[n, l][c][m] (the product block's o3.Linear): mul_ir
    in and out, values and first and second derivatives against float64 torch; a plan with more
    than one block per degree is refused."""
    from ictc_o3.backends.hip.degree_linear import DegreeLinearPlan, degree_linear_mul_ir
    g = torch.Generator().manual_seed(lmax * 100 + c + o)
    plan = DegreeLinearPlan([1] * (lmax + 1), c, o)
    alpha = 1.0 / c ** 0.5
    x = torch.randn(nodes, c * (lmax + 1) ** 2, generator=g, dtype=torch.float64)
    ws = [torch.randn(o, c, generator=g, dtype=torch.float64) for _ in range(lmax + 1)]

    def reference(x, ws):
        out, off = [], 0
        for l, w in enumerate(ws):
            d = 2 * l + 1
            blk = x[:, off:off + c * d].reshape(-1, c, d)
            off += c * d
            out.append((torch.einsum("oc,ncm->nom", w, blk) * alpha).reshape(x.shape[0], -1))
        return torch.cat(out, -1)
    xd = x.float().to(gpu).requires_grad_()
    wd = [w.float().to(gpu).requires_grad_() for w in ws]
    xc = x.clone().requires_grad_()
    wc = [w.clone().requires_grad_() for w in ws]
    got = degree_linear_mul_ir(xd, wd, plan, alpha)
    want = reference(xc, wc)
    assert got.shape == want.shape
    assert_rel(got, want, what="mul_ir map forward")
    gy = torch.randn(want.shape, generator=g, dtype=torch.float64)
    first = torch.autograd.grad(got, [xd, *wd], gy.float().to(gpu), create_graph=True)
    efirst = torch.autograd.grad(want, [xc, *wc], gy, create_graph=True)
    for i, (a, b) in enumerate(zip(first, efirst)):
        assert_rel(a, b, what=f"mul_ir map first derivative {i}")
    hs = [torch.randn(t.shape, generator=g, dtype=torch.float64) for t in efirst]
    loss = sum((a * h.float().to(gpu)).sum() for a, h in zip(first, hs))
    eloss = sum((a * h).sum() for a, h in zip(efirst, hs))
    second = torch.autograd.grad(loss, [xd, *wd], allow_unused=True)
    esecond = torch.autograd.grad(eloss, [xc, *wc], allow_unused=True)
    for i, (a, b) in enumerate(zip(second, esecond)):
        if b is None:
            assert a is None or float(a.abs().max()) == 0.0
            continue
        assert_rel(a, b, what=f"mul_ir map second derivative {i}")
    with pytest.raises(ValueError):
        degree_linear_mul_ir(xd, wd, DegreeLinearPlan([2] * (lmax + 1), c, o), alpha)
