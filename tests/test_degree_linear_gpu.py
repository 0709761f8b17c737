"""The fp32-MFMA per-degree channel linear (``csrc/linear_api.hip``,
``ictc_o3/backends/hip/degree_linear.py``): the path-preserving message linear of reference
``pure_cartesian_ictd_fix.py:629-661`` applied to the message kernels' packed output, against a
float64 torch restatement of the same map (blocks rearranged and multiplied per degree):
values, first derivatives (features and every weight) and second derivatives, at the cfg-4
shapes (C = 128, lmax 3, path counts 4/6/7/6), odd channel counts and row counts that do not
fill a tile, and a degree without path blocks (zero output rows).
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


CASES = [((4, 6, 7, 6), 128, 128, 2048, 1 / 50.0), ((3, 4, 4), 64, 64, 77, 0.3), ((2, 0, 3), 40, 24, 33, 1.0),
         ((1,), 16, 8, 5, 2.0)]


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
