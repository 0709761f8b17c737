"""ictc_o3.backends.hip.linear (the model's dense layers): the split-K matrix product equals
a @ b, and its first and second derivatives (every derivative is the same Function) pass
gradcheck / gradgradcheck.  Small row blocks force the split path (several blocks plus a
remainder) on the CPU.  On the GPU the plain products run through ictc_hip_sgemm with the
operands' storage order passed as transpose flags."""
import pytest
import torch

from ictc_o3.backends.hip import linear as L
from mace_hip.linear import Linear


@pytest.fixture
def small_blocks(monkeypatch):
    monkeypatch.setattr(L, "SPLIT_ROWS", 8)


@pytest.mark.parametrize("m,k,n", [(3, 200, 4), (4, 203, 2), (6, 50, 5), (40, 30, 2)])
def test_product_and_derivatives(small_blocks, m, k, n):
    g = torch.Generator().manual_seed(m * 1000 + k + n)
    a = torch.randn(m, k, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(k, n, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.allclose(L.mm(a, b), a @ b, atol=1e-12)
    assert torch.autograd.gradcheck(L.mm, (a, b))
    assert torch.autograd.gradgradcheck(L.mm, (a, b))


def test_split_path_taken_for_transposed_activations(small_blocks):
    """The weight-gradient shape (a transposed [K, M] activation times a [K, N] cotangent)
    goes through the row-block path and matches the plain product."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1000, 4, generator=g, dtype=torch.float64)
    y = torch.randn(1000, 3, generator=g, dtype=torch.float64)
    assert 1000 // L.SPLIT_ROWS >= 2 and 1000 >= L.SPLIT_MIN_RATIO * 4
    assert torch.allclose(L._product(x.t(), y), x.t() @ y, atol=1e-11)


def test_linear_module_keeps_parameter_contract():
    lin = Linear(8, 5)
    assert [n for n, _ in lin.named_parameters()] == ["weight"] and lin.weight.shape == (5, 8)
    x = torch.randn(7, 3, 8)
    assert torch.allclose(lin(x), x @ lin.weight.t(), atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("k,n", [(64, 64), (64, 512), (64, 2944), (8, 64)])
def test_tall_products_on_gpu(k, n):
    """Edge-sized products ([E, K] @ [K, N]) on ictc_hip_sgemm; value, first and second
    derivatives (all through the same Function, the weight gradient through the split-K
    path) against float64, with the right operand both row-major and a transposed weight."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    dev = torch.device("cuda", 0)
    rows = 40000 + 1234
    g = torch.Generator().manual_seed(n + k)
    a64 = torch.randn(rows, k, generator=g, dtype=torch.float64)
    w64 = torch.randn(n, k, generator=g, dtype=torch.float64) / 8
    go = torch.randn(rows, n, generator=g, dtype=torch.float64)
    h = torch.randn(rows, k, generator=g, dtype=torch.float64)

    def run(a, w, transposed):
        a = a.clone().requires_grad_()
        w = w.clone().requires_grad_()
        right = w.t() if transposed else w.t().contiguous()
        out = L.mm(a, right) if a.is_cuda else a @ right
        ga, = torch.autograd.grad(out, a, go.to(a.device), create_graph=True)
        second = torch.autograd.grad((ga * h.to(a.device)).sum(), w)[0]
        return out, ga, second

    for transposed in (True, False):
        got = run(a64.float().to(dev), w64.float().to(dev), transposed)
        expect = run(a64, w64, transposed)
        for name, x, y in zip(("product", "input grad", "weight grad of input grad"), got, expect):
            err = (x.double().cpu() - y).abs().max() / y.abs().max()
            assert err < 1e-5, f"{name} (transposed={transposed}): relative error {err:.2e}"


@pytest.mark.gpu
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_storage_orders(ta, tb):
    """ictc_hip_sgemm through every storage order of both operands, including row strides
    larger than the row (slices of wider tensors), against float64."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(ta * 2 + tb)
    m, k, n = 37, 19, 23
    a = torch.randn(m, k, generator=g, dtype=torch.float64)
    b = torch.randn(k, n, generator=g, dtype=torch.float64)
    wide_a = torch.randn(m + 5, k + 3, generator=g, dtype=torch.float64) if not ta else \
        torch.randn(k + 3, m + 5, generator=g, dtype=torch.float64)
    wide_b = torch.randn(k + 2, n + 4, generator=g, dtype=torch.float64) if not tb else \
        torch.randn(n + 4, k + 2, generator=g, dtype=torch.float64)
    if ta:
        wide_a[:k, :m] = a.t()
        av = wide_a.float().to(dev)[:k, :m].t()
    else:
        wide_a[:m, :k] = a
        av = wide_a.float().to(dev)[:m, :k]
    if tb:
        wide_b[:n, :k] = b.t()
        bv = wide_b.float().to(dev)[:n, :k].t()
    else:
        wide_b[:k, :n] = b
        bv = wide_b.float().to(dev)[:k, :n]
    assert L._storage(av)[1] == ta and L._storage(bv)[1] == tb
    got = L._sgemm(av, bv).double().cpu()
    err = (got - a @ b).abs().max() / (a @ b).abs().max()
    assert err < 1e-6, f"relative error {err:.2e}"


@pytest.mark.gpu
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_k_zero_scales_c(ta, tb):
    """ictc_hip_sgemm with k = 0 through the C ABI: C = beta * C whatever leading dimensions and
    operand pointers the caller passes (rocBLAS's own checks do not apply to unread operands)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ictc_o3 import _lib
    dev = torch.device("cuda", 0)
    m, n = 37, 23
    c = torch.randn(m, n, device=dev)
    want = c * 0.5
    st = _lib.lib().ictc_hip_sgemm(ta, tb, m, n, 0, 1.0, None, 0, None, 0, 0.5, c.data_ptr(), n,
                                   _lib.stream_of(dev))
    torch.cuda.synchronize()
    assert st == 0
    assert torch.equal(c, want)
