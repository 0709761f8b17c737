"""GPU parity of the HIP direction-harmonics kernel and its derivative modes against
the oracle (``direction_harmonics_all`` + float64 autograd)."""
import pytest
import torch

from conftest import assert_rel
from oracle import ictc_basis as B

pytestmark = pytest.mark.gpu


def _dirs(rows, seed, unit=True):
    g = torch.Generator().manual_seed(seed)
    n = torch.randn(rows, 3, generator=g, dtype=torch.float64)
    return torch.nn.functional.normalize(n, dim=-1) if unit else n


@pytest.mark.parametrize("lmax", [0, 1, 2, 3, 4, 6])
def test_values(gpu, lmax):
    from ictc_o3 import direction_harmonics
    n = _dirs(1000, lmax)
    got = direction_harmonics(n.float().to(gpu), lmax)
    expect = B.direction_harmonics_all(n.float().double(), lmax)
    for l, (a, b) in enumerate(zip(got, expect)):
        assert_rel(a, b, what=f"Y_{l}")


@pytest.mark.parametrize("lmax", [2, 3])
def test_first_second_third_derivatives(gpu, lmax):
    from ictc_o3.backends.hip.harmonics import direction_harmonics_packed
    rows = 64
    n = _dirs(rows, 7, unit=False).float()   # the map is a polynomial; any vector is valid
    gen = torch.Generator().manual_seed(8)
    w = torch.randn(rows, (lmax + 1) ** 2, generator=gen)
    v = torch.randn(rows, 3, generator=gen)
    u = torch.randn(rows, 3, generator=gen)

    def chain(fn, nn, ww, vv, uu):
        nn = nn.clone().requires_grad_()
        s = (fn(nn) * ww).sum()
        (d1,) = torch.autograd.grad(s, nn, create_graph=True)
        (d2,) = torch.autograd.grad((d1 * vv).sum(), nn, create_graph=True)
        (d3,) = torch.autograd.grad((d2 * uu).sum(), nn)
        return d1, d2, d3

    got = chain(lambda t: direction_harmonics_packed(t, lmax), *(t.to(gpu) for t in (n, w, v, u)))
    expect = chain(lambda t: B.direction_harmonics_packed(t, lmax), *(t.double() for t in (n, w, v, u)))
    for name, a, b in zip(("first", "second", "third"), got, expect):
        assert_rel(a, b, rtol=2e-5, what=f"{name} derivative")


def test_mixed_derivative_wrt_cotangent(gpu):
    """d/dw of the VJP (the JVP mode) and the Hessian wrt (n, w) of <w, Y(n)>."""
    from ictc_o3.backends.hip.harmonics import direction_harmonics_packed
    rows, lmax = 32, 3
    n = _dirs(rows, 9).float()
    gen = torch.Generator().manual_seed(10)
    w = torch.randn(rows, 16, generator=gen)
    h = torch.randn(rows, 3, generator=gen)

    def mixed(fn, nn, ww, hh):
        nn, ww = nn.clone().requires_grad_(), ww.clone().requires_grad_()
        (d1,) = torch.autograd.grad((fn(nn) * ww).sum(), nn, create_graph=True)
        return torch.autograd.grad((d1 * hh).sum(), (nn, ww))

    got = mixed(lambda t: direction_harmonics_packed(t, lmax), n.to(gpu), w.to(gpu), h.to(gpu))
    expect = mixed(lambda t: B.direction_harmonics_packed(t, lmax), n.double(), w.double(), h.double())
    for a, b in zip(got, expect):
        assert_rel(a, b, rtol=2e-5, what="mixed")


def test_batched_shape_and_empty(gpu):
    from ictc_o3.backends.hip.harmonics import direction_harmonics_packed
    n = _dirs(24, 11).float().reshape(2, 3, 4, 3).to(gpu)
    assert direction_harmonics_packed(n, 3).shape == (2, 3, 4, 16)
    assert direction_harmonics_packed(n[:0], 3).shape == (0, 3, 4, 16)
