"""GPU parity of the element-conditioned linear map (``ictc_hip_species_linear``, the MACE
self connection on a frozen weight) through the C ABI, against the per-node float64 product
W[s_n] x[n] on the CPU: both modes at channel counts with and without float4 rows, every
derivative order through the mutually adjoint Functions, and the model's SpeciesLinear, which
takes the kernel for a frozen weight and the composed product otherwise."""
import pytest
import torch

from conftest import assert_rel

pytestmark = pytest.mark.gpu


def _case(c, nodes, species, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(species, c, c, generator=g)
    x = torch.randn(nodes, c, generator=g)
    s = torch.randint(0, species, (nodes,), generator=g)
    return w, x, s


@pytest.mark.parametrize("c,nodes,species", [(128, 1000, 10), (70, 333, 3), (8, 5, 1), (4, 64, 2)])
def test_modes_match_per_node_products(gpu, c, nodes, species):
    from mace_hip.species_linear import APPLY, TRANSPOSE, _launch
    w, x, s = _case(c, nodes, species, c + nodes)
    wd = w.double()[s]                                   # [N, C, C]
    apply_ref = torch.einsum("noi,ni->no", wd, x.double())
    trans_ref = torch.einsum("noi,no->ni", wd, x.double())
    dev = [t.to(gpu) for t in (w, x, s)]
    assert_rel(_launch(APPLY, dev[0], dev[1], dev[2]), apply_ref, what="apply")
    assert_rel(_launch(TRANSPOSE, dev[0], dev[1], dev[2]), trans_ref, what="transpose")


def test_derivatives_alternate_modes(gpu):
    """y = W[s] x with W constant: dy/dx^T g = W[s]^T g, and the derivative of that in g is W[s] h."""
    from mace_hip.species_linear import species_linear
    w, x, s = _case(128, 257, 10, 7)
    gen = torch.Generator().manual_seed(8)
    g, h = torch.randn(257, 128, generator=gen), torch.randn(257, 128, generator=gen)
    wd = w.double()[s]
    xd = x.to(gpu).requires_grad_()
    y = species_linear(xd, w.to(gpu), s.to(gpu))
    gd = g.to(gpu).requires_grad_()
    (dx,) = torch.autograd.grad(y, xd, gd, create_graph=True)
    assert_rel(dx, torch.einsum("noi,no->ni", wd, g.double()), what="first derivative")
    (dg,) = torch.autograd.grad(dx, gd, h.to(gpu))
    assert_rel(dg, torch.einsum("noi,ni->no", wd, h.double()), what="second derivative")


def test_model_layer_routes(gpu):
    """SpeciesLinear: the kernel for a frozen weight equals the composed product (and the weight
    gradient route stays composed when the weight trains)."""
    from mace_hip.model import SpeciesLinear
    from mace_hip import species_linear as sl
    w, x, s = _case(128, 500, 10, 3)
    layer = SpeciesLinear(10, 128).to(gpu)
    with torch.no_grad():
        layer.weight.copy_(w)
    xg, sg = x.to(gpu), s.to(gpu)
    composed = layer(xg, sg)                              # the weight requires a gradient
    assert not sl.supported(xg, layer.weight, sg)
    layer.requires_grad_(False)
    assert sl.supported(xg, layer.weight, sg)
    assert_rel(layer(xg, sg), composed.detach(), what="kernel vs composed")
