"""GPU parity of the HIP symmetric contraction against the oracle's restatement of
``_forward_selected_elements`` on the same U tensors (float64), through the C ABI.

Covers every target degree of the cfg-3 and cfg-4 configurations, lower correlation
orders, channel counts that do not fill a wave, feature VJP, weight gradients,
species selection by one-hot attributes, validation, and full-size (65,536-node)
properties: equivariance under a rotation and linearity in the weights.
"""
import pytest
import torch

from conftest import assert_rel
from oracle import ictc_basis as B
from oracle.symmetric_contraction import SymmetricContractionOracle

pytestmark = pytest.mark.gpu


def _module(ref, device):
    """The pure-ICTC module: its weights address the coupling chains the oracle's U holds."""
    from ictc_o3 import configure_symmetric_contraction
    from ictc_o3.ops.symmetric_contraction import ICTDPureUSymmetricContractionSO3
    mod = ICTDPureUSymmetricContractionSO3(num_elements=ref.S, lmax=ref.lmax, target_lmax=ref.target_lmax,
                                           channels=ref.C, correlation=ref.correlation).to(device)
    configure_symmetric_contraction(mod)
    with torch.no_grad():
        for l, con in enumerate(mod.contractions):
            con.weights_max.copy_(ref.weights[(l, ref.correlation)].float())
            for i, nu in enumerate(range(ref.correlation - 1, 0, -1)):
                con.weights[i].copy_(ref.weights[(l, nu)].float())
    return mod


def _inputs(ref, nodes, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(nodes, ref.C * (ref.lmax + 1) ** 2, generator=g) * 0.7
    species = torch.randint(0, ref.S, (nodes,), generator=g)
    return x, species


CASES = [(3, 1, 3, 128), (3, 3, 3, 64), (3, 0, 3, 128), (2, 2, 3, 48), (1, 1, 2, 96), (3, 2, 1, 32),
         (0, 0, 3, 64)]


@pytest.mark.parametrize("lmax,target,corr,c", CASES)
def test_forward_vjp_and_weight_grad(gpu, lmax, target, corr, c):
    ref = SymmetricContractionOracle(5, c, lmax, target, corr, seed=lmax * 10 + target)
    mod = _module(ref, gpu)
    x, species = _inputs(ref, 23, 3)
    go = torch.randn(23, c * (target + 1) ** 2, generator=torch.Generator().manual_seed(4))
    xd = x.to(gpu).requires_grad_()
    out = mod(xd, node_type_idx=species.to(gpu))
    xc = x.double().requires_grad_()
    wref = {k: v.clone().requires_grad_() for k, v in ref.weights.items()}
    expect = ref.forward(xc, species, wref)
    assert_rel(out, expect, what="sc forward")
    params = [p for con in mod.contractions for p in con.columns()]
    grads = torch.autograd.grad(out, [xd, *params], go.to(gpu))
    keys = [(l, nu) for l in range(target + 1) for nu in range(corr, 0, -1)]
    egrads = torch.autograd.grad(expect, [xc, *[wref[k] for k in keys]], go.double())
    assert_rel(grads[0], egrads[0], what="sc grad features")
    for k, a, b in zip(keys, grads[1:], egrads[1:]):
        assert_rel(a, b, what=f"sc grad weights {k}")


def test_one_hot_attributes_and_validation(gpu):
    ref = SymmetricContractionOracle(4, 64, 2, 1, 3, seed=7)
    mod = _module(ref, gpu)
    x, species = _inputs(ref, 9, 8)
    attrs = torch.nn.functional.one_hot(species, 4).float()
    out = mod(x.to(gpu), attrs.to(gpu))
    assert_rel(out, ref.forward(x.double(), species), what="one-hot species")
    with pytest.raises(ValueError):
        mod(x.to(gpu), node_type_idx=torch.full((9,), 4, device=gpu))
    with pytest.raises(ValueError):
        mod(x[:, :-1].to(gpu), node_type_idx=species.to(gpu))


def test_full_size_equivariance_and_weight_linearity(gpu):
    """cfg 3: C=128, lmax 3 -> 0e+1o, correlation 3, 65,536 nodes, 10 species."""
    ref = SymmetricContractionOracle(10, 128, 3, 1, 3, seed=11)
    mod = _module(ref, gpu)
    n = 65536
    gen = torch.Generator(device=gpu).manual_seed(12)
    x = torch.randn(n, 128 * 16, device=gpu, generator=gen) * 0.5
    species = torch.randint(0, 10, (n,), device=gpu, generator=gen)
    out = mod(x, node_type_idx=species)
    # rotation: each degree block [C, 2l+1] -> block @ D_l^T
    om = torch.tensor([0.7, -0.2, 1.3], dtype=torch.float64)
    ds = [B.wigner_d(l, om).float().to(gpu) for l in range(4)]

    def rotate(t, lmax):
        parts, off = [], 0
        for l in range(lmax + 1):
            w = 128 * (2 * l + 1)
            parts.append((t[:, off:off + w].reshape(-1, 128, 2 * l + 1) @ ds[l].T).reshape(-1, w))
            off += w
        return torch.cat(parts, -1)
    out_rot = mod(rotate(x, 3), node_type_idx=species)
    assert_rel(out_rot, rotate(out, 1), rtol=2e-5, what="equivariance")
    # linearity in the weights: f(W1 + W2) = f(W1) + f(W2)
    from ictc_o3.backends.hip.symmetric_contraction import symmetric_contraction
    w1 = mod.weight_table().detach()
    w2 = torch.randn_like(w1)
    f = lambda w: symmetric_contraction(mod.plan, x, species, w)  # noqa: E731
    assert_rel(f(w1 + w2), f(w1) + f(w2), rtol=2e-5, what="weight linearity")


@pytest.mark.parametrize("lmax,target,corr,c,with_weights",
                         [(3, 1, 3, 128, True), (3, 3, 3, 64, True), (3, 0, 3, 32, False), (2, 2, 2, 48, True),
                          (1, 0, 3, 96, False)])
def test_second_derivatives(gpu, lmax, target, corr, c, with_weights):
    """Double backward: d/d(x, go, W) of <a, dx> + <B, dW> with dx, dW from create_graph=True
    (with_weights=False is the force-training pattern: only dx is differentiated)."""
    ref = SymmetricContractionOracle(4, c, lmax, target, corr, seed=lmax * 7 + target + corr)
    mod = _module(ref, gpu)
    n = 19
    x, species = _inputs(ref, n, 21)
    g = torch.Generator().manual_seed(22)
    go = torch.randn(n, c * (target + 1) ** 2, generator=g)
    a = torch.randn(n, c * (lmax + 1) ** 2, generator=g)
    keys = [(l, nu) for l in range(target + 1) for nu in range(corr, 0, -1)]
    bs = [torch.randn(ref.weights[k].shape, generator=g, dtype=torch.float64) for k in keys]

    params = [p for con in mod.contractions for p in con.columns()]
    xd, god = x.to(gpu).requires_grad_(), go.to(gpu).requires_grad_()
    out = mod(xd, node_type_idx=species.to(gpu))
    wrt = [xd, *params] if with_weights else [xd]
    first = torch.autograd.grad(out, wrt, god, create_graph=True)
    loss = (first[0] * a.to(gpu)).sum()
    if with_weights:
        loss = loss + sum((d * b.float().to(gpu)).sum() for d, b in zip(first[1:], bs))
    got = torch.autograd.grad(loss, [xd, god, *params])

    xc, goc = x.double().requires_grad_(), go.double().requires_grad_()
    wref = {k: v.clone().requires_grad_() for k, v in ref.weights.items()}
    expect = ref.forward(xc, species, wref)
    ewrt = [xc, *[wref[k] for k in keys]] if with_weights else [xc]
    efirst = torch.autograd.grad(expect, ewrt, goc, create_graph=True)
    eloss = (efirst[0] * a.double()).sum()
    if with_weights:
        eloss = eloss + sum((d * b).sum() for d, b in zip(efirst[1:], bs))
    want = torch.autograd.grad(eloss, [xc, goc, *[wref[k] for k in keys]])
    names = ["x", "grad_out"] + [f"W{k}" for k in keys]
    for name, u, v in zip(names, got, want):
        assert_rel(u, v, what=f"sc second derivative wrt {name}")
