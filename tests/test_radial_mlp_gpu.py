"""Radial MLP kernel (ictc_hip_radial_mlp) against the composed layers in float64 on the CPU:
values, first derivatives (features and weights), the double backward of force training
(J u and the feature and weight gradients of <u, J^T g>), a third derivative through the
composed route, the autograd wiring of mace_hip.radial_mlp, and run-to-run determinism.
Reference: mace_ictc/models/pure_cartesian_ictd_fix.py:1545-1553 (fc up to its last Linear),
:610-619 (normalised SiLU)."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

SCALE = 1.6791767923989418
DEV = torch.device("cuda", 0)


def _inputs(edges, basis, seed):
    g = torch.Generator().manual_seed(seed)
    f = torch.randn(edges, basis, generator=g, dtype=torch.float64)
    w1 = torch.randn(64, basis, generator=g, dtype=torch.float64) / math.sqrt(basis)
    w2 = torch.randn(64, 64, generator=g, dtype=torch.float64) / 8
    w3 = torch.randn(64, 64, generator=g, dtype=torch.float64) / 8
    gh = torch.randn(edges, 64, generator=g, dtype=torch.float64)
    u = torch.randn(edges, basis, generator=g, dtype=torch.float64)
    return f, w1, w2, w3, gh, u


def _ref_hidden(f, w1, w2, w3):
    from mace_hip.radial_mlp import hidden_formula
    return hidden_formula(f, w1, w2, w3, SCALE)


def _gpu(*ts):
    return [t.to(DEV, torch.float32).contiguous() for t in ts]


def _close(got, want, tol=2e-5):
    want = want.to(torch.float64)
    err = (got.double().cpu() - want).abs().max().item() if want.numel() else 0.0
    scale = max(want.abs().max().item() if want.numel() else 0.0, 1.0)
    assert err <= tol * scale, f"max error {err:.3e} against scale {scale:.3e}"


CASES = [(0, 8), (1, 8), (15, 8), (17, 5), (64, 16), (1000, 8), (4099, 1), (6151, 8)]


@pytest.mark.parametrize("edges,basis", CASES)
def test_value_and_first_derivatives(edges, basis):
    from mace_hip.radial_mlp import VALUE, VJP, _launch
    f, w1, w2, w3, gh, _ = _inputs(edges, basis, 10 + edges)
    fr, w1r, w2r, w3r = [t.clone().requires_grad_() for t in (f, w1, w2, w3)]
    h = _ref_hidden(fr, w1r, w2r, w3r)
    want = torch.autograd.grad(h, (fr, w1r, w2r, w3r), gh)
    F_, W1, W2, W3, G = _gpu(f, w1, w2, w3, gh)
    out = _launch(VALUE, F_, W1, W2, W3, SCALE, hidden=True)[0]
    torch.cuda.synchronize()
    _close(out, h.detach())
    _, gf, _, g1, g2, g3 = _launch(VJP, F_, W1, W2, W3, SCALE, G, grad_feats=True, grad_weights=(True, True, True))
    torch.cuda.synchronize()
    for got, ref in zip((gf, g1, g2, g3), want):
        _close(got, ref, 2e-5 if edges < 5000 else 5e-5)


@pytest.mark.parametrize("edges,basis", CASES)
def test_double_backward(edges, basis):
    """<u, J^T g>: its gradients in g (= J u), f and the weights."""
    from mace_hip.radial_mlp import VJP_VJP, _launch
    f, w1, w2, w3, gh, u = _inputs(edges, basis, 20 + edges)
    fr, w1r, w2r, w3r, ghr = [t.clone().requires_grad_() for t in (f, w1, w2, w3, gh)]
    h = _ref_hidden(fr, w1r, w2r, w3r)
    gf, = torch.autograd.grad(h, fr, ghr, create_graph=True)
    want = torch.autograd.grad(gf, (fr, w1r, w2r, w3r, ghr), u, allow_unused=True)
    want = [torch.zeros_like(t) if w is None else w for w, t in zip(want, (f, w1, w2, w3, gh))]
    F_, W1, W2, W3, G, U = _gpu(f, w1, w2, w3, gh, u)
    _, df, dg, d1, d2, d3 = _launch(VJP_VJP, F_, W1, W2, W3, SCALE, G, U, grad_feats=True, grad_grad=True,
                                    grad_weights=(True, True, True))
    torch.cuda.synchronize()
    for got, ref in zip((df, d1, d2, d3, dg), want):
        _close(got, ref, 2e-5 if edges < 5000 else 5e-5)


def test_partial_outputs_and_determinism():
    """Each output alone equals the same output of a full call; weight gradients are
    bit-identical from call to call."""
    from mace_hip.radial_mlp import VJP, VJP_VJP, _launch
    F_, W1, W2, W3, G, U = _gpu(*_inputs(20_011, 8, 5))
    full = _launch(VJP_VJP, F_, W1, W2, W3, SCALE, G, U, grad_feats=True, grad_grad=True,
                   grad_weights=(True, True, True))
    only_w2 = _launch(VJP_VJP, F_, W1, W2, W3, SCALE, G, U, grad_weights=(False, True, False))
    only_gg = _launch(VJP_VJP, F_, W1, W2, W3, SCALE, G, U, grad_grad=True)
    again = _launch(VJP_VJP, F_, W1, W2, W3, SCALE, G, U, grad_feats=True, grad_grad=True,
                    grad_weights=(True, True, True))
    first = _launch(VJP, F_, W1, W2, W3, SCALE, G, grad_feats=True, grad_weights=(True, True, True))
    first2 = _launch(VJP, F_, W1, W2, W3, SCALE, G, grad_weights=(True, False, True))
    torch.cuda.synchronize()
    assert torch.equal(only_w2[4], full[4]) and torch.equal(only_gg[2], full[2])
    for a, b in zip(full[1:], again[1:]):
        assert torch.equal(a, b)
    assert torch.equal(first2[3], first[3]) and torch.equal(first2[5], first[5])


def test_autograd_force_training_pattern():
    """h -> gates -> energy; forces by a create_graph gradient in the features; a loss on both
    back to the weights (the model's force-loss step), against float64 autograd."""
    from mace_hip.radial_mlp import radial_hidden
    f, w1, w2, w3, _, _ = _inputs(3001, 8, 7)
    w4 = torch.randn(96, 64, generator=torch.Generator().manual_seed(3), dtype=torch.float64) / 8
    coef = torch.randn(3001, 96, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    target = torch.randn(3001, 8, generator=torch.Generator().manual_seed(5), dtype=torch.float64)

    def step(ins, hidden):
        fr, a, b, c, d, k, tg = ins
        h = hidden(fr, a, b, c)
        energy = ((h @ d.t()) ** 2 * k).sum() * 1e-3
        gf, = torch.autograd.grad(energy, fr, create_graph=True)
        loss = energy + ((gf - tg) ** 2).sum()
        return torch.autograd.grad(loss, (a, b, c, d))

    ref = step([f.clone().requires_grad_(), *[t.clone().requires_grad_() for t in (w1, w2, w3, w4)], coef, target],
               _ref_hidden)
    gpu_ins = [t.clone().requires_grad_() for t in _gpu(f, w1, w2, w3, w4)]
    coef_g, target_g = _gpu(coef, target)
    got = step([*gpu_ins, coef_g, target_g], lambda fr, a, b, c: radial_hidden(fr, a, b, c, SCALE))
    for a, b in zip(got, ref):
        _close(a, b, 1e-4)


def test_third_derivative_through_composed_route():
    """A graph recorded through the double backward (create_graph twice) differentiates the
    composed formula: d/dw2 of <v, d<u, J^T g>/dg>, against float64."""
    from mace_hip.radial_mlp import radial_hidden
    f, w1, w2, w3, gh, u = _inputs(257, 8, 9)
    v = torch.randn(257, 64, generator=torch.Generator().manual_seed(11), dtype=torch.float64)

    def third(ins, hidden):
        fr, a, b, c, g, uu, vv = ins
        h = hidden(fr, a, b, c)
        gf, = torch.autograd.grad(h, fr, g, create_graph=True)
        dg, = torch.autograd.grad(gf, g, uu, create_graph=True)
        return torch.autograd.grad((dg * vv).sum(), b)[0]

    ref = third([t.clone().requires_grad_() for t in (f, w1, w2, w3, gh)] + [u, v], _ref_hidden)
    got = third([t.clone().requires_grad_() for t in _gpu(f, w1, w2, w3, gh)] + _gpu(u, v),
                lambda fr, a, b, c: radial_hidden(fr, a, b, c, SCALE))
    _close(got, ref, 1e-4)
