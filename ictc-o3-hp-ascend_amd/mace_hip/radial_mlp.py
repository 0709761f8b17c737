"""Radial MLP of the MACE interaction up to its last Linear, one HIP kernel per derivative order
(``ictc_hip_radial_mlp``): per edge h = silu(s W3 silu(s W2 silu(W1 f))), the reference's ``fc``
without its last layer (``mace_ictc/models/pure_cartesian_ictd_fix.py:1545-1553``, applied at
:1795) with the normalised-SiLU constant s (:610-619) folded into the layer after each activation.

Derivatives.  The adjoint of ``radial_hidden`` is ``_RadialVJP``: the feature gradient and the
three weight gradients from one launch, each only when the autograd engine will use it.  The
adjoint of that is the kernel's VJP_VJP mode (J u as the gradient of the incoming adjoint g, and
the feature and weight gradients of <u, J^T g>), which is force-loss training's double backward.
Anything beyond (a graph recorded through the double backward, or cotangents on the weight
gradients) differentiates the composed formula ``vjp_formula`` under autograd, so every order
stays available.  The kernel takes fp32 GPU tensors with at most 16 basis functions and 64
hidden features (``supported``); the model keeps its composed layers for anything else.
"""
from __future__ import annotations

from typing import Sequence, Tuple

import torch
import torch.nn.functional as F

from ictc_o3 import _lib
from ictc_o3.autograd.adjoint_requirements import required_gradients

WIDTH = 64
MAX_BASIS = 16
VALUE, VJP, VJP_VJP = 0, 1, 2


def supported(f: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor) -> bool:
    """Whether the kernel covers this call (fp32 GPU tensors, 1..16 basis functions, width 64)."""
    if f.dim() != 2 or not 1 <= f.shape[1] <= MAX_BASIS:
        return False
    if tuple(w1.shape) != (WIDTH, f.shape[1]) or tuple(w2.shape) != (WIDTH, WIDTH) or tuple(w3.shape) != (WIDTH, WIDTH):
        return False
    return all(t.is_cuda and t.dtype == torch.float32 and t.device == f.device for t in (f, w1, w2, w3))


def hidden_formula(f, w1, w2, w3, scale: float):
    """The composed layers: silu(s W3 silu(s W2 silu(W1 f)))."""
    a1 = F.silu(f @ w1.t())
    a2 = F.silu(scale * (a1 @ w2.t()))
    return F.silu(scale * (a2 @ w3.t()))


def _dsilu(z, s):
    return s * (1 + z * (1 - s))


def vjp_formula(f, w1, w2, w3, g, scale: float):
    """(J^T g, dW1, dW2, dW3) of ``hidden_formula`` for the adjoint g, written out with
    differentiable ops (the derivative route past the kernel's second order)."""
    z1 = f @ w1.t()
    s1 = torch.sigmoid(z1)
    a1 = z1 * s1
    z2 = scale * (a1 @ w2.t())
    s2 = torch.sigmoid(z2)
    a2 = z2 * s2
    z3 = scale * (a2 @ w3.t())
    c3 = g * _dsilu(z3, torch.sigmoid(z3))
    c2 = scale * (c3 @ w3) * _dsilu(z2, s2)
    c1 = scale * (c2 @ w2) * _dsilu(z1, s1)
    return c1 @ w1, c1.t() @ f, scale * (c2.t() @ a1), scale * (c3.t() @ a2)


def _launch(mode: int, f, w1, w2, w3, scale: float, g=None, u=None, *, hidden=False, grad_feats=False,
            grad_grad=False, grad_weights: Sequence[bool] = (False, False, False)):
    """One ictc_hip_radial_mlp call; returns (hidden, grad_feats, grad_grad, gw1, gw2, gw3) with
    None for what was not asked."""
    lib = _lib.lib()
    edges, basis = f.shape
    dev = f.device
    out_h = torch.empty(edges, WIDTH, device=dev, dtype=torch.float32) if hidden else None
    out_gf = torch.empty(edges, basis, device=dev, dtype=torch.float32) if grad_feats else None
    out_gg = torch.empty(edges, WIDTH, device=dev, dtype=torch.float32) if grad_grad else None
    gws = [torch.empty_like(w) if n else None for w, n in zip((w1, w2, w3), grad_weights)]
    ws, ws_floats = None, 0
    if any(grad_weights):
        ws_floats = int(lib.ictc_hip_radial_mlp_workspace(edges))
        if ws_floats < 0:
            _lib.check(-ws_floats, "ictc_hip_radial_mlp_workspace")
        ws = torch.empty(max(ws_floats, 1), device=dev, dtype=torch.float32)
    p = _lib.ptr
    _lib.check(lib.ictc_hip_radial_mlp(
        mode, p(f), p(w1), p(w2), p(w3), float(scale), p(g), p(u), p(out_h), p(out_gf), p(out_gg), p(ws), ws_floats,
        *(p(t) for t in gws), basis, edges, _lib.stream_of(dev)), "ictc_hip_radial_mlp")
    return (out_h, out_gf, out_gg, *gws)


class _Radial(torch.autograd.Function):
    @staticmethod
    def forward(ctx, f, w1, w2, w3, scale):
        ctx.scale = scale
        ctx.save_for_backward(f, w1, w2, w3)
        return _launch(VALUE, f, w1, w2, w3, scale, hidden=True)[0]

    @staticmethod
    def backward(ctx, g):
        f, w1, w2, w3 = ctx.saved_tensors
        need = required_gradients((f, w1, w2, w3), ctx.needs_input_grad[:4])
        if g is None or not any(need):
            return None, None, None, None, None
        return (*_RadialVJP.apply(f, w1, w2, w3, g.contiguous(), ctx.scale, need), None)


class _RadialVJP(torch.autograd.Function):
    """(J^T g, dW1, dW2, dW3) for the adjoint g of the hidden features; the entries not in
    ``need`` are None."""

    @staticmethod
    def forward(ctx, f, w1, w2, w3, g, scale, need):
        ctx.scale = scale
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(f, w1, w2, w3, g)
        _, gf, _, gw1, gw2, gw3 = _launch(VJP, f, w1, w2, w3, scale, g, grad_feats=need[0], grad_weights=need[1:4])
        return gf, gw1, gw2, gw3

    @staticmethod
    def backward(ctx, ggf, gg1, gg2, gg3):
        f, w1, w2, w3, g = ctx.saved_tensors
        need = required_gradients((f, w1, w2, w3, g), ctx.needs_input_grad[:5])
        if not any(need) or all(c is None for c in (ggf, gg1, gg2, gg3)):
            return (None,) * 7
        if gg1 is None and gg2 is None and gg3 is None and not torch.is_grad_enabled():
            _, d_f, d_g, d_w1, d_w2, d_w3 = _launch(VJP_VJP, f, w1, w2, w3, ctx.scale, g, ggf.contiguous(),
                                                    grad_feats=need[0], grad_grad=need[4], grad_weights=need[1:4])
            return d_f, d_w1, d_w2, d_w3, d_g, None, None
        return (*_formula_adjoint((f, w1, w2, w3, g), need, (ggf, gg1, gg2, gg3), ctx.scale), None, None)


def _formula_adjoint(inputs: Tuple[torch.Tensor, ...], need, cotangents, scale: float):
    """Adjoint of ``vjp_formula`` in the needed inputs, recorded when grad mode is on."""
    create = torch.is_grad_enabled()
    with torch.enable_grad():
        ins = inputs if create else tuple(t.detach().requires_grad_(bool(n)) for t, n in zip(inputs, need))
        outs = vjp_formula(*ins, scale)
        pairs = [(o, c) for o, c in zip(outs, cotangents) if c is not None and o.requires_grad]
        targets = [t for t, n in zip(ins, need) if n]
        if not pairs:
            return tuple(None for _ in need)
        grads = torch.autograd.grad([o for o, _ in pairs], targets, [c for _, c in pairs], create_graph=create,
                                    allow_unused=True)
    it = iter(grads)
    return tuple(next(it) if n else None for n in need)


def radial_hidden(f: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor, scale: float) -> torch.Tensor:
    """h [E, 64] for edge features f [E, B]: on the kernel when ``supported``, else the composed layers."""
    if supported(f, w1, w2, w3):
        return _Radial.apply(f.contiguous(), w1.contiguous(), w2.contiguous(), w3.contiguous(), float(scale))
    return hidden_formula(f, w1, w2, w3, float(scale))
