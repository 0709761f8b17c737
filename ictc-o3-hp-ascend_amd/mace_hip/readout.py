"""The model's energy readouts as one HIP kernel per derivative order (``ictc_hip_readout``): the
layer readout of the second-to-last layer (bias-free Linear(C, 1), reference
EquivariantScalarReadoutSO3, ``mace_ictc/models/pure_cartesian_ictd_layers.py:46-70``) plus the last
layer's MLP readout (Linear(C, H), normalised SiLU, Linear(H, 1);
``mace_ictc/models/pure_cartesian_ictd_fix.py:1434-1449``), summed per node.

The kernel route serves frozen readout weights (inference and force evaluation); its adjoint is the
kernel's VJP mode.  A further derivative (a graph recorded through the backward) differentiates the
composed formula ``readout_formula`` under autograd, so every order stays available; trainable
weights keep the model's composed layers.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from ictc_o3 import _lib

VALUE, VJP = 0, 1
MAX_CHANNELS, MAX_HIDDEN = 1024, 256


def supported(x: torch.Tensor, y: Optional[torch.Tensor], w_lin: Optional[torch.Tensor], w1: torch.Tensor,
              w2: torch.Tensor) -> bool:
    """fp32 GPU tensors of matching shapes and no gradient to any weight."""
    ws = [w for w in (w_lin, w1, w2) if w is not None]
    if torch.is_grad_enabled() and any(w.requires_grad for w in ws):
        return False
    if x.dim() != 2 or not 1 <= x.shape[1] <= MAX_CHANNELS:
        return False
    c = x.shape[1]
    if w1.dim() != 2 or w1.shape[1] != c or not 1 <= w1.shape[0] <= MAX_HIDDEN or w2.numel() != w1.shape[0]:
        return False
    if (y is None) != (w_lin is None) or (y is not None and (y.shape != x.shape or w_lin.numel() != c)):
        return False
    ts = [x, *ws] + ([y] if y is not None else [])
    return all(t.is_cuda and t.dtype == torch.float32 and t.device == x.device for t in ts)


def readout_formula(y, x, w_lin, w1, w2, scale: float):
    """The composed readouts: w_lin . y + w2 . (scale silu(w1 x)) per node."""
    e = (F.silu(x @ w1.t()) * scale) @ w2.reshape(-1)
    return e if y is None else y @ w_lin.reshape(-1) + e


def _launch(mode, y, x, w_lin, w1, w2, scale, g=None, need=(False, False)):
    n, c = x.shape
    p = _lib.ptr
    atomic = torch.empty(n, device=x.device, dtype=torch.float32) if mode == VALUE else None
    gy = torch.empty_like(x) if mode == VJP and need[0] else None
    gx = torch.empty_like(x) if mode == VJP and need[1] else None
    _lib.check(_lib.lib().ictc_hip_readout(mode, p(y), p(w_lin), p(x), p(w1), p(w2), float(scale), p(g), p(atomic),
                                           p(gy), p(gx), c, w1.shape[0], n, _lib.stream_of(x.device)),
               "ictc_hip_readout")
    return atomic if mode == VALUE else (gy, gx)


class _Readout(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, x, w_lin, w1, w2, scale):
        ctx.scale = scale
        ctx.save_for_backward(y, x, w_lin, w1, w2)
        return _launch(VALUE, y, x, w_lin, w1, w2, scale)

    @staticmethod
    def backward(ctx, g):
        y, x, w_lin, w1, w2 = ctx.saved_tensors
        need_y, need_x = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if g is None or not (need_y or need_x):
            return None, None, None, None, None, None
        if torch.is_grad_enabled():
            # a graph is being recorded through this backward: the composed formula's adjoint
            targets = [t for t, n in ((y, need_y), (x, need_x)) if n]
            e = readout_formula(y, x, w_lin, w1, w2, ctx.scale)
            grads = iter(torch.autograd.grad(e, targets, g, create_graph=True))
            gy = next(grads) if need_y else None
            gx = next(grads) if need_x else None
            return gy, gx, None, None, None, None
        gy, gx = _launch(VJP, y, x, w_lin, w1, w2, ctx.scale, g.contiguous(), (need_y, need_x))
        return gy, gx, None, None, None, None


def readout(y: Optional[torch.Tensor], x: torch.Tensor, w_lin: Optional[torch.Tensor], w1: torch.Tensor,
            w2: torch.Tensor, scale: float) -> torch.Tensor:
    """Atomic energies [N] on the kernel (the caller checks ``supported``); the weights are constants."""
    cont = lambda t: None if t is None else t.contiguous()          # noqa: E731
    return _Readout.apply(cont(y), x.contiguous(), cont(None if w_lin is None else w_lin.detach().reshape(-1)),
                          w1.detach().contiguous(), w2.detach().reshape(-1).contiguous(), float(scale))
