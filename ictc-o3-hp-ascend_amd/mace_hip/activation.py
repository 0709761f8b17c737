"""SiLU for the radial MLP with a one-pass double backward.

Force training differentiates the radial MLP's first-order backward ``y = g * silu'(x)`` once
more.  ``silu`` keeps every derivative differentiable (the first-order backward is the
Function ``_SiLUGrad``); when the backward of ``_SiLUGrad`` runs without recording a further
graph (the last backward of a training step) on fp32 GPU tensors, its two outputs come from one
pass of ``ictc_hip_silu_second`` instead of the ~nine elementwise passes of the composed formula.
The reference ships the same derivative forms as modes of its fp32 elementwise kernel
(``ascendc/elementwise.py:7-97``).
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from ictc_o3 import _lib


def _silu_prime(x: torch.Tensor) -> torch.Tensor:
    s = torch.sigmoid(x)
    return s * (1 + x * (1 - s))


def _silu_second(x: torch.Tensor) -> torch.Tensor:
    s = torch.sigmoid(x)
    return s * (1 - s) * (2 + x * (1 - 2 * s))


class _SiLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return F.silu(x)

    @staticmethod
    def backward(ctx, g):
        x, = ctx.saved_tensors
        return _SiLUGrad.apply(x, g)


class _SiLUGrad(torch.autograd.Function):
    """y = g * silu'(x)."""

    @staticmethod
    def forward(ctx, x, g):
        ctx.save_for_backward(x, g)
        return torch.ops.aten.silu_backward(g, x)

    @staticmethod
    def backward(ctx, h):
        x, g = ctx.saved_tensors
        need_x, need_g = ctx.needs_input_grad
        if h is None or not (need_x or need_g):
            return None, None
        fused = (not torch.is_grad_enabled() and x.is_cuda and x.dtype == torch.float32 and h.dtype == torch.float32
                 and g.dtype == torch.float32)
        if not fused:
            dx = h * g * _silu_second(x) if need_x else None
            dg = h * _silu_prime(x) if need_g else None
            return dx, dg
        x, g, h = x.contiguous(), g.contiguous(), h.contiguous()
        dx = torch.empty_like(x) if need_x else None
        dg = torch.empty_like(x) if need_g else None
        _lib.check(_lib.lib().ictc_hip_silu_second(
            x.data_ptr(), g.data_ptr(), h.data_ptr(), None if dg is None else dg.data_ptr(),
            None if dx is None else dx.data_ptr(), x.numel(), _lib.stream_of(x.device)), "ictc_hip_silu_second")
        return dx, dg


def silu(x: torch.Tensor) -> torch.Tensor:
    return _SiLU.apply(x)
