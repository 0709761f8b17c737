"""Direction harmonics on the HIP kernel with analytic derivatives to third order.

Y(n) is a polynomial, so each derivative contraction is a kernel mode and each
mode's adjoint is another mode (see include/ictc_hip.h):

    Y     : d<gY, Y>        -> VJP(n; gY)
    VJP   : d<h, VJP(n;u)>  -> n: HVP(n; u, h)      u: JVP(n; h)
    JVP   : d<k, JVP(n;t)>  -> n: HVP(n; k, t)      t: VJP(n; k)
    HVP   : d<h, HVP(n;u,t)> -> n: T3(n; u, t, h)   u: JVP2(n; t, h)   t: HVP(n; u, h)
    JVP2  : d<k, JVP2(n;t,s)> -> n: T3(n; k, t, s)  t: HVP(n; k, s)    s: HVP(n; k, t)
    T3    : t: T3(n; u, h, s)   s: T3(n; u, t, h)   (n, u: fourth order, not provided)

Force training needs VJP (forces) and its adjoint (HVP, JVP); the rest lets
third-order probes run without an eager fallback.
"""
from __future__ import annotations

import torch

from ... import _lib
from ...autograd.adjoint_requirements import required_gradients

VALUE, VJP, JVP, HVP, JVP2, T3 = range(6)
MAX_LMAX = 6


def _raw(mode: int, n: torch.Tensor, lmax: int, u=None, t=None, s=None) -> torch.Tensor:
    rows = n.shape[0]
    width = 3 if mode in (VJP, HVP, T3) else (lmax + 1) ** 2
    out = torch.empty(rows, width, device=n.device, dtype=torch.float32)
    args = [None if v is None else v.contiguous() for v in (u, t, s)]
    _lib.check(_lib.lib().ictc_hip_direction_harmonics(
        lmax, mode, n.data_ptr(), *[_lib.ptr(a) for a in args], out.data_ptr(), rows,
        _lib.stream_of(n.device)), "ictc_hip_direction_harmonics")
    return out


def _add(a, b):
    if b is None:
        return a
    return b if a is None else a + b


class _Value(torch.autograd.Function):
    @staticmethod
    def forward(ctx, n, lmax):
        ctx.lmax = lmax
        ctx.save_for_backward(n)
        return _raw(VALUE, n, lmax)

    @staticmethod
    def backward(ctx, gy):
        (n,) = ctx.saved_tensors
        if gy is None or not ctx.needs_input_grad[0]:
            return None, None
        if not torch.is_grad_enabled():       # nothing recorded: skip the autograd Function
            return _raw(VJP, n, ctx.lmax, u=gy), None
        return _Vjp.apply(n, gy, ctx.lmax), None


class _Vjp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, n, u, lmax):
        ctx.lmax = lmax
        ctx.save_for_backward(n, u)
        return _raw(VJP, n, lmax, u=u)

    @staticmethod
    def backward(ctx, h):
        n, u = ctx.saved_tensors
        need = required_gradients((n, u), ctx.needs_input_grad[:2])
        if h is None:
            return None, None, None
        gn = _Hvp.apply(n, u, h, ctx.lmax) if need[0] else None
        gu = _Jvp.apply(n, h, ctx.lmax) if need[1] else None
        return gn, gu, None


class _Jvp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, n, t, lmax):
        ctx.lmax = lmax
        ctx.save_for_backward(n, t)
        return _raw(JVP, n, lmax, t=t)

    @staticmethod
    def backward(ctx, k):
        n, t = ctx.saved_tensors
        need = required_gradients((n, t), ctx.needs_input_grad[:2])
        if k is None:
            return None, None, None
        gn = _Hvp.apply(n, k, t, ctx.lmax) if need[0] else None
        gt = _Vjp.apply(n, k, ctx.lmax) if need[1] else None
        return gn, gt, None


class _Hvp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, n, u, t, lmax):
        ctx.lmax = lmax
        ctx.save_for_backward(n, u, t)
        return _raw(HVP, n, lmax, u=u, t=t)

    @staticmethod
    def backward(ctx, h):
        n, u, t = ctx.saved_tensors
        need = required_gradients((n, u, t), ctx.needs_input_grad[:3])
        if h is None:
            return None, None, None, None
        gn = _T3.apply(n, u, t, h, ctx.lmax) if need[0] else None
        gu = _Jvp2.apply(n, t, h, ctx.lmax) if need[1] else None
        gt = _Hvp.apply(n, u, h, ctx.lmax) if need[2] else None
        return gn, gu, gt, None


class _Jvp2(torch.autograd.Function):
    @staticmethod
    def forward(ctx, n, t, s, lmax):
        ctx.lmax = lmax
        ctx.save_for_backward(n, t, s)
        return _raw(JVP2, n, lmax, t=t, s=s)

    @staticmethod
    def backward(ctx, k):
        n, t, s = ctx.saved_tensors
        need = required_gradients((n, t, s), ctx.needs_input_grad[:3])
        if k is None:
            return None, None, None, None
        gn = _T3.apply(n, k, t, s, ctx.lmax) if need[0] else None
        gt = _Hvp.apply(n, k, s, ctx.lmax) if need[1] else None
        gs = _Hvp.apply(n, k, t, ctx.lmax) if need[2] else None
        return gn, gt, gs, None


class _T3(torch.autograd.Function):
    @staticmethod
    def forward(ctx, n, u, t, s, lmax):
        ctx.lmax = lmax
        ctx.save_for_backward(n, u, t, s)
        return _raw(T3, n, lmax, u=u, t=t, s=s)

    @staticmethod
    def backward(ctx, h):
        n, u, t, s = ctx.saved_tensors
        need = required_gradients((n, u, t, s), ctx.needs_input_grad[:4])
        if h is None:
            return None, None, None, None, None
        if need[0] or need[1]:
            raise NotImplementedError("fourth-order derivatives of direction harmonics are not provided")
        gt = _T3.apply(n, u, h, s, ctx.lmax) if need[2] else None
        gs = _T3.apply(n, u, t, h, ctx.lmax) if need[3] else None
        return None, None, gt, gs, None


def direction_harmonics_packed(directions: torch.Tensor, lmax: int) -> torch.Tensor:
    """Y_0 | Y_1 | ... | Y_lmax of unit directions [..., 3] -> [..., (lmax+1)^2] (ICTC basis,
    component normalisation; reference ictd_irreps.py:1113-1168)."""
    if not 0 <= int(lmax) <= MAX_LMAX:
        raise ValueError(f"direction harmonics are compiled for lmax <= {MAX_LMAX}")
    if directions.shape[-1] != 3:
        raise ValueError("directions must have a trailing dimension of 3")
    lead = directions.shape[:-1]
    flat = directions.reshape(-1, 3).contiguous()
    out = _Value.apply(flat, int(lmax))
    return out.reshape(*lead, (int(lmax) + 1) ** 2)
