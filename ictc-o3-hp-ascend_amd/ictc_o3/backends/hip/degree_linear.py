"""Per-degree channel linear on the fp32-MFMA kernels of ``csrc/linear_api.hip``: the
path-preserving message linear of the MACE interaction (reference
``mace_ictc/models/pure_cartesian_ictd_fix.py:629-661``), read straight from the message
kernels' packed ir_mul output and written in the mul_ir node layout.

    y[n, l-block][o, m] = alpha * sum_{k, c} W_l[o, k C + c] * x[n, l-block][k, m, c]

x rows hold, per degree l, ``counts[l]`` path blocks of [2l+1][C]; y rows hold, per degree,
[O][2l+1]; ``weights[l]`` is [O, counts[l] C].  The map is bilinear in (x, W): its input
adjoint is the second kernel (``ictc_hip_degree_linear_input_grad``), whose own adjoints are
the forward kernel again, and every weight adjoint alpha * gY_l^T X_l is a third kernel
(``ictc_hip_degree_linear_weight_grad``: split-row MFMA partials summed in order) that reads
both layouts in place; its own adjoints are the forward and input-adjoint kernels with the
weight cotangent as weights, so derivatives of any order stay on these kernels.
"""
from __future__ import annotations

import ctypes
from typing import List, Sequence

import torch

from ... import _lib
from ...autograd.adjoint_requirements import required_gradients


class DegreeLinearPlan:
    def __init__(self, counts: Sequence[int], channels: int, out_channels: int):
        self.counts = [int(c) for c in counts]
        self.lmax = len(self.counts) - 1
        if not 0 <= self.lmax < 8:
            raise ValueError("degree linear supports degrees 0..7")
        self.channels, self.out_channels = int(channels), int(out_channels)
        self.desc = _lib.DegreeLinearDesc()
        self.desc.lmax, self.desc.channels, self.desc.out_channels = self.lmax, self.channels, self.out_channels
        for l, c in enumerate(self.counts):
            self.desc.counts[l] = c
        self.in_width = sum(c * (2 * l + 1) * self.channels for l, c in enumerate(self.counts))
        self.out_width = self.out_channels * (self.lmax + 1) ** 2
        self._transposed = None
        self._ws_floats = {}   # (x layout, nodes) -> weight-adjoint workspace floats

    def x_rows(self, x: torch.Tensor, l: int) -> torch.Tensor:
        """Packed x -> the degree-l rows [N (2l+1), counts[l] C] (column k C + c)."""
        d, k, c = 2 * l + 1, self.counts[l], self.channels
        off = sum(self.counts[j] * (2 * j + 1) * c for j in range(l))
        blk = x[:, off:off + k * d * c].reshape(x.shape[0], k, d, c)
        return blk.transpose(1, 2).reshape(x.shape[0] * d, k * c)

    def transposed(self) -> "DegreeLinearPlan":
        """The plan of the transposed map (channels and out_channels swapped; one block per degree)."""
        if self._transposed is None:
            self._transposed = DegreeLinearPlan(self.counts, self.out_channels, self.channels)
            self._transposed._transposed = self
        return self._transposed

    def mul_ir_rows(self, x: torch.Tensor, l: int) -> torch.Tensor:
        """mul_ir x with one channel block per degree -> the degree-l rows [N (2l+1), C]."""
        d, c = 2 * l + 1, self.channels
        blk = x[:, c * l * l:c * (l + 1) ** 2].reshape(x.shape[0], c, d)
        return blk.transpose(1, 2).reshape(x.shape[0] * d, c)

    def y_rows(self, y: torch.Tensor, l: int) -> torch.Tensor:
        """mul_ir y -> the degree-l rows [N (2l+1), O]."""
        d, o = 2 * l + 1, self.out_channels
        blk = y[:, o * l * l:o * (l + 1) ** 2].reshape(y.shape[0], o, d)
        return blk.transpose(1, 2).reshape(y.shape[0] * d, o)


def _pointers(weights: List[torch.Tensor]):
    arr = (ctypes.c_void_p * len(weights))()
    for i, w in enumerate(weights):
        arr[i] = w.data_ptr() if w.numel() else None
    return arr


def _forward_raw(plan: DegreeLinearPlan, x, weights, alpha):
    y = torch.empty(x.shape[0], plan.out_width, device=x.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_degree_linear_forward(
        ctypes.byref(plan.desc), x.data_ptr() if x.numel() else None, _pointers(weights), float(alpha),
        y.data_ptr() if y.numel() else None, x.shape[0], _lib.stream_of(x.device)), "ictc_hip_degree_linear_forward")
    return y


def _input_grad_raw(plan: DegreeLinearPlan, gy, weights, alpha):
    gx = torch.empty(gy.shape[0], plan.in_width, device=gy.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_degree_linear_input_grad(
        ctypes.byref(plan.desc), gy.data_ptr() if gy.numel() else None, _pointers(weights), float(alpha),
        gx.data_ptr() if gx.numel() else None, gy.shape[0], _lib.stream_of(gy.device)),
        "ictc_hip_degree_linear_input_grad")
    return gx


_IR_MUL, _MUL_IR = 0, 1   # x layouts of the weight adjoint (the forward's, the mul_ir map's)


def _weight_grad_raw(plan: DegreeLinearPlan, layout: int, gy, x, alpha, need):
    """[alpha * gY_l^T X_l if need[l] and counts[l] else None] in one kernel pair."""
    nodes = gy.shape[0]
    grads = [torch.empty(plan.out_channels, k * plan.channels, device=gy.device, dtype=torch.float32)
             if n and k else None for n, k in zip(need, plan.counts)]
    if not any(g is not None for g in grads):
        return grads
    key = (layout, nodes)
    floats = plan._ws_floats.get(key)
    if floats is None:
        floats = _lib.lib().ictc_hip_degree_linear_weight_grad_workspace(ctypes.byref(plan.desc), layout, nodes)
        _lib.check(-int(floats) if floats < 0 else 0, "ictc_hip_degree_linear_weight_grad_workspace")
        plan._ws_floats[key] = floats
    ws = torch.empty(max(int(floats), 1), device=gy.device, dtype=torch.float32)
    ptrs = (ctypes.c_void_p * (plan.lmax + 1))()
    for l, g in enumerate(grads):
        ptrs[l] = g.data_ptr() if g is not None and g.numel() else None
    _lib.check(_lib.lib().ictc_hip_degree_linear_weight_grad(
        ctypes.byref(plan.desc), layout, gy.data_ptr() if gy.numel() else None, x.data_ptr() if x.numel() else None,
        float(alpha), ws.data_ptr(), int(floats), ptrs, nodes, _lib.stream_of(gy.device)),
        "ictc_hip_degree_linear_weight_grad")
    return grads


class _WeightGrad(torch.autograd.Function):
    """The weight adjoint as a differentiable map of (gy, x): <gW, V> = alpha sum gy . (X V^T) rows,
    so d/dgy is the forward map of x with weights V and d/dx the input adjoint of gy with weights V
    (for the mul_ir layout: the mul_ir map and its transposed map)."""

    @staticmethod
    def forward(ctx, plan, alpha, layout, need, gy, x):
        ctx.plan, ctx.alpha, ctx.layout, ctx.need = plan, alpha, layout, need
        ctx.save_for_backward(gy, x)
        grads = _weight_grad_raw(plan, layout, gy, x, alpha, need)
        ctx.live = [g is not None for g in grads]
        return tuple(g for g in grads if g is not None)

    @staticmethod
    def backward(ctx, *gbar):
        gy, x = ctx.saved_tensors
        plan, alpha = ctx.plan, ctx.alpha
        it = iter(gbar)
        vs = []
        for l, live in enumerate(ctx.live):
            v = next(it) if live else None
            k = plan.counts[l] * plan.channels
            vs.append(v.contiguous() if v is not None else
                      torch.zeros(plan.out_channels, k, device=gy.device, dtype=torch.float32))
        dgy = dx = None
        if ctx.layout == _IR_MUL:
            if ctx.needs_input_grad[4]:
                dgy = _Forward.apply(plan, alpha, x, *vs)
            if ctx.needs_input_grad[5]:
                dx = _InputGrad.apply(plan, alpha, gy, *vs)
        else:
            if ctx.needs_input_grad[4]:
                dgy = _MulIr.apply(plan, alpha, x, *vs)
            if ctx.needs_input_grad[5]:
                dx = _MulIr.apply(plan.transposed(), alpha, gy, *[v.t().contiguous() for v in vs])
        return None, None, None, None, dgy, dx


def _weight_grads(plan: DegreeLinearPlan, gy, x, alpha, need, layout: int = _IR_MUL):
    """alpha * gY_l^T X_l per degree (None where not needed), differentiable."""
    need = tuple(bool(n) and plan.counts[l] > 0 for l, n in enumerate(need))
    if not any(need):
        return [None] * len(need)
    live = iter(_WeightGrad.apply(plan, float(alpha), layout, need, gy.contiguous(), x.contiguous()))
    return [next(live) if n else None for n in need]


class _Forward(torch.autograd.Function):
    @staticmethod
    def forward(ctx, plan, alpha, x, *weights):
        ctx.plan, ctx.alpha = plan, alpha
        ctx.save_for_backward(x, *weights)
        return _forward_raw(plan, x, list(weights), alpha)

    @staticmethod
    def backward(ctx, gy):
        x, *weights = ctx.saved_tensors
        need = required_gradients((x, *weights), ctx.needs_input_grad[2:])
        if gy is None or not any(need):
            return (None, None, None) + (None,) * len(weights)
        gy = gy.contiguous()
        gx = _InputGrad.apply(ctx.plan, ctx.alpha, gy, *weights) if need[0] else None
        return (None, None, gx, *_weight_grads(ctx.plan, gy, x, ctx.alpha, need[1:]))


class _InputGrad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, plan, alpha, gy, *weights):
        ctx.plan, ctx.alpha = plan, alpha
        ctx.save_for_backward(gy, *weights)
        return _input_grad_raw(plan, gy, list(weights), alpha)

    @staticmethod
    def backward(ctx, z):
        gy, *weights = ctx.saved_tensors
        need = required_gradients((gy, *weights), ctx.needs_input_grad[2:])
        if z is None or not any(need):
            return (None, None, None) + (None,) * len(weights)
        z = z.contiguous()
        ggy = _Forward.apply(ctx.plan, ctx.alpha, z, *weights) if need[0] else None
        return (None, None, ggy, *_weight_grads(ctx.plan, gy, z, ctx.alpha, need[1:]))


def _check_weights(weights, plan, device):
    if len(weights) != plan.lmax + 1:
        raise ValueError("one weight per degree is required")
    for l, w in enumerate(weights):
        if w.shape != (plan.out_channels, plan.counts[l] * plan.channels):
            raise ValueError(f"weight of degree {l} must have shape [O, counts[l] C]")
        if w.dtype != torch.float32 or w.device != device:
            raise ValueError("weights must be float32 on the features' device")


def _mul_ir_raw(plan: "DegreeLinearPlan", x, weights, alpha, transposed: bool = False):
    """alpha W_l x per degree, or alpha W_l^T x with W_l [plan.channels, plan.out_channels]."""
    y = torch.empty(x.shape[0], plan.out_width, device=x.device, dtype=torch.float32)
    name = "ictc_hip_degree_linear_mul_ir_transposed" if transposed else "ictc_hip_degree_linear_mul_ir"
    _lib.check(getattr(_lib.lib(), name)(
        ctypes.byref(plan.desc), x.data_ptr() if x.numel() else None, _pointers(weights), float(alpha),
        y.data_ptr() if y.numel() else None, x.shape[0], _lib.stream_of(x.device)), name)
    return y


class _MulIrT(torch.autograd.Function):
    """y = alpha W_l^T x per degree for the plan with channels and out_channels swapped, reading
    W_l [O, C] (the o3.Linear weight) as it is stored: the input adjoint of _MulIr without a
    transposed weight copy.  Adjoints: in x the _MulIr map of the cotangent, in W the weight
    adjoint with gY = x and X = the cotangent."""

    @staticmethod
    def forward(ctx, plan_t, alpha, x, *weights):
        ctx.plan_t, ctx.alpha = plan_t, alpha
        ctx.save_for_backward(x, *weights)
        return _mul_ir_raw(plan_t, x, list(weights), alpha, transposed=True)

    @staticmethod
    def backward(ctx, z):
        x, *weights = ctx.saved_tensors
        need = required_gradients((x, *weights), ctx.needs_input_grad[2:])
        if z is None or not any(need):
            return (None, None, None) + (None,) * len(weights)
        z = z.contiguous()
        plan = ctx.plan_t.transposed()
        gx = _MulIr.apply(plan, ctx.alpha, z, *weights) if need[0] else None
        return (None, None, gx, *_weight_grads(plan, x, z, ctx.alpha, need[1:], _MUL_IR))


class _MulIr(torch.autograd.Function):
    """y = alpha W_l x per degree, mul_ir in and out (one channel block per degree).  Its input
    adjoint is the same map with the transposed weights (plan.transposed); the weight adjoint is
    alpha gY_l^T X_l on the [N (2l+1), channels] rows of both; so every derivative order stays on
    this kernel and dense products."""

    @staticmethod
    def forward(ctx, plan, alpha, x, *weights):
        ctx.plan, ctx.alpha = plan, alpha
        ctx.save_for_backward(x, *weights)
        return _mul_ir_raw(plan, x, list(weights), alpha)

    @staticmethod
    def backward(ctx, gy):
        x, *weights = ctx.saved_tensors
        need = required_gradients((x, *weights), ctx.needs_input_grad[2:])
        if gy is None or not any(need):
            return (None, None, None) + (None,) * len(weights)
        gy = gy.contiguous()
        plan = ctx.plan
        gx = None
        if need[0]:
            gx = _MulIrT.apply(plan.transposed(), ctx.alpha, gy, *weights)
        return (None, None, gx, *_weight_grads(plan, gy, x, ctx.alpha, need[1:], _MUL_IR))


def degree_linear_mul_ir(x: torch.Tensor, weights: Sequence[torch.Tensor], plan: "DegreeLinearPlan",
                         alpha: float = 1.0) -> torch.Tensor:
    """Per-degree channel linear on mul_ir rows in and out: x [N, C (L+1)^2] (per degree
    [C][2l+1]), weights[l] [O, C] -> alpha W_l x per degree, [N, O (L+1)^2] (the e3nn o3.Linear of
    the MACE product block); the plan must have one channel block per degree."""
    if any(k != 1 for k in plan.counts):
        raise ValueError("the mul_ir map takes one channel block per degree")
    if x.ndim != 2 or x.shape[1] != plan.in_width:
        raise ValueError("features must have shape [N, C (L+1)^2]")
    _check_weights(weights, plan, x.device)
    if x.dtype != torch.float32 or not x.is_cuda:
        raise ValueError("features must be float32 on a ROCm GPU")
    return _MulIr.apply(plan, float(alpha), x.contiguous(), *[w.contiguous() for w in weights])


def degree_linear_adjoint(y: torch.Tensor, weights: Sequence[torch.Tensor], plan: DegreeLinearPlan,
                          alpha: float = 1.0) -> torch.Tensor:
    """The adjoint map of ``degree_linear`` in its first argument, as an operator of its own:
    y [N, plan.out_width] (mul_ir, per degree [O][2l+1]) -> alpha * W_l^T y per degree,
    [N, plan.in_width] (per degree counts[l] blocks of [2l+1][C], ir_mul).  With counts all 1 and
    the weights transposed this is a per-degree C x C channel linear from mul_ir to ir_mul (the
    MACE interaction's linear_up feeding the message kernels)."""
    if y.ndim != 2 or y.shape[1] != plan.out_width:
        raise ValueError("features must have shape [N, O (L+1)^2]")
    _check_weights(weights, plan, y.device)
    if y.dtype != torch.float32 or not y.is_cuda:
        raise ValueError("features must be float32 on a ROCm GPU")
    return _InputGrad.apply(plan, float(alpha), y.contiguous(), *[w.contiguous() for w in weights])


def degree_linear(x: torch.Tensor, weights: Sequence[torch.Tensor], plan: DegreeLinearPlan,
                  alpha: float = 1.0) -> torch.Tensor:
    """x [N, plan.in_width] (packed per-degree path blocks [count][2l+1][C]), weights[l]
    [O, counts[l] C] -> alpha * per-degree linear [N, O (L+1)^2] (mul_ir)."""
    if x.ndim != 2 or x.shape[1] != plan.in_width:
        raise ValueError("features must have shape [N, sum_l counts[l] (2l+1) C]")
    _check_weights(weights, plan, x.device)
    if x.dtype != torch.float32 or not x.is_cuda:
        raise ValueError("features must be float32 on a ROCm GPU")
    return _Forward.apply(plan, float(alpha), x.contiguous(), *[w.contiguous() for w in weights])
