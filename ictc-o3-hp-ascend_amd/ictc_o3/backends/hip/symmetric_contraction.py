"""Symmetric contraction on the HIP kernels (correlation <= 3, species-selected weights).

    out[n, c, l, m] = sum_p W[s_n, p, c] * chain_p(x[n, c, :])_m

The kernels evaluate the U-tensor columns as coupling chains with shared pair
prefixes (see ictc_o3/basis/symmetric_u.py).  Gradients:

* node features: the ``ictc_hip_sc_backward`` kernel;
* weights: the map is linear in W, so dW[s] is the sum over the nodes of species s
  of the per-node chain features <u, chain_p(x)> (``ictc_hip_sc_weight_features``),
  reduced by species as one GEMM with the species one-hot matrix.

The backward is itself a differentiable Function (second derivatives, as force
training needs).  With cotangents (a, B) of (dx, dW):
  d/d go = J(x) a + forward(x, B)
  d/d x  = H_go(x) a + vjp(x, B, go)
  d/d W  = species-sum of <go, d chain_p(x)[a]>
through the directional kernels (``ictc_hip_sc_jvp``, ``_hvp``, ``_weight_features_jvp``);
third derivatives are not provided.
"""
from __future__ import annotations

import ctypes

import torch

from ... import _lib
from ...autograd.adjoint_requirements import required_gradients


class ContractionPlan:
    def __init__(self, lmax: int, target_lmax: int, correlation: int, channels: int, num_elements: int):
        self.lmax, self.target_lmax, self.correlation = int(lmax), int(target_lmax), int(correlation)
        self.channels, self.num_elements = int(channels), int(num_elements)
        ktot = _lib.lib().ictc_hip_sc_weight_columns(self.lmax, self.target_lmax, self.correlation)
        if ktot < 0:
            raise ValueError(f"symmetric contraction (lmax={lmax}, target_lmax={target_lmax}, "
                             f"correlation={correlation}) is not compiled into libictc_hip.so")
        self.ktot = ktot
        self.in_width = self.channels * (self.lmax + 1) ** 2
        self.out_width = self.channels * (self.target_lmax + 1) ** 2


def _forward_raw(plan: ContractionPlan, x, species, w):
    out = torch.empty(x.shape[0], plan.out_width, device=x.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_sc_forward(
        plan.lmax, plan.target_lmax, plan.correlation, plan.channels, x.data_ptr(), species.data_ptr(),
        w.data_ptr(), plan.num_elements, out.data_ptr(), x.shape[0], _lib.stream_of(x.device)),
        "ictc_hip_sc_forward")
    return out


def _vjp_raw(plan: ContractionPlan, x, species, w, go):
    dx = torch.empty(x.shape[0], plan.in_width, device=x.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_sc_backward(
        plan.lmax, plan.target_lmax, plan.correlation, plan.channels, x.data_ptr(), species.data_ptr(),
        w.data_ptr(), plan.num_elements, go.data_ptr(), dx.data_ptr(), x.shape[0],
        _lib.stream_of(x.device)), "ictc_hip_sc_backward")
    return dx


def _species_sum(plan: ContractionPlan, species, phi):
    """sum of phi [N, KTOT, C] over the nodes of each species -> [S, KTOT, C], as one GEMM with the
    species one-hot matrix (a few species rows: atomic adds into them would all contend)."""
    n = phi.shape[0]
    onehot = torch.nn.functional.one_hot(species, plan.num_elements).to(torch.float32)
    return torch.mm(onehot.t(), phi.reshape(n, plan.ktot * plan.channels)).reshape(
        plan.num_elements, plan.ktot, plan.channels)


def _weight_grad(plan: ContractionPlan, x, species, go):
    """dW[s,p,c] = sum_{n: s_n = s} <go[n,c], chain_p(x[n,c])>."""
    phi = torch.empty(x.shape[0], plan.ktot, plan.channels, device=x.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_sc_weight_features(
        plan.lmax, plan.target_lmax, plan.correlation, plan.channels, x.data_ptr(), species.data_ptr(),
        plan.num_elements, go.data_ptr(), phi.data_ptr(), x.shape[0], _lib.stream_of(x.device)),
        "ictc_hip_sc_weight_features")
    return _species_sum(plan, species, phi)


def _jvp_raw(plan: ContractionPlan, x, species, w, t):
    out = torch.empty(x.shape[0], plan.out_width, device=x.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_sc_jvp(
        plan.lmax, plan.target_lmax, plan.correlation, plan.channels, x.data_ptr(), species.data_ptr(),
        w.data_ptr(), plan.num_elements, t.data_ptr(), out.data_ptr(), x.shape[0], _lib.stream_of(x.device)),
        "ictc_hip_sc_jvp")
    return out


def _hvp_raw(plan: ContractionPlan, x, species, w, go, t):
    out = torch.empty(x.shape[0], plan.in_width, device=x.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_sc_hvp(
        plan.lmax, plan.target_lmax, plan.correlation, plan.channels, x.data_ptr(), species.data_ptr(),
        w.data_ptr(), plan.num_elements, go.data_ptr(), t.data_ptr(), out.data_ptr(), x.shape[0],
        _lib.stream_of(x.device)), "ictc_hip_sc_hvp")
    return out


def _weight_grad_jvp(plan: ContractionPlan, x, species, go, t):
    """sum over the nodes of each species of <go[n,c], d chain_p(x[n,c])[t[n,c]]>."""
    phi = torch.empty(x.shape[0], plan.ktot, plan.channels, device=x.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_sc_weight_features_jvp(
        plan.lmax, plan.target_lmax, plan.correlation, plan.channels, x.data_ptr(), species.data_ptr(),
        plan.num_elements, go.data_ptr(), t.data_ptr(), phi.data_ptr(), x.shape[0], _lib.stream_of(x.device)),
        "ictc_hip_sc_weight_features_jvp")
    return _species_sum(plan, species, phi)


def _add(a, b):
    return b if a is None else (a if b is None else a + b)


class _Forward(torch.autograd.Function):
    @staticmethod
    def forward(ctx, plan, x, species, w):
        ctx.plan = plan
        ctx.save_for_backward(x, species, w)
        return _forward_raw(plan, x, species, w)

    @staticmethod
    def backward(ctx, go):
        x, species, w = ctx.saved_tensors
        nx, nw = required_gradients((x, w), (ctx.needs_input_grad[1], ctx.needs_input_grad[3]))
        if go is None or not (nx or nw):
            return None, None, None, None
        go = go.contiguous()
        if torch.is_grad_enabled():
            dx, dw = _Backward.apply(ctx.plan, x, species, w, go, nx, nw)
        else:
            dx = _vjp_raw(ctx.plan, x, species, w, go) if nx else None
            dw = _weight_grad(ctx.plan, x, species, go) if nw else None
        return None, dx, None, dw


class _Backward(torch.autograd.Function):
    """(x, W, go) -> (J(x)^T go, species-summed <go, chain(x)>), differentiable once more."""

    @staticmethod
    def forward(ctx, plan, x, species, w, go, nx, nw):
        ctx.plan = plan
        ctx.save_for_backward(x, species, w, go)
        dx = _vjp_raw(plan, x, species, w, go) if nx else None
        dw = _weight_grad(plan, x, species, go) if nw else None
        return dx, dw

    @staticmethod
    def backward(ctx, a, b):
        if torch.is_grad_enabled():
            raise NotImplementedError("third derivatives through the symmetric contraction are not provided")
        plan = ctx.plan
        x, species, w, go = ctx.saved_tensors
        need_x, need_w, need_go = ctx.needs_input_grad[1], ctx.needs_input_grad[3], ctx.needs_input_grad[4]
        a = None if a is None else a.contiguous()
        b = None if b is None else b.contiguous()
        gx = gw = ggo = None
        if need_go:
            ggo = _add(_jvp_raw(plan, x, species, w, a) if a is not None else None,
                       _forward_raw(plan, x, species, b) if b is not None else None)
        if need_x:
            gx = _add(_hvp_raw(plan, x, species, w, go, a) if a is not None else None,
                      _vjp_raw(plan, x, species, b, go) if b is not None else None)
        if need_w and a is not None:
            gw = _weight_grad_jvp(plan, x, species, go, a)
        return None, gx, None, gw, ggo, None, None


def symmetric_contraction(plan: ContractionPlan, x: torch.Tensor, species: torch.Tensor,
                          weights: torch.Tensor) -> torch.Tensor:
    """x [N, C*(L+1)^2] (mul_ir), species int64 [N], weights [S, KTOT, C] -> [N, C*(T+1)^2]."""
    return _Forward.apply(plan, x.contiguous(), species.contiguous(), weights.contiguous())
