"""Edge directions and radial embedding of the MACE interaction on one HIP kernel per derivative
order (``ictc_hip_edge_embedding``).

From the edge vectors v [E, 3] (r = |v|):

    n     = v / max(r, 1e-8)                                   (the harmonics' input)
    emb_b = sqrt(2 / r_max) sin(b pi r / r_max) / max(r, 1e-12) * u(r / r_max)   (b = 1..B)

with u the polynomial cutoff envelope, as reference ``pure_cartesian_ictd_fix.py:2935-2936`` and
``radial_basis.py:11-92`` (Bessel basis, no sqrt(B) factor) compute them with library ops.  The
map f(v) = (n, emb) is differentiated analytically; each derivative contraction is a kernel mode
and each mode's adjoint another mode:

    VALUE : d<(gn, ge), f>           -> VJP(v; gn, ge)
    VJP   : d<h, VJP(v; g)>          -> v: HVP(v; g, h)        g: JVP(v; h)
    JVP   : d<k, JVP(v; t)>          -> v: HVP(v; k, t)        t: VJP(v; k)
    HVP   : third order, not provided

Force training needs VALUE, VJP (forces) and the VJP's adjoint (HVP, JVP).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from ictc_o3 import _lib
from ictc_o3.autograd.adjoint_requirements import required_gradients

VALUE, VJP, JVP, HVP = range(4)


class EmbeddingSpec:
    """Radial basis parameters (hashable; passed through the autograd Functions)."""

    def __init__(self, r_max: float, num_basis: int, cutoff_p: int):
        self.r_max, self.num_basis, self.cutoff_p = float(r_max), int(num_basis), int(cutoff_p)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _raw(mode: int, v: torch.Tensor, spec: EmbeddingSpec, gn=None, ge=None, t=None, want_n=True, want_e=True):
    rows = v.shape[0]
    gn, ge, t = (None if x is None else x.contiguous() for x in (gn, ge, t))
    out_n = torch.empty(rows, 3, device=v.device, dtype=torch.float32) if want_n else None
    out_e = torch.empty(rows, spec.num_basis, device=v.device, dtype=torch.float32) if want_e else None
    _lib.check(_lib.lib().ictc_hip_edge_embedding(
        mode, v.data_ptr(), _ptr(gn), _ptr(ge), _ptr(t), _ptr(out_n), _ptr(out_e), spec.num_basis, spec.cutoff_p,
        spec.r_max, rows, _lib.stream_of(v.device)), "ictc_hip_edge_embedding")
    return out_n, out_e


def _vjp_raw(v, spec, gn, ge):
    return _raw(VJP, v, spec, gn=gn, ge=ge, want_e=False)[0]


class _Value(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v, spec):
        ctx.spec = spec
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(v)
        return _raw(VALUE, v, spec)

    @staticmethod
    def backward(ctx, gn, ge):
        (v,) = ctx.saved_tensors
        if (gn is None and ge is None) or not ctx.needs_input_grad[0]:
            return None, None
        if not torch.is_grad_enabled():       # nothing recorded: skip the autograd Function
            return _vjp_raw(v, ctx.spec, gn, ge), None
        return _Vjp.apply(v, gn, ge, ctx.spec), None


class _Vjp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v, gn, ge, spec):
        ctx.spec = spec
        ctx.has = (gn is not None, ge is not None)
        ctx.save_for_backward(v, gn, ge)
        return _vjp_raw(v, spec, gn, ge)

    @staticmethod
    def backward(ctx, h):
        v, gn, ge = ctx.saved_tensors
        if h is None:
            return None, None, None, None
        need = required_gradients((v, gn, ge), ctx.needs_input_grad[:3])
        gv = _Hvp.apply(v, gn, ge, h, ctx.spec) if need[0] else None
        ggn = gge = None
        if need[1] or need[2]:
            ggn, gge = _Jvp.apply(v, h, ctx.spec, need[1], need[2])
        return gv, ggn if need[1] else None, gge if need[2] else None, None


class _Jvp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v, t, spec, want_n=True, want_e=True):
        ctx.spec = spec
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(v, t)
        out_n, out_e = _raw(JVP, v, spec, t=t, want_n=want_n, want_e=want_e)
        empty = v.new_empty(0)
        outs = (out_n if want_n else empty, out_e if want_e else empty)
        for o, w in zip(outs, (want_n, want_e)):
            if not w:
                ctx.mark_non_differentiable(o)
        return outs

    @staticmethod
    def backward(ctx, kn, ke):
        v, t = ctx.saved_tensors
        kn = kn if kn is not None and kn.numel() else None
        ke = ke if ke is not None and ke.numel() else None
        if kn is None and ke is None:
            return None, None, None, None, None
        need = required_gradients((v, t), ctx.needs_input_grad[:2])
        gv = _Hvp.apply(v, kn, ke, t, ctx.spec) if need[0] else None
        gt = _Vjp.apply(v, kn, ke, ctx.spec) if need[1] else None
        return gv, gt, None, None, None


class _Hvp(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v, gn, ge, t, spec):
        return _raw(HVP, v, spec, gn=gn, ge=ge, t=t, want_e=False)[0]

    @staticmethod
    def backward(ctx, h):
        raise NotImplementedError("third-order derivatives of the edge embedding are not provided")


def edge_embedding(vectors: torch.Tensor, *, r_max: float, num_basis: int = 8,
                   cutoff_p: int = 5) -> Tuple[torch.Tensor, torch.Tensor]:
    """Edge vectors [E, 3] (float32, on the GPU) -> (unit directions [E, 3], Bessel x cutoff
    embedding [E, num_basis]), differentiable to second order."""
    if vectors.ndim != 2 or vectors.shape[1] != 3 or vectors.dtype != torch.float32 or not vectors.is_cuda:
        raise ValueError("edge vectors must be a float32 [E, 3] GPU tensor")
    return _Value.apply(vectors.contiguous(), EmbeddingSpec(r_max, num_basis, cutoff_p))
