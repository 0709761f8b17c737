"""Element-conditioned linear map on the scalar block (the interaction's self connection,
reference ``mace_ictc/models/pure_cartesian_ictd_fix.py:335-390``): out[n] = W[s_n] x[n], one HIP
kernel (``ictc_hip_species_linear``) instead of a product with every species' weight and a gather.

The kernel route serves a frozen weight (no gradient to W: inference and force evaluation).  The
map is then linear in x with a constant W, so its adjoint is the same kernel in its transposed mode
and the adjoint's adjoint the forward: ``_Apply`` and ``_Transpose`` call each other from their
backward, and every derivative order stays on the kernel.  A weight that requires a gradient
(training) keeps the composed route in ``mace_hip.model.SpeciesLinear``.
"""
from __future__ import annotations

import torch

from ictc_o3 import _lib

APPLY, TRANSPOSE = 0, 1


def supported(x: torch.Tensor, weight: torch.Tensor, species: torch.Tensor) -> bool:
    """fp32 GPU tensors, x [N, C], weight [S, C, C], species [N] int64, and no gradient to W."""
    if weight.requires_grad and torch.is_grad_enabled():
        return False
    if x.dim() != 2 or weight.dim() != 3 or weight.shape[1:] != (x.shape[1], x.shape[1]):
        return False
    if species.dim() != 1 or species.shape[0] != x.shape[0] or species.dtype != torch.int64:
        return False
    return (x.is_cuda and x.dtype == torch.float32 and weight.dtype == torch.float32
            and weight.device == x.device and species.device == x.device)


def _launch(mode: int, weight: torch.Tensor, x: torch.Tensor, species: torch.Tensor) -> torch.Tensor:
    out = torch.empty_like(x)
    p = _lib.ptr
    _lib.check(_lib.lib().ictc_hip_species_linear(mode, p(weight), p(x), p(species), p(out), x.shape[1],
                                                   weight.shape[0], x.shape[0], _lib.stream_of(x.device)),
               "ictc_hip_species_linear")
    return out


class _Apply(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, species):
        ctx.save_for_backward(weight, species)
        return _launch(APPLY, weight, x, species)

    @staticmethod
    def backward(ctx, g):
        weight, species = ctx.saved_tensors
        return _Transpose.apply(g.contiguous(), weight, species), None, None


class _Transpose(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, species):
        ctx.save_for_backward(weight, species)
        return _launch(TRANSPOSE, weight, x, species)

    @staticmethod
    def backward(ctx, g):
        weight, species = ctx.saved_tensors
        return _Apply.apply(g.contiguous(), weight, species), None, None


def species_linear(x: torch.Tensor, weight: torch.Tensor, species: torch.Tensor) -> torch.Tensor:
    """W[s_n] x[n] on the kernel (the caller checks ``supported``); W is treated as a constant."""
    return _Apply.apply(x.contiguous(), weight.detach().contiguous(), species.contiguous())
