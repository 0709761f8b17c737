"""Shared channel GEMMs with live first and higher derivatives (reference
``ictc_o3/backends/ascend/linear.py:8-52``, native route ``ascendc/linear.py:12-136``).

``channel_linear`` and ``species_channel_linear`` keep the reference's shapes, validation and
bias rules.  Their arithmetic is ``mm``: a differentiable product whose every derivative is
again ``mm`` (any order, as force-loss training needs), with adjoints the autograd engine will
not run skipped.

Routing of ``mm`` (measured on MI355X at the MACE cfg-4 shapes, E = 105,634 edges):

* plain products call rocBLAS explicitly through ``ictc_hip_sgemm`` with the operands' own
  storage order passed as transpose flags (no copies, no process-wide library preference);
  an edge-sized left operand against a weight (``x @ W^T``, and ``g @ W`` in the backward, where
  the weight-sized right operand is copied column-major) runs with a column-major right operand:
  0.485 vs 0.571 ms for ``[E,64]@[64,2944]`` on hipBLASLt, 0.372 vs 0.39-0.41 ms for
  ``[E,2944]@[2944,64]``; a short reduction (K < 16, ``[E,8]@[8,64]``) keeps a row-major right
  operand (25 vs 35 us);
* a weight gradient ``g^T x`` reduces over ~10^5 rows into a small output, which one GEMM
  covers with a handful of output tiles (0.3 ms for 0.9 GFLOP); it is split into row blocks
  multiplied as one batched GEMM (torch.bmm on its default library) and summed: 2,048-row
  blocks, 8,192 for outputs of 2^17+ entries; outputs of at most 4,096 entries stay one GEMM.
"""
from __future__ import annotations

import torch

from ... import _lib
from ...autograd.adjoint_requirements import required_gradients
from .runtime import require_gpu_fp32
from .species import validate_species

SPLIT_ROWS = 2048          # rows per partial product
SPLIT_MIN_RATIO = 16       # split when K >= 16 * max(M, N) ...
SPLIT_MAX_OUTPUT = 1 << 18  # ... and the output has at most this many entries
SPLIT_ROWS_LARGE = 8192
SPLIT_LARGE_OUTPUT = 1 << 17
SPLIT_SINGLE_GEMM_OUTPUT = 4096
ROW_MAJOR_RIGHT_BELOW_K = 16
TALL_ROWS = 8192           # edge-sized left operand ...
TALL_MAX_RIGHT = 1 << 22   # ... against a weight-sized right operand: column-major right operand


def _storage(t: torch.Tensor):
    """(tensor, transposed, leading dimension) describing a 2-D operand for ictc_hip_sgemm:
    row-major [r, c] with row stride >= c, or the transpose of a row-major [c, r]."""
    r, c = t.shape
    s0, s1 = t.stride()
    if (s1 == 1 or c <= 1) and s0 >= max(c, 1):
        return t, 0, max(s0, 1)
    if (s0 == 1 or r <= 1) and s1 >= max(r, 1):
        return t, 1, max(s1, 1)
    t = t.contiguous()
    return t, 0, max(c, 1)


def _sgemm(a: torch.Tensor, b: torch.Tensor, *, row_major_b: bool = False) -> torch.Tensor:
    """a [M, K] @ b [K, N] on rocBLAS (ictc_hip_sgemm), fp32, one device."""
    m, k = a.shape
    n = b.shape[1]
    out = torch.empty(m, n, device=a.device, dtype=torch.float32)
    if m == 0 or n == 0:
        return out
    if k == 0:
        return out.zero_()
    if row_major_b:
        b = b.contiguous()
    a, ta, lda = _storage(a)
    b, tb, ldb = _storage(b)
    _lib.check(_lib.lib().ictc_hip_sgemm(ta, tb, m, n, k, 1.0, a.data_ptr(), lda, b.data_ptr(), ldb, 0.0,
                                         out.data_ptr(), n, _lib.stream_of(a.device)), "ictc_hip_sgemm")
    return out


def sgemm_into(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out = a [M, K] @ b [K, N] on rocBLAS with no autograd record, into a caller-owned row-major
    out (a row slice of a larger matrix is fine); the operands' storage orders are passed as is."""
    m, k = a.shape
    n = b.shape[1]
    if out.shape != (m, n) or out.stride(1) != 1 or out.dtype != torch.float32:
        raise ValueError("sgemm_into needs a row-major float32 output of shape [M, N]")
    if m == 0 or n == 0:
        return out
    if k == 0:
        return out.zero_()
    a, ta, lda = _storage(a)
    b, tb, ldb = _storage(b)
    _lib.check(_lib.lib().ictc_hip_sgemm(ta, tb, m, n, k, 1.0, a.data_ptr(), lda, b.data_ptr(), ldb, 0.0,
                                         out.data_ptr(), max(out.stride(0), 1), _lib.stream_of(a.device)),
               "ictc_hip_sgemm")
    return out


def _plain(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    if not a.is_cuda:
        return a @ b
    m, k = a.shape
    if k < ROW_MAJOR_RIGHT_BELOW_K:
        return _sgemm(a, b, row_major_b=True)
    if m >= TALL_ROWS and k * b.shape[1] <= TALL_MAX_RIGHT and b.stride(0) != 1:
        b = b.t().contiguous().t()             # weight-sized copy: column-major right operand
    return _sgemm(a, b)


def _product(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    m, k = a.shape
    n = b.shape[1]
    rows = SPLIT_ROWS_LARGE if m * n >= SPLIT_LARGE_OUTPUT else SPLIT_ROWS
    blocks = k // rows
    if (blocks < 2 or k < SPLIT_MIN_RATIO * max(m, n) or m * n > SPLIT_MAX_OUTPUT
            or m * n <= SPLIT_SINGLE_GEMM_OUTPUT):
        return _plain(a, b)
    main = blocks * rows
    at = a.t()                                   # [K, M]: contiguous when a is a transposed activation
    left = at[:main].reshape(blocks, rows, m).transpose(1, 2)      # [blocks, M, rows]
    right = b[:main].reshape(blocks, rows, n)                       # [blocks, rows, N]
    out = torch.bmm(left, right).sum(0)
    if main < k:
        out = out + _plain(a[:, main:], b[main:])
    return out


class _MM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return _product(a, b)

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        need_a, need_b = required_gradients((a, b), ctx.needs_input_grad)
        prod = mm if torch.is_grad_enabled() else _product   # nothing recorded: no Function needed
        ga = prod(g, b.t()) if need_a else None
        gb = prod(a.t(), g) if need_b else None
        return ga, gb


def mm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a [M, K] @ b [K, N], differentiable to any order."""
    return _MM.apply(a, b)


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x [R, in] @ weight[out, in]^T (no bias)."""
    return mm(x, weight.t())


def channel_linear(features, weight, bias=None):
    """features [..., I, M], weight [O, I], optional bias [O] (scalar blocks only) -> [..., O, M]."""
    require_gpu_fp32(features, weight, *(() if bias is None else (bias,)))
    if features.ndim < 2 or weight.ndim != 2 or features.shape[-2] != weight.shape[1]:
        raise ValueError("Expected features [...,I,M] and weight [O,I]")
    if bias is not None and (features.shape[-1] != 1 or bias.shape != (weight.shape[0],)):
        raise ValueError("Bias is allowed only for scalar angular blocks with shape [O]")
    angular = features.movedim(-2, -1)                             # [..., M, I]
    lead = angular.shape[:-1]
    rows = angular.reshape(-1, weight.shape[1])
    result = linear(rows, weight)
    if bias is not None:
        result = result + bias
    return result.reshape(*lead, weight.shape[0]).movedim(-1, -2)


def species_channel_linear(features, weight, species, bias=None):
    """features [N, I, M], weight [S, O, I], integer species [N], optional bias [S, O] (scalar
    blocks only) -> [N, O, M] with out[n] = weight[species[n]] @ features[n]: one GEMM against
    every species' weights, then each node's own block is selected (no [N, O, I] temporary and
    no host sorting; every weight and mixed derivative stays live)."""
    require_gpu_fp32(features, weight, *(() if bias is None else (bias,)))
    if (features.ndim != 3 or weight.ndim != 3 or features.shape[1] != weight.shape[2]
            or species.shape != (features.shape[0],) or species.device != features.device
            or species.dtype not in (torch.int32, torch.int64) or weight.shape[0] < 1):
        raise ValueError("Expected features [N,I,M], weight [S,O,I] and integer species [N]")
    validate_species(species, weight.shape[0])
    if bias is not None and (features.shape[-1] != 1 or bias.shape != weight.shape[:2]):
        raise ValueError("Bias is allowed only for scalar angular blocks with shape [S,O]")
    n, i, m = features.shape
    s, o = weight.shape[:2]
    rows = features.transpose(1, 2).reshape(n * m, i)
    every = linear(rows, weight.reshape(s * o, i)).reshape(n, m, s, o)
    index = species.to(torch.int64).view(n, 1, 1, 1).expand(n, m, 1, o)
    picked = every.gather(2, index).squeeze(2)                      # [N, M, O]
    if bias is not None:
        # one_hot(species) @ bias: the bias gradient is a GEMM (fixed order), not an atomic index_add
        hot = (species.to(torch.int64).view(n, 1) == torch.arange(s, device=species.device)).to(torch.float32)
        picked = picked + mm(hot, bias).unsqueeze(1)
    return picked.transpose(1, 2)


__all__ = ["channel_linear", "species_channel_linear", "mm", "linear"]
