"""Differentiable matrix product for the model's dense layers, with split-K weight gradients.

The weight gradient of a layer applied to every edge (or every (node, m) row) is
``g^T x``: a product whose reduction dimension is the row count (about 10^5 edges at
cfg 4) and whose output is only, e.g., 64 x 64.  As one GEMM it covers a handful of
output tiles and leaves most of the GPU idle (~0.3 ms for 0.9 GFLOP).  ``mm`` splits
such a reduction into row blocks, multiplies the blocks as one batched GEMM and sums the
partial products.  Every derivative of ``mm`` is again ``mm`` (any order, as needed by
force-loss training), and adjoints the autograd engine will not run are skipped.
"""
from __future__ import annotations

import warnings

import torch
import torch.nn as nn

from ictc_o3.autograd.adjoint_requirements import required_gradients

SPLIT_ROWS = 2048          # rows per partial product
SPLIT_MIN_RATIO = 16       # split when K >= 16 * max(M, N) ...
SPLIT_MAX_OUTPUT = 1 << 18  # ... and the output has at most this many entries
# Measured on MI355X at K = 105,634 rows: outputs of 2^17 entries or more ([64, 2944] and its
# transpose) split best into 8,192-row blocks (0.45 / 0.40 ms vs 0.50 / 0.43 ms at 2,048), and outputs
# of at most 4,096 entries ([64, 64], [8, 64]) are fastest as one rocBLAS GEMM (0.04 ms vs 0.065 ms
# split); the split at 2,048 rows stays best in between ([64, 512], [512, 64]).
SPLIT_ROWS_LARGE = 8192
SPLIT_LARGE_OUTPUT = 1 << 17
SPLIT_SINGLE_GEMM_OUTPUT = 4096

# Edge-sized products against a weight-sized right operand ([E, K] @ [K, N] with E in the 10^5 range
# and K, N <= a few thousand: the radial MLP and its adjoints) run on rocBLAS with the right operand
# column-major (copied when needed; it is weight-sized).  Measured on MI355X at E = 105,634 against
# the default hipBLASLt choice: [E,64]@[64,2944] 0.485 vs 0.571 ms, [E,2944]@[2944,64] 0.372 vs
# 0.393-0.407 ms, [E,64]@[64,64] 0.014 vs 0.028-0.038 ms, [E,64]@[64,512] 0.068 vs 0.102 ms,
# [E,512]@[512,64] 0.064 vs 0.094 ms.  The other plain products (node-level layers) also run on
# rocBLAS: its host cost per call is about half hipBLASLt's (8-9 us vs 18.6 us measured), which
# matters because an eager energy-and-forces step issues ~60 of them and is bound by host issue
# time.  The split-K weight gradients (batched products) keep the default, faster for them.
# The backend is switched per product (a global setting, restored after the call: the product
# is issued from the thread that runs the model).
TALL_ROWS = 32768
TALL_MAX_RIGHT = 1 << 22
TALL_ROW_MAJOR_BELOW_K = 16
warnings.filterwarnings("ignore", message="torch.backends.cuda.preferred_blas_library is an experimental feature")


def _rows_view(t: torch.Tensor, blocks: int, rows: int) -> torch.Tensor:
    """[K', X] (K' = blocks * rows) -> [blocks, rows, X] (a view when t is contiguous)."""
    return t.reshape(blocks, rows, t.shape[1])


def _on_rocblas(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    prev = torch.backends.cuda.preferred_blas_library()
    torch.backends.cuda.preferred_blas_library("cublas")        # rocBLAS on ROCm
    try:
        return a @ b
    finally:
        torch.backends.cuda.preferred_blas_library(prev)


def _tall_product(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    # column-major right operand, except for a short reduction ([E, 8] @ [8, 64]: 25 us row-major,
    # 35 us column-major, 45 us on hipBLASLt)
    if b.shape[0] < TALL_ROW_MAJOR_BELOW_K:
        return _on_rocblas(a, b.contiguous())
    return _on_rocblas(a, b if b.stride(0) == 1 else b.t().contiguous().t())


def _product(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    m, k = a.shape
    n = b.shape[1]
    rows = SPLIT_ROWS_LARGE if m * n >= SPLIT_LARGE_OUTPUT else SPLIT_ROWS
    blocks = k // rows
    if blocks < 2 or k < SPLIT_MIN_RATIO * max(m, n) or m * n > SPLIT_MAX_OUTPUT:
        if a.is_cuda and m >= TALL_ROWS and k * n <= TALL_MAX_RIGHT:
            return _tall_product(a, b)
        return _on_rocblas(a, b) if a.is_cuda else a @ b
    if a.is_cuda and m * n <= SPLIT_SINGLE_GEMM_OUTPUT:
        return _on_rocblas(a, b)
    main = blocks * rows
    at = a.t()                                   # [K, M]: contiguous when a is a transposed activation
    left = _rows_view(at[:main], blocks, rows).transpose(1, 2)    # [blocks, M, rows]
    right = _rows_view(b[:main], blocks, rows)                     # [blocks, rows, N]
    out = torch.bmm(left, right).sum(0)
    if main < k:
        out = out + a[:, main:] @ b[main:]
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
    """a [M, K] @ b [K, N]."""
    return _MM.apply(a, b)


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x [R, in] @ weight[out, in]^T (no bias)."""
    return mm(x, weight.t())


class Linear(nn.Linear):
    """Bias-free nn.Linear (same parameter name and shape) computed through ``linear``; inputs
    of any leading shape."""

    def __init__(self, fan_in: int, fan_out: int):
        super().__init__(fan_in, fan_out, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        return linear(x.reshape(-1, x.shape[-1]), self.weight).reshape(*lead, self.out_features)
