"""Projection of a contraction module's actual U buffers onto the coupling chains the HIP
kernels evaluate (reference ``ictc_o3/ops/factorized_contraction.py:51-149``).

The MACE contraction of order nu computes sum_k W[s, k, c] <U[..., k], x (x) ... (x) x>, which
depends on each U column only through its part symmetric in the nu input legs.  Any module
whose symmetric U columns lie in the span of the chain columns therefore runs on the chain
kernels: with compress(U) the symmetric compression (sum of the entries of every permutation
of each index multiset, ``factorized_contraction.py:17-24``),

    compress(U_module) = compress(U_chain) A        (A [K_chain, K_module], least squares, float64)

and the kernel weights are W_chain[s, :, c] = A W_module[s, :, c], a differentiable map whose
adjoint carries the weight gradient back (A^T) and every higher derivative.  The
reconstruction is gated as in the reference (``:84-92``): the largest residual entry relative
to the largest U entry must stay within 4e-6 for float32 U, 2e-11 for float64; otherwise no
plan exists and the caller refuses the module.
"""
from __future__ import annotations

import itertools
from functools import lru_cache
from typing import List, Optional, Tuple

import numpy as np
import torch


@lru_cache(maxsize=None)
def _multiset_index(dim: int, order: int) -> Tuple[np.ndarray, int]:
    """For every flat index of D^order, the index of its sorted multiset among the
    combinations with replacement (and their count)."""
    combos = list(itertools.combinations_with_replacement(range(dim), order))
    lookup = {c: i for i, c in enumerate(combos)}
    mapping = np.array([lookup[tuple(sorted(idx))] for idx in itertools.product(range(dim), repeat=order)],
                       dtype=np.int64)
    return mapping, len(combos)


def compress(u: np.ndarray, order: int, dim: int, l_out: int) -> np.ndarray:
    """Symmetric compression of U [(2l+1)?, D^order, K] -> [(2l+1) * multisets, K]."""
    rows = 1 if l_out == 0 else 2 * l_out + 1
    k = u.shape[-1]
    flat = u.reshape(rows, dim ** order, k)
    mapping, count = _multiset_index(dim, order)
    out = np.zeros((rows, count, k))
    for r in range(rows):
        np.add.at(out[r], mapping, flat[r])
    return out.reshape(rows * count, k)


@lru_cache(maxsize=None)
def _chain_basis(lmax: int, l_out: int, order: int) -> np.ndarray:
    from ictc_o3.basis.symmetric_u import u_matrix
    return compress(u_matrix(lmax, l_out, order), order, (lmax + 1) ** 2, l_out)


def projection(u_module: np.ndarray, lmax: int, l_out: int, order: int,
               tolerance: float) -> Tuple[Optional[np.ndarray], float]:
    """(A [K_chain, K_module], relative residual); A is None when the residual exceeds the
    tolerance (the module's U has components the chain columns cannot reproduce)."""
    dim = (lmax + 1) ** 2
    basis = _chain_basis(lmax, l_out, order)
    actual = compress(np.asarray(u_module, dtype=np.float64), order, dim, l_out)
    if basis.shape[0] != actual.shape[0]:
        return None, float("inf")
    scale = float(np.abs(actual).max()) if actual.size else 0.0
    if scale == 0.0:
        return np.zeros((basis.shape[1], actual.shape[1])), 0.0
    a = np.linalg.lstsq(basis, actual, rcond=None)[0]
    relative = float(np.abs(basis @ a - actual).max()) / scale
    return (a if relative <= tolerance else None), relative


class FactorizedPlan:
    """Per (target degree, order) projection matrices of one module, in the kernels' weight
    column order (target degree ascending, orders correlation..1)."""

    def __init__(self, matrices: List[List[torch.Tensor]], reconstruction: List[float]):
        self.matrices = matrices
        self.reconstruction_relative = reconstruction
        rows = sum(a.shape[0] for mats in matrices for a in mats)
        cols = sum(a.shape[1] for mats in matrices for a in mats)
        # every (target degree, order) projection on the diagonal of one [KTOT, K_module] matrix
        first = matrices[0][0]
        self.block = torch.zeros(rows, cols, dtype=first.dtype, device=first.device)
        r = c = 0
        for mats in matrices:
            for a in mats:
                self.block[r:r + a.shape[0], c:c + a.shape[1]] = a
                r, c = r + a.shape[0], c + a.shape[1]
        self._table_key, self._table = None, None

    def weight_table(self, contractions) -> torch.Tensor:
        """[S, KTOT, C] kernel weights from the modules' live weights (differentiable): one product
        of the block-diagonal projection with the concatenated module weights.  When no weight
        requires a gradient the table is kept until a weight is replaced or modified in place."""
        from ictc_o3.backends.hip.linear import mm
        ws = [w for con in contractions for w in (con.weights_max, *con.weights)]
        frozen = not (torch.is_grad_enabled() and any(w.requires_grad for w in ws))
        key = tuple((id(w), w.data_ptr(), w._version) for w in ws) if frozen else None
        if frozen and key == self._table_key:
            return self._table
        w = torch.cat(ws, 1)                                    # [S, K_module, C]
        s, k, c = w.shape
        flat = w.transpose(0, 1).reshape(k, s * c)
        # rocBLAS on the GPU; a module built on the host (the factory's reconstruction gate) uses torch
        table = mm(self.block, flat) if flat.is_cuda else self.block @ flat
        table = table.reshape(-1, s, c).transpose(0, 1).contiguous()
        if frozen:
            self._table_key, self._table = key, table
        else:
            self._table_key, self._table = None, None
        return table


def constant_key(owner, device) -> tuple:
    """Identity, storage and version of every U buffer (a replaced or modified U re-plans)."""
    key = [str(device)]
    for con in owner.symmetric_contractions.contractions:
        for nu in range(1, con.correlation + 1):
            u = con.U_tensors(nu)
            key.append((id(u), u.data_ptr(), u._version, u.dtype, tuple(u.shape)))
    return tuple(key)


def _plan(owner, x: torch.Tensor) -> Optional[FactorizedPlan]:
    """The projection plan of a bridge-U module for inputs like x, cached on the module; None
    when a U buffer does not reconstruct within the gate (reference ``_plan``, ``:51-149``)."""
    modules = list(owner.symmetric_contractions.contractions)
    correlation = modules[0].correlation
    if owner.lmax < 0 or correlation not in (1, 2, 3) or any(m.correlation != correlation for m in modules):
        return None
    if any(m.U_tensors(nu).requires_grad for m in modules for nu in range(1, correlation + 1)):
        return None
    key = constant_key(owner, x.device)
    cached = getattr(owner, "_factorized_u_cache", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    matrices, reconstruction = [], []
    plan = None
    for con in modules:
        mats = []
        for nu in range(correlation, 0, -1):
            u = con.U_tensors(nu).detach().to("cpu", torch.float64).numpy()
            tolerance = 4e-6 if con.U_tensors(nu).dtype == torch.float32 else 2e-11
            a, relative = projection(u, owner.lmax, con.output_lmax, nu, tolerance)
            if a is None:
                owner._factorized_u_cache = (key, None)
                return None
            mats.append(torch.from_numpy(a).to(device=x.device, dtype=x.dtype))
            reconstruction.append(relative)
        matrices.append(mats)
    plan = FactorizedPlan(matrices, reconstruction)
    owner._factorized_u_cache = (key, plan)
    return plan
