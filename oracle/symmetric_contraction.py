"""Oracle: correlation <= 3 symmetric contraction in the ICTC basis (CPU).

Restates
* the pure-ICTC coupling basis and U tensors -- ``_ictd_so3_coupled_basis`` /
  ``_ictd_u_matrix_so3_compute`` / ``ictd_u_matrix_so3``
  (reference ``ictc_o3/basis/ictd_irreps.py:1387-1517``), built from the null-space
  intertwiners ``build_full_cg_tensor_so3`` (``:1304-1374``) with 'component'
  normalisation (``:136-142``);
* the MACE contraction recursion with species-selected weights --
  ``_Contraction._forward_selected_elements``
  (``ictc_o3/ops/_mace_symmetric_contraction.py:298-346``): weights
  ``weights_max [S,K_nu,C]`` (nu = correlation), ``weights[i] [S,K,C]`` for the
  lower orders, init ``randn / K`` (``:153-156, 200-205``);
* the module's flat layouts: input ``[N, C*(L+1)^2]`` with each degree block
  ``[C, 2l+1]`` (``ops/symmetric_contraction.py:14-16``), output concatenated per
  target degree as ``[C, 2l+1]`` (``_mace_symmetric_contraction.py:345``).

The reference's shipped ``create_symmetric_contraction`` folds e3nn U tensors through
an SVD-fitted basis bridge (``ops/symmetric_contraction.py:24-206``); e3nn is not
available here, so those U *values* are parity-unpinned.  The U used here is the
reference's own e3nn-free generator, which spans the same intertwiner space
(``ICTDPureUSymmetricContractionSO3``, ``mace_ictc/models/pure_cartesian_ictd_fix.py:1310-1389``).
Test infrastructure only.
"""
from __future__ import annotations

import math
from functools import lru_cache
from typing import Dict, List, Sequence, Tuple

import torch

from . import ictc_basis as B

_F64 = torch.float64


def _parity(l: int) -> int:
    return 1 if l % 2 == 0 else -1


def coupled_basis(lmax: int, correlation: int) -> List[Tuple[int, int, torch.Tensor]]:
    """``_ictd_so3_coupled_basis`` (``ictd_irreps.py:1387-1446``): list of
    (l_out, parity, tensor[2l_out+1, D, ..., D]) over all coupling chains."""
    dim = (lmax + 1) ** 2
    starts = {l: l * l for l in range(lmax + 1)}
    eye = torch.eye(dim, dtype=_F64)
    basis = [(l, _parity(l), eye[starts[l]:starts[l] + 2 * l + 1]) for l in range(lmax + 1)]
    for _ in range(2, correlation + 1):
        nxt = []
        for l_left, p_left, left in basis:
            for l_right in range(lmax + 1):
                rs = starts[l_right]
                for l_out in range(abs(l_left - l_right), l_left + l_right + 1):
                    cg = B.full_cg_tensor(l_left, l_right, l_out)
                    cg = B.cg_component_normalised(cg, l_out)
                    flat = left.reshape(2 * l_left + 1, -1)
                    coupled = torch.einsum("ar,abq->qrb", flat, cg)
                    full = torch.zeros(2 * l_out + 1, flat.shape[1], dim, dtype=_F64)
                    full[:, :, rs:rs + 2 * l_right + 1] = coupled
                    nxt.append((l_out, p_left * _parity(l_right),
                                full.reshape(2 * l_out + 1, *left.shape[1:], dim)))
        basis = sorted(nxt, key=lambda item: (item[0], item[1]))
    return basis


@lru_cache(maxsize=None)
def u_matrix(lmax: int, output_l: int, correlation: int) -> torch.Tensor:
    """``_ictd_u_matrix_so3_compute`` (``ictd_irreps.py:1466-1492``): stack of the chains
    with l_out = output_l and natural parity; scalar outputs drop the leading axis."""
    tensors = [t for l, p, t in coupled_basis(lmax, correlation)
               if l == output_l and p == _parity(output_l)]
    dim = (lmax + 1) ** 2
    if not tensors:
        shape = [dim] * correlation + [1]
        return torch.zeros(*([2 * output_l + 1] if output_l else []), *shape, dtype=_F64)
    if output_l == 0:
        tensors = [t.squeeze(0) for t in tensors]
    return torch.stack(tensors, -1).contiguous()


class SymmetricContractionOracle:
    """Species-conditioned symmetric contraction (one ``_Contraction`` per target degree)."""

    def __init__(self, num_elements: int, channels: int, lmax: int, target_lmax: int,
                 correlation: int = 3, *, seed: int = 0, dtype=_F64):
        self.S, self.C, self.lmax, self.target_lmax = num_elements, channels, lmax, target_lmax
        self.correlation = correlation
        gen = torch.Generator().manual_seed(seed)
        self.u: Dict[Tuple[int, int], torch.Tensor] = {}
        self.weights: Dict[Tuple[int, int], torch.Tensor] = {}
        for l in range(target_lmax + 1):
            for nu in range(correlation, 0, -1):        # creation order of the reference
                u = u_matrix(lmax, l, nu)
                self.u[(l, nu)] = u
                k = u.shape[-1]
                self.weights[(l, nu)] = (torch.randn(num_elements, k, channels, generator=gen,
                                                     dtype=torch.float64) / k).to(dtype)

    def input_blocks(self, x: torch.Tensor) -> torch.Tensor:
        """Flat [N, C*(L+1)^2] (degree blocks [C,2l+1]) -> [N, C, (L+1)^2]."""
        parts, off = [], 0
        for l in range(self.lmax + 1):
            w = self.C * (2 * l + 1)
            parts.append(x[:, off:off + w].reshape(-1, self.C, 2 * l + 1))
            off += w
        return torch.cat(parts, -1)

    def contract(self, x: torch.Tensor, species: torch.Tensor, output_l: int,
                 weights: Dict[Tuple[int, int], torch.Tensor] | None = None) -> torch.Tensor:
        """``_forward_selected_elements`` (``_mace_symmetric_contraction.py:298-346``)."""
        w = self.weights if weights is None else weights
        xb = self.input_blocks(x)
        idx = species.long()

        def coeff(order):
            sel = w[(output_l, order)].to(x.dtype).index_select(0, idx)      # [N, K, C]
            u = self.u[(output_l, order)].to(x.dtype)
            if output_l == 0:
                spec = {1: "ip,bpc->bci", 2: "ijp,bpc->bcij", 3: "ijkp,bpc->bcijk"}[order]
            else:
                spec = {1: "mip,bpc->bcmi", 2: "mijp,bpc->bcmij", 3: "mijkp,bpc->bcmijk"}[order]
            return torch.einsum(spec, u, sel)

        out = coeff(self.correlation)
        for order in range(self.correlation - 1, 0, -1):
            out = torch.einsum("bc...i,bci->bc...", out, xb)
            out = out + coeff(order)
        out = torch.einsum("bc...i,bci->bc...", out, xb)
        return out.reshape(out.shape[0], self.C * (2 * output_l + 1))

    def forward(self, x: torch.Tensor, species: torch.Tensor, weights=None) -> torch.Tensor:
        """Concatenation over target degrees (``ops/symmetric_contraction.py:199-206``)."""
        return torch.cat([self.contract(x, species, l, weights) for l in range(self.target_lmax + 1)], -1)
