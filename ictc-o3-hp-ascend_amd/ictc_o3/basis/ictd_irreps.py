"""ICTC harmonic basis, Clebsch-Gordan coefficients and path plans (host side).

Float64 numpy construction of the constants the HIP kernels consume.  The
mathematics follows the reference's ``ictc_o3/basis/ictd_irreps.py``:

* frozen monomial->harmonic basis ``B_l`` with its SHA-256 pins (``:632-694``);
* Gaussian Gram matrix on Sym^L (``:614-629``) and r^2k lifts (``ictd_fast.py:50-77``);
* trace-chain projector ``P_{L->l} = (V^T G V)^-1 V^T G`` (``:817-842``);
* ``C[m1,m2,m3]`` = project(poly-product(B_l1, B_l2)) (``:1223-1263``);
* 'component' CG normalisation (``:136-142``) and 'element' path
  normalisation over the output degree (``:101-133``);
* direction-harmonic monomial tables and component scale (``:891-953``).

Only immutable constants live here; all per-call arithmetic runs in HIP.
"""
from __future__ import annotations

import hashlib
import math
import os
from functools import lru_cache
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

_DATA = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data", "ictc_basis_v1.npz")

# SHA-256 of the float64 bytes of each frozen B_l (reference ictd_irreps.py:633-647).
_BASIS_SHA256 = (
    "6c3c396ed6b5c36dcae172271f462051b1266b851e92df3deea8ac65478fd712",
    "1332df685c45a61a0ac008a6a653295b8c5655361c1d34b6304b22ec40235fb8",
    "0881fbfd2a1866b76334d823d216ec74773a91a5f77234c45bb956838df7c315",
    "a7440553d51231cc044287b305d35cb5cafc59f77d7528d8189956c51a52a9e0",
    "f89f4b7f49ed9be8cc7fbbcec5e1a8947442c612d239bd42ce36180c6c644225",
    "8cce9bfb0a710f2c19d50ca3bcf6a79593697b5bd129085f10422066c2030ea8",
    "01cc08fe54c00daaff6899a86c923b62433f1691b7f283b95643c7be78ce9a96",
    "bde0ef7cf352a8cc83b4df959405616a390d270cf0b10bd93eed01da80e1a531",
    "85cdd2180f8078d9016110556076bf0464d12985ef079f51fee6c8f2641acf28",
    "190d6891295881dd5db122b80442a8feea21d0d716c6ff97faddcb0720509c6b",
    "fed2be677a84dc357b0e9b27e14b5bbc4c8a110520f44e536e7bc11365d70586",
    "4708bb0367de5a1c0d8d6bb01de80cb1a9a84ce6e128bc1913fecceabdf834ec",
    "761c7af5c246722d57a910b32ffe82741ac39326d6cba627be7db3b14d4ab689",
)

MAX_FROZEN_L = len(_BASIS_SHA256) - 1


def monomials(L: int) -> List[Tuple[int, int, int]]:
    """Exponent triples (a,b,c), a+b+c=L, in the basis' row order (a-major, then b)."""
    return [(a, b, L - a - b) for a in range(L + 1) for b in range(L - a + 1)]


@lru_cache(maxsize=None)
def harmonic_basis(l: int) -> np.ndarray:
    """Frozen ``B_l`` [dim Sym^l, 2l+1]; refuses data whose SHA-256 pin differs."""
    if not 0 <= l <= MAX_FROZEN_L:
        raise ValueError(f"the frozen ICTC basis covers l <= {MAX_FROZEN_L}, got {l}")
    with np.load(_DATA, allow_pickle=False) as blob:
        arr = np.ascontiguousarray(blob[f"l{l}"], dtype=np.float64)
    if hashlib.sha256(arr.tobytes()).hexdigest() != _BASIS_SHA256[l]:
        raise RuntimeError(f"ICTC basis data for l={l} does not match its SHA-256 pin")
    arr.setflags(write=False)
    return arr


def _odd_double_factorial(n: int) -> float:
    return float(math.prod(range(n, 0, -2))) if n > 0 else 1.0


@lru_cache(maxsize=None)
def gaussian_gram(L: int) -> np.ndarray:
    """<x^a y^b z^c, x^a' y^b' z^c'> under N(0, I3): product of 1-D Gaussian moments."""
    def moment(n: int) -> float:
        return 0.0 if n % 2 else _odd_double_factorial(n - 1)
    mons = monomials(L)
    g = np.array([[moment(a + a2) * moment(b + b2) * moment(c + c2) for (a2, b2, c2) in mons]
                  for (a, b, c) in mons], dtype=np.float64)
    g.setflags(write=False)
    return g


def _lift(l: int, k: int) -> np.ndarray:
    """Coefficient map of multiplication by (x^2+y^2+z^2)^k: Sym^l -> Sym^(l+2k)."""
    src, dst = monomials(l), monomials(l + 2 * k)
    row = {t: r for r, t in enumerate(dst)}
    out = np.zeros((len(dst), len(src)))
    for col, (a, b, c) in enumerate(src):
        for u in range(k + 1):
            for v in range(k - u + 1):
                w = k - u - v
                out[row[(a + 2 * u, b + 2 * v, c + 2 * w)], col] += (
                    math.factorial(k) / (math.factorial(u) * math.factorial(v) * math.factorial(w)))
    return out


@lru_cache(maxsize=None)
def trace_chain_projector(L: int, l: int) -> np.ndarray:
    """Gram-weighted least-squares projector Sym^L -> harmonic coordinates of degree l."""
    v = _lift(l, (L - l) // 2) @ harmonic_basis(l)
    g = gaussian_gram(L)
    return np.linalg.solve(v.T @ g @ v, v.T @ g)


@lru_cache(maxsize=None)
def coupling_tensor(l1: int, l2: int, l3: int) -> np.ndarray:
    """Raw ICTC coupling C[m1,m2,m3]: c = P_{l1+l2 -> l3}(poly(a) * poly(b)).

    Zero for triangle- or parity-forbidden triples."""
    out = np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    if not abs(l1 - l2) <= l3 <= l1 + l2 or (l1 + l2 + l3) % 2:
        return out
    basis1, basis2 = harmonic_basis(l1), harmonic_basis(l2)
    m1, m2 = monomials(l1), monomials(l2)
    target = {t: r for r, t in enumerate(monomials(l1 + l2))}
    # polynomial product of basis polynomials, column (i,j) -> coefficients on Sym^(l1+l2)
    prod = np.zeros((len(target), 2 * l1 + 1, 2 * l2 + 1))
    for r1, (a, b, c) in enumerate(m1):
        for r2, (a2, b2, c2) in enumerate(m2):
            prod[target[(a + a2, b + b2, c + c2)]] += np.outer(basis1[r1], basis2[r2])
    proj = trace_chain_projector(l1 + l2, l3)  # [2l3+1, dim Sym^(l1+l2)]
    out[:] = np.einsum("kr,rij->ijk", proj, prod)
    return out


def normalised_coupling(l1: int, l2: int, l3: int) -> np.ndarray:
    """'component' normalisation: Frobenius norm sqrt(2 l3 + 1)."""
    c = coupling_tensor(l1, l2, l3)
    norm = float(np.linalg.norm(c))
    return c * (math.sqrt(2 * l3 + 1) / norm) if norm > 1e-30 else c


# ----------------------------------------------------------------------------- paths
def triangle_paths(input_lmax: int, edge_lmax: int, output_lmax: int) -> List[Tuple[int, int, int]]:
    """All (l1,l2,l3) with l1<=L_in, l2<=L_edge, l3<=L_out, |l1-l2|<=l3<=l1+l2 and even
    l1+l2+l3, in ascending (l1,l2,l3) order (reference operators.py:54-55 with the
    owner's ordering, ictd_irreps.py:2161-2175)."""
    return [(i, j, k) for i in range(input_lmax + 1) for j in range(edge_lmax + 1)
            for k in range(output_lmax + 1) if abs(i - j) <= k <= i + j and (i + j + k) % 2 == 0]


def element_path_scales(paths: Sequence[Tuple[int, int, int]]) -> List[float]:
    """1/sqrt(#paths sharing the output degree) -- 'element' path normalisation."""
    count: Dict[int, int] = {}
    for p in paths:
        count[p[2]] = count.get(p[2], 0) + 1
    return [1.0 / math.sqrt(count[p[2]]) for p in paths]


class PathPlan:
    """Bookkeeping of a path-preserving TP (mirrors the owner's ``paths``,
    ``path_offset``, ``path_counts_by_l``; reference ictd_irreps.py:2194-2212, 2514-2526).

    Output layout: per output degree l (ascending), per path with that l3 in
    owner order, ``2l+1`` components, each a channel-contiguous row of C floats
    (the public ``ir_mul`` packing)."""

    def __init__(self, paths: Sequence[Tuple[int, int, int]], channels: int):
        self.paths = [tuple(int(v) for v in p) for p in paths]
        self.channels = int(channels)
        self.lmax = max(max(p) for p in self.paths) if self.paths else 0
        by_group: Dict[Tuple[int, int], List[int]] = {}
        for idx, (l1, l2, _) in enumerate(self.paths):
            by_group.setdefault((l1, l2), []).append(idx)
        self.path_offset = [0] * len(self.paths)
        self.path_counts_by_l = {l: 0 for l in range(self.lmax + 1)}
        for key in sorted(by_group):
            for idx in by_group[key]:
                l3 = self.paths[idx][2]
                self.path_offset[idx] = self.path_counts_by_l[l3]
                self.path_counts_by_l[l3] += 1
        self.scales = element_path_scales(self.paths)
        offsets, acc = {}, 0
        for l in range(self.lmax + 1):
            offsets[l] = acc
            acc += self.path_counts_by_l[l] * (2 * l + 1)
        self.output_components = acc
        # first output component of each path
        self.output_component_offset = [offsets[l3] + self.path_offset[i] * (2 * l3 + 1)
                                        for i, (_, _, l3) in enumerate(self.paths)]

    @property
    def num_paths(self) -> int:
        return len(self.paths)


# ----------------------------------------------------------------------------- harmonics
@lru_cache(maxsize=None)
def harmonics_tables(l: int) -> Tuple[List[Tuple[int, int, int]], np.ndarray, float]:
    """(monomials, multinomial-weighted projection [dim Sym^l, 2l+1], component scale).

    Y_l(n) = scale * sum_r n^mon_r * multinomial_r * (G_l B_l)[r, :]; the scale gives
    every component unit mean square over the unit sphere (reference ictd_irreps.py:891-953)."""
    mons = monomials(l)
    multi = np.array([math.factorial(l) / (math.factorial(a) * math.factorial(b) * math.factorial(c))
                      for a, b, c in mons])
    proj = gaussian_gram(l) @ harmonic_basis(l)
    if l == 0:
        return mons, np.ones((1, 1)), 1.0

    def sphere(a: int, b: int, c: int) -> float:
        if a % 2 or b % 2 or c % 2:
            return 0.0
        return (_odd_double_factorial(a - 1) * _odd_double_factorial(b - 1) * _odd_double_factorial(c - 1)
                / _odd_double_factorial(a + b + c + 1))
    s = np.array([[multi[i] * multi[j] * sphere(a + a2, b + b2, c + c2)
                   for j, (a2, b2, c2) in enumerate(mons)] for i, (a, b, c) in enumerate(mons)])
    mean_square = float(np.trace(proj.T @ s @ proj)) / (2 * l + 1)
    return mons, multi[:, None] * proj, 1.0 / math.sqrt(max(mean_square, 1e-30))


# ----------------------------------------------------------------------------- owner module
import torch  # noqa: E402
import torch.nn as nn  # noqa: E402


def _irrep_factor(l1: int, l2: int, l3: int, normalization: str) -> float:
    """Scale of a CG tensor relative to the compiled 'component' normalisation."""
    if normalization == "component":
        return 1.0
    if normalization == "norm":
        return 1.0 / math.sqrt(2 * l3 + 1)
    return float(np.linalg.norm(coupling_tensor(l1, l2, l3))) / math.sqrt(2 * l3 + 1)


class EdgeWeightedPathPreservingTensorProduct(nn.Module):
    """Path-preserving channelwise TP owner (reference ``ictd_irreps.py:2125-2794``).

    Holds ``paths`` (ascending (l1,l2,l3) among the allowed ones), the learnable
    per-(path, channel) ``weight`` [P, C], ``path_offset`` / ``path_counts_by_l``
    and the per-path normalisation.  ``forward`` takes the owner's dict layout
    ``x1[l] [E,C,2l+1]``, ``x2[l] [E,1,2l+1]``, gates ``[E,P,C]`` or ``[E,P*C]`` and
    returns ``{l: [E, count_l*C, 2l+1]}``; the arithmetic runs in the HIP kernels.
    """

    def __init__(self, channels: int, lmax: int, *, allowed_paths=None, path_policy: str = "full",
                 max_rank_other: Optional[int] = None, normalization: str = "component",
                 irrep_normalization: Optional[str] = None, path_normalization: str = "element",
                 internal_compute_dtype: Optional[torch.dtype] = None):
        super().__init__()
        self.channels, self.lmax = int(channels), int(lmax)
        norm = irrep_normalization if irrep_normalization is not None else normalization
        if norm not in ("component", "norm", "none"):
            raise ValueError("irrep_normalization must be 'component', 'norm' or 'none'")
        if path_normalization not in ("element", "path", "none"):
            raise ValueError("path_normalization must be 'element', 'path' or 'none'")
        self._normalization, self._path_normalization = norm, path_normalization
        self.internal_compute_dtype = (torch.get_default_dtype() if internal_compute_dtype is None
                                       else internal_compute_dtype)
        every = [(a, b, c) for a in range(self.lmax + 1) for b in range(self.lmax + 1)
                 for c in range(abs(a - b), min(a + b, self.lmax) + 1) if (a + b + c) % 2 == 0]
        if allowed_paths is not None:
            allowed = {tuple(p) for p in allowed_paths}
            self.paths = [p for p in every if p in allowed]
        elif path_policy == "full":
            self.paths = every
        elif path_policy == "max_rank_other":
            if max_rank_other is None:
                raise ValueError("path_policy='max_rank_other' requires max_rank_other")
            self.paths = [p for p in every if min(p[0], p[1]) <= int(max_rank_other)]
        else:
            raise ValueError(f"Unknown path_policy={path_policy!r}")
        self.num_paths = len(self.paths)
        self.weight = nn.Parameter(torch.randn(self.num_paths, self.channels) * 0.02)
        plan = PathPlan(self.paths, self.channels)
        self.path_offset = list(plan.path_offset)
        self.path_counts_by_l = {l: plan.path_counts_by_l.get(l, 0) for l in range(self.lmax + 1)}
        self.path_l3 = [p[2] for p in self.paths]
        if path_normalization == "none":
            path_scales = [1.0] * self.num_paths
        else:
            path_scales = element_path_scales(self.paths)
        self.path_scales = [s * _irrep_factor(*p, norm) for s, p in zip(path_scales, self.paths)]
        self._plans: Dict[Tuple[int, int], object] = {}

    def hip_plan(self, input_lmax: int, edge_lmax: int):
        """Launch plan for the given input/edge degrees (cached)."""
        key = (int(input_lmax), int(edge_lmax))
        plan = self._plans.get(key)
        if plan is None:
            from ictc_o3.backends.hip.tensor_product import TensorProductPlan
            plan = TensorProductPlan(self.paths, self.channels, input_lmax, edge_lmax, self.lmax)
            for i, scale in enumerate(self.path_scales):
                plan.set_scale(i, scale)
            self._plans[key] = plan
        return plan

    def effective_gates(self, gates: Optional[torch.Tensor], rows: int) -> torch.Tensor:
        """gates * weight as [E, P*C]: the per-(path, channel) weight is always folded, as the
        reference does (``backends/ascend/packed_tensor_product.py:163-164``), so any change of
        the weight -- including writes through ``weight.data`` -- is seen by the next call.
        A unit weight multiplies exactly (g * 1 == g), so the result equals the gates then."""
        w = self.weight
        if gates is None:
            return w.reshape(1, -1).expand(rows, -1).contiguous()
        gates = gates.reshape(rows, self.num_paths, self.channels)
        return (gates * w[None]).reshape(rows, self.num_paths * self.channels)

    def output_weight_rows(self) -> torch.Tensor:
        """The weight laid out along the packed ir_mul output: entry (l3 block, path offset, m, c)
        holds weight[p, c] of the path p that writes that row.  The message is linear in each
        path's gate and sums over edges, so ``message(g * weight) == weight_rows * message(g)``:
        a receiver-level product instead of one over every edge's gates (the reference folds
        into the gates, ``packed_tensor_product.py:163-164``; the results agree to rounding).
        Differentiable with respect to a live weight."""
        parts = []
        for l3 in range(self.lmax + 1):
            ordered = sorted((self.path_offset[p], p) for p in range(self.num_paths) if self.paths[p][2] == l3)
            if not ordered:
                continue
            idx = torch.tensor([p for _, p in ordered], device=self.weight.device)
            rows = self.weight.index_select(0, idx)                     # [count, C]
            parts.append(rows[:, None, :].expand(len(ordered), 2 * l3 + 1, self.channels).reshape(-1))
        return torch.cat(parts) if parts else self.weight.new_zeros(0)

    def forward(self, x1: Dict[int, torch.Tensor], x2: Dict[int, torch.Tensor],
                gates: Optional[torch.Tensor] = None) -> Dict[int, torch.Tensor]:
        """The reference's HP hook (ictd_irreps.py:2773-2775) taken unconditionally: the HIP
        ``tensor_product(owner, x1, x2, gates)``."""
        from ictc_o3.backends.hip.tensor_product import tensor_product
        return tensor_product(self, x1, x2, gates)
