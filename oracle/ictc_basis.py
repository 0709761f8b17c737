"""Oracle: ICTC harmonic basis, CG tensors and direction harmonics (CPU, float64).

Restates ``ictc_o3/basis/ictd_fast.py`` and the basis/CG/harmonics part of
``ictc_o3/basis/ictd_irreps.py`` of the reference.  Test infrastructure only.
"""
from __future__ import annotations

import hashlib
import math
import os
from functools import lru_cache
from typing import Dict, List, Sequence, Tuple

import numpy as np
import torch

_F64 = torch.float64
_BASIS_NPZ = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                          "tests", "golden", "ictc_basis_v1.npz")

# ictc_o3/basis/ictd_irreps.py:633-647 -- SHA-256 of the float64 bytes of B_l.
BASIS_SHA256 = {
    0: "6c3c396ed6b5c36dcae172271f462051b1266b851e92df3deea8ac65478fd712",
    1: "1332df685c45a61a0ac008a6a653295b8c5655361c1d34b6304b22ec40235fb8",
    2: "0881fbfd2a1866b76334d823d216ec74773a91a5f77234c45bb956838df7c315",
    3: "a7440553d51231cc044287b305d35cb5cafc59f77d7528d8189956c51a52a9e0",
    4: "f89f4b7f49ed9be8cc7fbbcec5e1a8947442c612d239bd42ce36180c6c644225",
    5: "8cce9bfb0a710f2c19d50ca3bcf6a79593697b5bd129085f10422066c2030ea8",
    6: "01cc08fe54c00daaff6899a86c923b62433f1691b7f283b95643c7be78ce9a96",
    7: "bde0ef7cf352a8cc83b4df959405616a390d270cf0b10bd93eed01da80e1a531",
    8: "85cdd2180f8078d9016110556076bf0464d12985ef079f51fee6c8f2641acf28",
    9: "190d6891295881dd5db122b80442a8feea21d0d716c6ff97faddcb0720509c6b",
    10: "fed2be677a84dc357b0e9b27e14b5bbc4c8a110520f44e536e7bc11365d70586",
    11: "4708bb0367de5a1c0d8d6bb01de80cb1a9a84ce6e128bc1913fecceabdf834ec",
    12: "761c7af5c246722d57a910b32ffe82741ac39326d6cba627be7db3b14d4ab689",
}


# --------------------------------------------------------------------------- monomials
def counts_list(L: int) -> List[Tuple[int, int, int]]:
    """All (a,b,c) with a+b+c=L, a-major order (``ictd_fast.py:11-18``)."""
    return [(a, b, L - a - b) for a in range(L + 1) for b in range(L - a + 1)]


def sym_dim(L: int) -> int:
    """dim Sym^L(R^3) (``ictd_irreps.py:575-577``)."""
    return (L + 2) * (L + 1) // 2


def r2k_lift(l_src: int, k: int) -> torch.Tensor:
    """Multiplication by (x^2+y^2+z^2)^k on monomial coefficients (``ictd_fast.py:50-77``)."""
    src = counts_list(l_src)
    if k == 0:
        return torch.eye(len(src), dtype=_F64)
    dst = counts_list(l_src + 2 * k)
    index = {t: i for i, t in enumerate(dst)}
    out = torch.zeros(len(dst), len(src), dtype=_F64)
    for col, (a, b, c) in enumerate(src):
        for u in range(k + 1):
            for v in range(k - u + 1):
                w = k - u - v
                coef = math.factorial(k) / (math.factorial(u) * math.factorial(v) * math.factorial(w))
                out[index[(a + 2 * u, b + 2 * v, c + 2 * w)], col] += coef
    return out


def _double_factorial(n: int) -> int:
    out = 1
    for k in range(n, 0, -2):
        out *= k
    return out


def _gaussian_moment(n: int) -> float:
    """E[x^n], x ~ N(0,1) (``ictd_irreps.py:589-593``)."""
    return 0.0 if n % 2 else float(_double_factorial(n - 1))


def _sphere_moment(a: int, b: int, c: int) -> float:
    """E[x^a y^b z^c] on the unit sphere (``ictd_irreps.py:596-611``)."""
    if a % 2 or b % 2 or c % 2:
        return 0.0
    p, q, r = a // 2, b // 2, c // 2
    return (_double_factorial(2 * p - 1) * _double_factorial(2 * q - 1) * _double_factorial(2 * r - 1)
            / _double_factorial(2 * (p + q + r) + 1))


@lru_cache(maxsize=None)
def gram_gaussian(L: int) -> torch.Tensor:
    """Rotation-invariant Gaussian Gram matrix on Sym^L (``ictd_irreps.py:614-629``)."""
    counts = counts_list(L)
    g = torch.zeros(len(counts), len(counts), dtype=_F64)
    for i, (a, b, c) in enumerate(counts):
        for j, (a2, b2, c2) in enumerate(counts):
            g[i, j] = _gaussian_moment(a + a2) * _gaussian_moment(b + b2) * _gaussian_moment(c + c2)
    return g


# --------------------------------------------------------------------------- frozen basis
@lru_cache(maxsize=None)
def harmonic_basis(l: int) -> torch.Tensor:
    """Frozen B_l [sym_dim(l), 2l+1], SHA-verified (``ictd_irreps.py:650-694``)."""
    with np.load(_BASIS_NPZ, allow_pickle=False) as blob:
        arr = np.ascontiguousarray(blob[f"l{int(l)}"], dtype=np.float64)
    if hashlib.sha256(arr.tobytes()).hexdigest() != BASIS_SHA256[int(l)]:
        raise RuntimeError(f"ICTC basis fixture l={l} failed its SHA-256 pin")
    if arr.shape != (sym_dim(l), 2 * l + 1):
        raise RuntimeError("bad basis shape")
    return torch.from_numpy(arr.copy())


@lru_cache(maxsize=None)
def harmonic_projector(L: int, l: int) -> torch.Tensor:
    """P_{L->l} = (V^T G V)^-1 V^T G with V = lift(l, (L-l)/2) B_l (``ictd_irreps.py:817-842``)."""
    v = r2k_lift(l, (L - l) // 2) @ harmonic_basis(l)
    g = gram_gaussian(L)
    return torch.linalg.solve(v.T @ g @ v, v.T @ g)


# --------------------------------------------------------------------------- CG
def poly_mult_matrix(l1: int, l2: int) -> torch.Tensor:
    """Monomial product map Sym^l1 x Sym^l2 -> Sym^(l1+l2) (``ictd_irreps.py:1204-1220``)."""
    c1, c2, cl = counts_list(l1), counts_list(l2), counts_list(l1 + l2)
    index = {t: i for i, t in enumerate(cl)}
    m = torch.zeros(len(cl), len(c1) * len(c2), dtype=_F64)
    for i, a in enumerate(c1):
        for j, b in enumerate(c2):
            m[index[(a[0] + b[0], a[1] + b[1], a[2] + b[2])], i * len(c2) + j] = 1.0
    return m


@lru_cache(maxsize=None)
def cg_tensor(l1: int, l2: int, l3: int) -> torch.Tensor:
    """Raw coupling tensor C[m1,m2,m3] in the ICTC basis (``ictd_irreps.py:1223-1263``)."""
    if not (abs(l1 - l2) <= l3 <= l1 + l2) or (l1 + l2 + l3) % 2:
        return torch.zeros(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1, dtype=_F64)
    b1, b2 = harmonic_basis(l1), harmonic_basis(l2)
    outer = torch.einsum("im,jn->ijmn", b1, b2).reshape(b1.shape[0] * b2.shape[0], -1)
    c3 = harmonic_projector(l1 + l2, l3) @ (poly_mult_matrix(l1, l2) @ outer)
    return c3.T.reshape(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1).contiguous()


def cg_component_normalised(c: torch.Tensor, l3: int) -> torch.Tensor:
    """'component' irrep normalisation: scale to ||C||_F = sqrt(2l3+1) (``ictd_irreps.py:136-142``)."""
    norm = c.norm().item()
    return c * (math.sqrt(2 * l3 + 1) / norm) if norm > 1e-30 else c


def path_normalisation_scales(paths: Sequence[Tuple[int, int, int]]) -> List[float]:
    """'element' path normalisation over output l3, num_elements=1 (``ictd_irreps.py:101-133``)."""
    counts: Dict[int, int] = {}
    for p in paths:
        counts[p[2]] = counts.get(p[2], 0) + 1
    return [1.0 / math.sqrt(float(counts[p[2]])) for p in paths]


# --------------------------------------------------------------------------- rotations
def _monomial_generator(L: int, axis: str) -> torch.Tensor:
    """so(3) generator on degree-L monomial coefficients (``ictd_irreps.py:1266-1293``)."""
    counts = counts_list(L)
    idx = {t: i for i, t in enumerate(counts)}
    out = torch.zeros(len(counts), len(counts), dtype=_F64)
    for j, (a, b, c) in enumerate(counts):
        terms = []
        if axis == "x":
            if c:
                terms.append((float(c), (a, b + 1, c - 1)))
            if b:
                terms.append((float(-b), (a, b - 1, c + 1)))
        elif axis == "y":
            if a:
                terms.append((float(a), (a - 1, b, c + 1)))
            if c:
                terms.append((float(-c), (a + 1, b, c - 1)))
        else:
            if b:
                terms.append((float(b), (a + 1, b - 1, c)))
            if a:
                terms.append((float(-a), (a - 1, b + 1, c)))
        for coef, key in terms:
            out[idx[key], j] += coef
    return out


@lru_cache(maxsize=None)
def harmonic_generator(l: int, axis: str) -> torch.Tensor:
    """so(3) generator in the ICTC harmonic basis, B^T G J B (``ictd_irreps.py:1296-1301``)."""
    b = harmonic_basis(l)
    return (b.T @ gram_gaussian(l) @ _monomial_generator(l, axis) @ b).contiguous()


def wigner_d(l: int, omega: torch.Tensor) -> torch.Tensor:
    """D_l(R) = exp(sum_a omega_a J_a) in the ICTC basis; R = exp of the matching 3x3 generator."""
    gen = sum(float(omega[i]) * harmonic_generator(l, a) for i, a in enumerate("xyz"))
    return torch.linalg.matrix_exp(gen)


@lru_cache(maxsize=None)
def full_cg_tensor(l1: int, l2: int, l3: int) -> torch.Tensor:
    """SO(3) intertwiner solved from the infinitesimal equivariance equations
    (``ictd_irreps.py:1304-1374``): unit-Frobenius null vector, sign fixed so the
    largest-magnitude entry is positive.  Covers odd l1+l2+l3 paths too."""
    if not abs(l1 - l2) <= l3 <= l1 + l2:
        return torch.zeros(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1, dtype=_F64)
    d1, d2, d3 = 2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1
    rows = []
    for axis in "xyz":
        j1, j2, j3 = (harmonic_generator(l, axis) for l in (l1, l2, l3))
        jin = torch.kron(j1, torch.eye(d2, dtype=_F64)) + torch.kron(torch.eye(d1, dtype=_F64), j2)
        # vec(J3 C - C Jin) for C [d3, d1*d2] row-major: (J3 (x) I - I (x) Jin^T) vec(C)
        rows.append(torch.kron(j3, torch.eye(d1 * d2, dtype=_F64))
                    - torch.kron(torch.eye(d3, dtype=_F64), jin.T.contiguous()))
    a = torch.cat(rows, 0)
    c = torch.from_numpy(null_vector(a.numpy())).reshape(d3, d1 * d2).T.reshape(d1, d2, d3).contiguous()
    return fix_sign(c)


def null_vector(a: np.ndarray) -> np.ndarray:
    """Right singular vector of the smallest singular value; LAPACK gesdd, falling back to
    gesvd and then to the eigenvector of A^T A (``_robust_svd_vh``, ictd_irreps.py:1322-1342)."""
    try:
        return np.linalg.svd(a, full_matrices=True)[2][-1].copy()
    except np.linalg.LinAlgError:
        pass
    try:
        import scipy.linalg
        return scipy.linalg.svd(a, full_matrices=True, lapack_driver="gesvd")[2][-1].copy()
    except (np.linalg.LinAlgError, ValueError):
        w, v = np.linalg.eigh(a.T @ a)
        return v[:, 0].copy()


def fix_sign(c: torch.Tensor) -> torch.Tensor:
    """Largest-magnitude entry positive (``ictd_irreps.py:1369-1372``); among entries within
    1e-9 of the maximum magnitude the first in row-major order decides, so round-off
    cannot flip the sign between machines."""
    flat = c.flatten()
    mag = flat.abs()
    first = int(torch.nonzero(mag >= mag.max() * (1 - 1e-9))[0])
    return -c if flat[first] < 0 else c


# --------------------------------------------------------------------------- harmonics
@lru_cache(maxsize=None)
def _monomial_exps_coefs(l: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(a,b,c) exponents and multinomial coefficients (``ictd_irreps.py:891-909``)."""
    counts = counts_list(l)
    exps = torch.tensor(counts, dtype=torch.int64)
    coefs = torch.tensor([math.factorial(l) / (math.factorial(a) * math.factorial(b) * math.factorial(c))
                          for a, b, c in counts], dtype=_F64)
    return exps, coefs


@lru_cache(maxsize=None)
def direction_projection(l: int) -> torch.Tensor:
    """G_l B_l (``ictd_irreps.py:912-922``)."""
    if l == 0:
        return torch.ones(1, 1, dtype=_F64)
    return (gram_gaussian(l) @ harmonic_basis(l)).contiguous()


@lru_cache(maxsize=None)
def direction_component_scale(l: int) -> float:
    """Scale giving unit RMS per component over the sphere (``ictd_irreps.py:925-953``)."""
    if l == 0:
        return 1.0
    counts = counts_list(l)
    _, coefs = _monomial_exps_coefs(l)
    d = len(counts)
    sg = torch.zeros(d, d, dtype=_F64)
    for i, (a, b, c) in enumerate(counts):
        for j, (a2, b2, c2) in enumerate(counts):
            sg[i, j] = float(coefs[i]) * float(coefs[j]) * _sphere_moment(a + a2, b + b2, c + c2)
    p = direction_projection(l)
    ms = torch.trace(p.T @ sg @ p) / float(2 * l + 1)
    return float(ms.clamp_min(1e-30).rsqrt().item())


def _power_table(x: torch.Tensor, max_power: int) -> torch.Tensor:
    """[x^0..x^max] by repeated products (``ictd_irreps.py:962-976``)."""
    powers, cur = [torch.ones_like(x)], torch.ones_like(x)
    for _ in range(max_power):
        cur = cur * x
        powers.append(cur)
    return torch.stack(powers, -1)


def direction_harmonics_all(n: torch.Tensor, lmax: int) -> List[torch.Tensor]:
    """Y_l(n) for l=0..lmax, list of [..., 2l+1] (``ictd_irreps.py:1113-1168``)."""
    out = [torch.ones(*n.shape[:-1], 1, dtype=n.dtype)]
    if lmax == 0:
        return out
    xp, yp, zp = (_power_table(n[..., i], lmax) for i in range(3))
    for l in range(1, lmax + 1):
        exps, coefs = _monomial_exps_coefs(l)
        t = xp[..., exps[:, 0]] * yp[..., exps[:, 1]] * zp[..., exps[:, 2]]
        t = t * coefs.to(n.dtype)
        out.append((t @ direction_projection(l).to(n.dtype))
                   * torch.tensor(direction_component_scale(l), dtype=n.dtype))
    return out


def direction_harmonics_packed(n: torch.Tensor, lmax: int) -> torch.Tensor:
    """Y packed as [..., (lmax+1)^2] -- the ``harmonics`` argument of the public TP."""
    return torch.cat(direction_harmonics_all(n, lmax), -1)
