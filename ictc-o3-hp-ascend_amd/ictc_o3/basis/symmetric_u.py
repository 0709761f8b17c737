"""Coupling chains of the correlation <= 3 symmetric contraction (host side, float64).

Each column of the contraction's U tensor is one coupling chain of the ICTC
basis (reference ``ictc_o3/basis/ictd_irreps.py:1387-1517``, the pure-ICTC U):

    order 1:  x_{l}                                    (l = l_out)
    order 2:  CG(la, lb -> l_out)[x_la, x_lb]
    order 3:  CG(L1, lc -> l_out)[CG(la, lb -> L1)[x_la, x_lb], x_lc]

with the SO(3) intertwiners solved from the infinitesimal equivariance equations
(``:1304-1374``; unit Frobenius null vector, largest-magnitude entry positive) and
'component' normalisation.  Columns keep the reference's order: the coupled basis
is re-sorted by (l, parity) after every order, and only chains with the target
degree and natural parity survive.  The HIP kernels evaluate these chains through
shared pair prefixes ``P_{la,lb,L1} = CG(la,lb,L1)[x, x]``.
"""
from __future__ import annotations

import math
from functools import lru_cache
from typing import List, NamedTuple, Tuple

import numpy as np

from .ictd_irreps import gaussian_gram, harmonic_basis, monomials


def _monomial_rotation_generator(L: int, axis: str) -> np.ndarray:
    """so(3) generator acting on degree-L monomial coefficients (x d/dy type vector fields)."""
    mons = monomials(L)
    row = {t: r for r, t in enumerate(mons)}
    out = np.zeros((len(mons), len(mons)))
    for col, (a, b, c) in enumerate(mons):
        if axis == "x":
            terms = [(c, (a, b + 1, c - 1)), (-b, (a, b - 1, c + 1))]
        elif axis == "y":
            terms = [(a, (a - 1, b, c + 1)), (-c, (a + 1, b, c - 1))]
        else:
            terms = [(b, (a + 1, b - 1, c)), (-a, (a - 1, b + 1, c))]
        for coef, key in terms:
            if coef:
                out[row[key], col] += coef
    return out


@lru_cache(maxsize=None)
def rotation_generator(l: int, axis: str) -> np.ndarray:
    """Generator in the ICTC harmonic basis, B^T G J B."""
    b = harmonic_basis(l)
    return b.T @ gaussian_gram(l) @ _monomial_rotation_generator(l, axis) @ b


@lru_cache(maxsize=None)
def intertwiner(l1: int, l2: int, l3: int) -> np.ndarray:
    """Unique (up to sign) SO(3) intertwiner [2l1+1, 2l2+1, 2l3+1], unit Frobenius norm,
    largest-magnitude entry positive (first such entry in row-major order); zero outside
    the triangle."""
    d1, d2, d3 = 2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1
    if not abs(l1 - l2) <= l3 <= l1 + l2:
        return np.zeros((d1, d2, d3))
    rows = []
    for axis in "xyz":
        j1, j2, j3 = (rotation_generator(l, axis) for l in (l1, l2, l3))
        jin = np.kron(j1, np.eye(d2)) + np.kron(np.eye(d1), j2)
        rows.append(np.kron(j3, np.eye(d1 * d2)) - np.kron(np.eye(d3), jin.T))
    c = _null_vector(np.concatenate(rows, 0)).reshape(d3, d1 * d2).T.reshape(d1, d2, d3).copy()
    flat = c.reshape(-1)
    mag = np.abs(flat)
    first = int(np.flatnonzero(mag >= mag.max() * (1 - 1e-9))[0])   # tie-robust sign rule
    return -c if flat[first] < 0 else c


def _null_vector(a: np.ndarray) -> np.ndarray:
    """Right singular vector of the smallest singular value (gesdd, then gesvd, then the
    lowest eigenvector of A^T A): LAPACK builds differ in which driver converges."""
    try:
        return np.linalg.svd(a, full_matrices=True)[2][-1]
    except np.linalg.LinAlgError:
        pass
    try:
        import scipy.linalg
        return scipy.linalg.svd(a, full_matrices=True, lapack_driver="gesvd")[2][-1]
    except (np.linalg.LinAlgError, ValueError):
        return np.linalg.eigh(a.T @ a)[1][:, 0]


@lru_cache(maxsize=None)
def coupling(l1: int, l2: int, l3: int) -> np.ndarray:
    """Intertwiner with 'component' normalisation (Frobenius norm sqrt(2 l3 + 1))."""
    c = intertwiner(l1, l2, l3)
    n = float(np.linalg.norm(c))
    return c * (math.sqrt(2 * l3 + 1) / n) if n > 1e-30 else c


class Chain(NamedTuple):
    order: int           # 1, 2 or 3
    la: int              # first input degree
    lb: int              # second input degree (order >= 2)
    mid: int             # order 3: intermediate degree L1; order 2: equals l_out
    lc: int              # third input degree (order 3)
    l_out: int


def _parity(l: int) -> int:
    return 1 if l % 2 == 0 else -1


@lru_cache(maxsize=None)
def chains(lmax: int, l_out: int, order: int) -> Tuple[Chain, ...]:
    """U columns of (lmax, l_out, order) in the reference's column order."""
    basis: List[Tuple[int, int, tuple]] = [(l, _parity(l), (l,)) for l in range(lmax + 1)]
    for _ in range(2, order + 1):
        nxt = []
        for l_left, p_left, hist in basis:
            for lr in range(lmax + 1):
                for lo in range(abs(l_left - lr), l_left + lr + 1):
                    nxt.append((lo, p_left * _parity(lr), hist + (lr, lo)))
        basis = sorted(nxt, key=lambda item: (item[0], item[1]))   # stable, as the reference
    out = []
    for l, p, hist in basis:
        if l != l_out or p != _parity(l_out):
            continue
        if order == 1:
            out.append(Chain(1, hist[0], 0, l_out, 0, l_out))
        elif order == 2:
            out.append(Chain(2, hist[0], hist[1], hist[2], 0, l_out))
        else:
            out.append(Chain(3, hist[0], hist[1], hist[2], hist[3], l_out))
    return tuple(out)


def u_matrix(lmax: int, l_out: int, order: int) -> np.ndarray:
    """Dense U [(2l_out+1)?, D^order, K] assembled from the chains (for tests)."""
    dim = (lmax + 1) ** 2
    cols = []
    for ch in chains(lmax, l_out, order):
        t = np.zeros((2 * l_out + 1,) + (dim,) * order)
        if order == 1:
            for m in range(2 * l_out + 1):
                t[m, ch.la * ch.la + m] = 1.0
        elif order == 2:
            c = coupling(ch.la, ch.lb, l_out)
            sa, sb = ch.la * ch.la, ch.lb * ch.lb
            t[:, sa:sa + 2 * ch.la + 1, sb:sb + 2 * ch.lb + 1] = np.transpose(c, (2, 0, 1))
        else:
            c1 = coupling(ch.la, ch.lb, ch.mid)
            c2 = coupling(ch.mid, ch.lc, l_out)
            block = np.einsum("ija,akm->mijk", c1, c2)
            sa, sb, sc = ch.la * ch.la, ch.lb * ch.lb, ch.lc * ch.lc
            t[:, sa:sa + 2 * ch.la + 1, sb:sb + 2 * ch.lb + 1, sc:sc + 2 * ch.lc + 1] = block
        cols.append(t)
    if not cols:
        u = np.zeros((2 * l_out + 1,) + (dim,) * order + (1,))
    else:
        u = np.stack(cols, -1)
    return u[0] if l_out == 0 else u
