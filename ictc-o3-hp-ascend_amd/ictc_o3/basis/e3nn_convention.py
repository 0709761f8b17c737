"""The e3nn conventions behind the reference's bridge-U symmetric contraction (host side, float64).

The reference builds its shipped contraction's U tensors with e3nn (pinned
``e3nn>=0.4.4,<0.6``, ``pyproject.toml:12``), which is not available here: its real-basis
Wigner-3j symbols couple the MACE polynomial (``ictc_o3/basis/_mace_cg.py:39-190``,
``_wigner_nj`` / ``U_matrix_real``) and its real spherical harmonics fix the per-degree basis
bridge to the ICTC basis (``ictc_o3/ops/symmetric_contraction.py:24-60``).  This module
restates e3nn's published algorithm for both:

* ``su2_clebsch_gordan``: Clebsch-Gordan coefficients <j1 m1 j2 m2 | j3 m3> (Condon-Shortley
  phase) from Racah's closed formula, exact in rational arithmetic;
* ``change_basis_real_to_complex``: e3nn's unitary map between the complex and the real
  spherical-harmonic bases, with its extra factor (-i)^l that makes the coupling real;
* ``wigner_3j``: e3nn's real coupling tensor ``_so3_clebsch_gordan`` = the SU(2) coefficients
  carried into the real basis of each leg, Frobenius-normalised;
* ``spherical_harmonics``: e3nn's real harmonics in its (x, y, z) input order with the y axis
  as polar axis, 'component' normalisation (every component has unit mean square on the
  sphere);
* ``coupled_paths`` / ``u_matrix_real``: the MACE generalized coupling of ``_wigner_nj`` /
  ``U_matrix_real`` (``ictc_o3/basis/_mace_cg.py:39-190``) on these symbols;
* ``basis_bridge``: the per-degree orthogonal map Q_l of ``SO3ToE3NNBasisBridge``
  (``ictc_o3/ops/symmetric_contraction.py:41-60``) with Y_ictc_l Q_l = Y_e3nn_l.

Which sign each e3nn tensor carries cannot be checked against e3nn itself here; the tests
pin what the mathematics fixes (orthogonality and closed-form entries of the coefficients,
equivariance of the coupling tensors and of the harmonics under one and the same rotation
representation, the harmonics' normalisation).  A reference checkpoint carries its own U
buffers and basis bridge, which the HIP contraction consumes as they are.
"""
from __future__ import annotations

import math
from fractions import Fraction
from functools import lru_cache

import numpy as np


def _fact(n: int) -> int:
    return math.factorial(n)


def su2_clebsch_gordan_coefficient(j1: int, m1: int, j2: int, m2: int, j3: int, m3: int) -> float:
    """<j1 m1 j2 m2 | j3 m3> for integer spins (Racah's formula, Condon-Shortley phase)."""
    if m3 != m1 + m2 or not abs(j1 - j2) <= j3 <= j1 + j2:
        return 0.0
    if abs(m1) > j1 or abs(m2) > j2 or abs(m3) > j3:
        return 0.0
    pref = Fraction((2 * j3 + 1) * _fact(j3 + j1 - j2) * _fact(j3 - j1 + j2) * _fact(j1 + j2 - j3),
                    _fact(j1 + j2 + j3 + 1))
    pref *= (_fact(j3 + m3) * _fact(j3 - m3) * _fact(j1 - m1) * _fact(j1 + m1) * _fact(j2 - m2)
             * _fact(j2 + m2))
    total = Fraction(0)
    for k in range(0, j1 + j2 - j3 + 1):
        den = [k, j1 + j2 - j3 - k, j1 - m1 - k, j2 + m2 - k, j3 - j2 + m1 + k, j3 - j1 - m2 + k]
        if min(den) < 0:
            continue
        term = Fraction(1, math.prod(_fact(d) for d in den))
        total += -term if k % 2 else term
    return float(total) * math.sqrt(float(pref)) if total else 0.0


@lru_cache(maxsize=None)
def su2_clebsch_gordan(j1: int, j2: int, j3: int) -> np.ndarray:
    """C[j1 + m1, j2 + m2, j3 + m3] = <j1 m1 j2 m2 | j3 m3>."""
    c = np.zeros((2 * j1 + 1, 2 * j2 + 1, 2 * j3 + 1))
    for m1 in range(-j1, j1 + 1):
        for m2 in range(-j2, j2 + 1):
            m3 = m1 + m2
            if abs(m3) <= j3:
                c[j1 + m1, j2 + m2, j3 + m3] = su2_clebsch_gordan_coefficient(j1, m1, j2, m2, j3, m3)
    return c


@lru_cache(maxsize=None)
def change_basis_real_to_complex(l: int) -> np.ndarray:
    """e3nn's [2l+1, 2l+1] complex change of basis between real and complex harmonics of degree
    l, including its global factor (-i)^l."""
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    r = 1.0 / math.sqrt(2.0)
    for m in range(-l, 0):
        q[l + m, l + abs(m)] = r
        q[l + m, l - abs(m)] = -1j * r
    q[l, l] = 1.0
    for m in range(1, l + 1):
        q[l + m, l + abs(m)] = (-1) ** m * r
        q[l + m, l - abs(m)] = 1j * (-1) ** m * r
    return (-1j) ** l * q


@lru_cache(maxsize=None)
def wigner_3j(l1: int, l2: int, l3: int) -> np.ndarray:
    """e3nn's real coupling tensor [2l1+1, 2l2+1, 2l3+1] (unit Frobenius norm; zero outside the
    triangle): C[j, l, m] = sum_{i,k,n} Q1[i, j] Q2[k, l] conj(Q3[n, m]) C_su2[i, k, n]."""
    if not abs(l1 - l2) <= l3 <= l1 + l2:
        return np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    q1, q2, q3 = (change_basis_real_to_complex(l) for l in (l1, l2, l3))
    c = np.einsum("ij,kl,nm,ikn->jlm", q1, q2, np.conj(q3), su2_clebsch_gordan(l1, l2, l3).astype(np.complex128))
    if np.abs(c.imag).max() > 1e-9:
        raise ArithmeticError("the real-basis coupling tensor is not real")
    c = c.real
    return c / np.linalg.norm(c)


def spherical_harmonics(lmax: int, directions: np.ndarray) -> np.ndarray:
    """e3nn's real spherical harmonics Y_0 | Y_1 | ... | Y_lmax of directions [n, 3] in its
    (x, y, z) input order (y is the polar axis), 'component' normalisation: [n, (lmax+1)^2].

    Y_0 = 1, Y_1 = sqrt(3) (x, y, z), and for l >= 2 the polynomial e3nn generates its
    harmonics from, Y_l = c_l * wigner_3j(l-1, 1, l)[Y_{l-1}, Y_1] with c_l > 0 fixing the
    normalisation (sum_m Y_lm^2 = 2l + 1 on the unit sphere); at l = 2 this is e3nn's
    sqrt(5) * (sqrt(3) xz, sqrt(3) xy, y^2 - (x^2 + z^2)/2, sqrt(3) yz, sqrt(3)/2 (z^2 - x^2))."""
    d = np.asarray(directions, dtype=np.float64)
    d = d / np.linalg.norm(d, axis=-1, keepdims=True)
    blocks = [np.ones(d.shape[:-1] + (1,))]
    if lmax >= 1:
        blocks.append(math.sqrt(3.0) * d)
    probe = np.array([[0.0, 1.0, 0.0]])
    probe_blocks = [np.ones((1, 1)), math.sqrt(3.0) * probe]
    for l in range(2, lmax + 1):
        w = wigner_3j(l - 1, 1, l)
        raw = np.einsum("ijk,...i,...j->...k", w, blocks[-1], blocks[1])
        raw_probe = np.einsum("ijk,...i,...j->...k", w, probe_blocks[-1], probe_blocks[1])
        c = math.sqrt((2 * l + 1) / float((raw_probe ** 2).sum()))
        blocks.append(c * raw)
        probe_blocks.append(c * raw_probe)
    return np.concatenate(blocks[:lmax + 1], -1)


def _parity(l: int) -> int:
    return 1 if l % 2 == 0 else -1


@lru_cache(maxsize=None)
def coupled_paths(lmax: int, order: int):
    """_wigner_nj([irreps] * order) for irreps = 0e + 1o + ... + lmax (one copy of each natural
    parity degree): a tuple of (l_out, parity, tensor [2 l_out + 1, D, ..., D]) over every
    coupling path, sorted by (l_out, parity) with ties kept in enumeration order."""
    dim = (lmax + 1) ** 2
    eye = np.eye(dim)
    if order == 1:
        return tuple((l, _parity(l), eye[l * l:(l + 1) ** 2]) for l in range(lmax + 1))
    out = []
    for l_left, p_left, c_left in coupled_paths(lmax, order - 1):
        for l_right in range(lmax + 1):
            start = l_right * l_right
            for l_out in range(abs(l_left - l_right), l_left + l_right + 1):
                w = wigner_3j(l_out, l_left, l_right) * math.sqrt(2 * l_out + 1)
                c = np.einsum("jk,ijl->ikl", c_left.reshape(2 * l_left + 1, -1), w)
                c = c.reshape((2 * l_out + 1,) + (dim,) * (order - 1) + (2 * l_right + 1,))
                e = np.zeros((2 * l_out + 1,) + (dim,) * order)
                e[..., start:start + 2 * l_right + 1] = c
                out.append((l_out, p_left * _parity(l_right), e))
    return tuple(sorted(out, key=lambda item: (item[0], item[1])))


def u_matrix_real(lmax: int, l_out: int, order: int) -> np.ndarray:
    """U_matrix_real(irreps_in, irrep l_out with natural parity, order)[-1]: the paths with that
    output irrep stacked on a last axis, the output axis dropped for l_out = 0:
    [(2 l_out + 1,) D^order, K] (zeros with K = 1 when no path reaches it)."""
    dim = (lmax + 1) ** 2
    cols = [t for l, p, t in coupled_paths(lmax, order) if l == l_out and p == _parity(l_out)]
    if not cols:
        shape = ((2 * l_out + 1,) if l_out else ()) + (dim,) * order + (1,)
        return np.zeros(shape)
    u = np.stack(cols, -1)
    return u[0] if l_out == 0 else u


def basis_bridge(lmax: int, num_samples: int = 8192, seed: int = 20260426):
    """[Q_0, ..., Q_lmax]: orthogonal Procrustes fits of the ICTC harmonics onto e3nn's on seeded
    random unit directions (Y_ictc_l Q_l ~= Y_e3nn_l; SVD of Y_ictc_l^T Y_e3nn_l = U S V^T,
    Q_l = U V^T)."""
    import torch
    from .ictd_irreps import harmonics_tables
    gen = torch.Generator(device="cpu")
    gen.manual_seed(int(seed))
    dirs = torch.randn(int(num_samples), 3, generator=gen, dtype=torch.float64)
    dirs = (dirs / dirs.norm(dim=-1, keepdim=True).clamp_min(1e-12)).numpy()
    y_e3nn = spherical_harmonics(lmax, dirs)
    qs = []
    for l in range(lmax + 1):
        mons, proj, scale = harmonics_tables(l)
        mono = np.stack([dirs[:, 0] ** a * dirs[:, 1] ** b * dirs[:, 2] ** c for a, b, c in mons], -1)
        y_ictc = scale * mono @ proj
        u, _, vh = np.linalg.svd(y_ictc.T @ y_e3nn[:, l * l:(l + 1) ** 2])
        qs.append(u @ vh)
    return qs


def fold_u(u: np.ndarray, qs, lmax: int, l_out: int, order: int) -> np.ndarray:
    """The bridge-U tensor in the ICTC basis (``_transform_u_tensor``,
    ``ictc_o3/ops/symmetric_contraction.py:119-158``): every input leg mapped by the block
    diagonal of Q_0..Q_lmax and the output leg by Q_{l_out}."""
    dim = (lmax + 1) ** 2
    q_in = np.zeros((dim, dim))
    for l in range(lmax + 1):
        q_in[l * l:(l + 1) ** 2, l * l:(l + 1) ** 2] = qs[l]
    result = u if l_out == 0 else np.tensordot(qs[l_out], u, axes=([1], [0]))
    first = 0 if l_out == 0 else 1
    for axis in range(first, first + order):
        result = np.moveaxis(np.tensordot(q_in, result, axes=([1], [axis])), 0, axis)
    return result
