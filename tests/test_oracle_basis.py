"""Pin the oracle's basis, CG tensors and direction harmonics (CPU).

Pins (each chosen so a plausible mistake fails one of them):
* the 13 frozen basis fixtures carry the reference's SHA-256 pins;
* CG: equivariance under random rotations (wrong index/transposed operand fails),
  Frobenius norm before/after 'component' normalisation, exact zeros on
  parity-forbidden paths, l1=0 couplings are scaled identities
  (reference ictd_irreps.py:2550-2568), and agreement up to sign with the
  independent null-space intertwiner (ictd_irreps.py:1304-1374);
* CG sign and size in closed form: contracting a path's coupling with the harmonics of one
  direction gives sum_ij C[i,j,k] Y_l1(n)_i Y_l2(n)_j = c Y_l3(n)_k with
  c = +sqrt((2l1+1)(2l2+1)) |(l1 l2 l3; 0 0 0)| (the Gaunt coefficient of component-normalised
  harmonics; the product of Legendre polynomials has non-negative Legendre coefficients, so a
  coupling built from polynomial products is positive), for every natural-parity path;
* Y: Y_0 = 1, Y_1 = sqrt(3) * (z, y, x) (closed form of the l=1 basis),
  unit mean square per component on the sphere, rotation covariance;
* the product's host constants (CG, harmonics tables, path plans) equal the
  oracle's.
"""
import math

import numpy as np
import pytest
import torch

from oracle import ictc_basis as B
from oracle.tensor_product import TensorProductOracle, enumerate_paths


def _rotation(seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(3, generator=g, dtype=torch.float64)


def test_basis_fixture_sha_pins():
    for l in range(13):
        b = B.harmonic_basis(l)
        assert b.shape == (B.sym_dim(l), 2 * l + 1)


def test_basis_is_gram_orthonormal_and_harmonic():
    # B_l^T G_l B_l = I (orthonormal in the invariant metric), and every column is
    # harmonic: the Laplacian annihilates it.
    for l in range(7):
        b, g = B.harmonic_basis(l), B.gram_gaussian(l)
        assert torch.allclose(b.T @ g @ b, torch.eye(2 * l + 1, dtype=torch.float64), atol=1e-10)
        if l >= 2:
            counts, lower = B.counts_list(l), {t: i for i, t in enumerate(B.counts_list(l - 2))}
            lap = torch.zeros(len(lower), len(counts), dtype=torch.float64)
            for col, (a, bb, c) in enumerate(counts):
                if a >= 2:
                    lap[lower[(a - 2, bb, c)], col] += a * (a - 1)
                if bb >= 2:
                    lap[lower[(a, bb - 2, c)], col] += bb * (bb - 1)
                if c >= 2:
                    lap[lower[(a, bb, c - 2)], col] += c * (c - 1)
            assert (lap @ b).abs().max() < 1e-10


@pytest.mark.parametrize("l1,l2,l3", [(1, 1, 0), (1, 1, 2), (2, 2, 2), (3, 3, 2), (1, 2, 3), (2, 3, 3),
                                      (3, 3, 6), (2, 2, 4), (0, 3, 3), (3, 1, 2), (4, 4, 4), (5, 3, 6),
                                      (6, 6, 6)])
def test_cg_equivariant(l1, l2, l3):
    c = B.cg_tensor(l1, l2, l3)
    for seed in (1, 2):
        om = _rotation(seed)
        d1, d2, d3 = B.wigner_d(l1, om), B.wigner_d(l2, om), B.wigner_d(l3, om)
        lhs = torch.einsum("ia,jb,ijk->abk", d1, d2, c)
        rhs = torch.einsum("abk,ck->abc", c, d3)
        assert (lhs - rhs).abs().max() < 1e-12 * max(1.0, c.abs().max().item())


def test_cg_forbidden_paths_are_zero_and_normalisation():
    for l1 in range(7):
        for l2 in range(7):
            for l3 in range(7):
                c = B.cg_tensor(l1, l2, l3)
                ok = abs(l1 - l2) <= l3 <= l1 + l2 and (l1 + l2 + l3) % 2 == 0
                if not ok:
                    assert c.abs().max() == 0
                else:
                    n = B.cg_component_normalised(c, l3)
                    assert abs(n.norm().item() - math.sqrt(2 * l3 + 1)) < 1e-12


def test_cg_scalar_input_is_scaled_identity():
    for l in range(4):
        c = B.cg_component_normalised(B.cg_tensor(0, l, l), l)[0]
        assert torch.allclose(c, torch.eye(2 * l + 1, dtype=torch.float64), atol=1e-12)


@pytest.mark.parametrize("l1,l2,l3", [(1, 1, 2), (2, 2, 2), (1, 2, 3), (3, 3, 4), (2, 3, 1)])
def test_cg_matches_nullspace_intertwiner_up_to_sign(l1, l2, l3):
    c = B.cg_tensor(l1, l2, l3)
    f = B.full_cg_tensor(l1, l2, l3)
    c = c / c.norm()
    sign = torch.sign((c * f).sum())
    assert (c - sign * f).abs().max() < 1e-9


def _wigner_3j_000(l1, l2, l3):
    """(l1 l2 l3; 0 0 0) in closed form (Racah): zero for odd l1 + l2 + l3."""
    big = l1 + l2 + l3
    if big % 2:
        return 0.0
    g, f = big // 2, math.factorial
    return ((-1) ** g * math.sqrt(f(big - 2 * l1) * f(big - 2 * l2) * f(big - 2 * l3) / f(big + 1))
            * f(g) / (f(g - l1) * f(g - l2) * f(g - l3)))


@pytest.mark.parametrize("source", ["oracle", "product"])
def test_cg_sign_and_size_closed_form(source):
    from ictc_o3.basis import ictd_irreps as P
    g = torch.Generator().manual_seed(11)
    n = torch.nn.functional.normalize(torch.randn(64, 3, generator=g, dtype=torch.float64), dim=-1)
    ys = B.direction_harmonics_all(n, 6)
    checked = 0
    for l1 in range(7):          # every triple the kernels use (all degrees <= 6)
        for l2 in range(7):
            for l3 in range(abs(l1 - l2), min(l1 + l2, 6) + 1):
                if (l1 + l2 + l3) % 2:
                    continue
                raw = (B.cg_tensor(l1, l2, l3) if source == "oracle"
                       else torch.from_numpy(P.coupling_tensor(l1, l2, l3)))
                c = B.cg_component_normalised(raw, l3)
                f = torch.einsum("ijk,ni,nj->nk", c, ys[l1], ys[l2])
                want = math.sqrt((2 * l1 + 1) * (2 * l2 + 1)) * abs(_wigner_3j_000(l1, l2, l3))
                assert want > 0
                assert (f - want * ys[l3]).abs().max() < 1e-12 * max(1.0, float(ys[l3].abs().max())) * 50, \
                    (l1, l2, l3)
                checked += 1
    assert checked == 106


def test_harmonics_closed_forms_and_normalisation():
    g = torch.Generator().manual_seed(3)
    n = torch.nn.functional.normalize(torch.randn(400000, 3, generator=g, dtype=torch.float64), dim=-1)
    ys = B.direction_harmonics_all(n, 4)
    assert torch.equal(ys[0], torch.ones(400000, 1, dtype=torch.float64))
    assert torch.allclose(ys[1], math.sqrt(3) * n.flip(-1), atol=1e-14)
    # exact sphere mean square of each component = 1, checked against a
    # quasi-uniform Monte Carlo estimate (400k samples: ~0.5% noise)
    for l in range(1, 5):
        ms = (ys[l] ** 2).mean(0)
        assert (ms - 1).abs().max() < 0.02
        # and the exact trace identity the scale is defined by
        assert abs(ms.mean().item() - 1) < 0.01


def test_harmonics_rotation_covariant():
    g = torch.Generator().manual_seed(4)
    n = torch.nn.functional.normalize(torch.randn(9, 3, generator=g, dtype=torch.float64), dim=-1)
    om = _rotation(5)
    flip = torch.eye(3, dtype=torch.float64).flip(0)
    rot = flip @ B.wigner_d(1, om) @ flip  # D_1 acts on (z,y,x)
    assert torch.allclose(rot @ rot.T, torch.eye(3, dtype=torch.float64), atol=1e-12)
    y0, y1 = B.direction_harmonics_all(n, 4), B.direction_harmonics_all(n @ rot.T, 4)
    for l in range(5):
        assert (y1[l] - y0[l] @ B.wigner_d(l, om).T).abs().max() < 1e-12


def test_path_enumeration_sizes():
    # closed counts: C64/L2 -> 11 paths, C128/L3 -> 23 paths, 439 bond entries, 99 output comps
    p2, p3 = enumerate_paths(2, 2, 2), enumerate_paths(3, 3, 3)
    assert len(p2) == 11 and len(p3) == 23
    assert sum((2 * i + 1) * (2 * k + 1) for i, _, k in p3) == 439
    assert sum(2 * k + 1 for *_, k in p3) == 99
    assert TensorProductOracle(64, 2, 2).output_width == 2240
    assert TensorProductOracle(128, 3, 3).output_width == 12672


def test_product_host_constants_match_oracle():
    from ictc_o3.basis import ictd_irreps as P
    for l1 in range(7):
        for l2 in range(7):
            for l3 in range(abs(l1 - l2), min(l1 + l2, 6) + 1):
                assert np.abs(P.coupling_tensor(l1, l2, l3) - B.cg_tensor(l1, l2, l3).numpy()).max() < 1e-12
    for l in range(6):
        mons, proj, scale = P.harmonics_tables(l)
        assert mons == B.counts_list(l)
        assert abs(scale - B.direction_component_scale(l)) < 1e-12
        _, coefs = B._monomial_exps_coefs(l)
        assert np.abs(proj - (coefs[:, None] * B.direction_projection(l)).numpy()).max() < 1e-12


@pytest.mark.parametrize("lin,le,lout", [(2, 2, 2), (3, 3, 3), (0, 3, 3), (1, 2, 3), (3, 1, 0)])
def test_product_path_plan_matches_oracle(lin, le, lout):
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    ref = TensorProductOracle(16, lin, le, lout)
    paths = enumerate_paths(lin, le, lout)
    mod = EdgeWeightedPathPreservingTensorProduct(16, max(lin, le, lout), allowed_paths=paths)
    assert [tuple(p) for p in mod.paths] == ref.paths
    assert mod.path_offset == ref.path_offset
    assert mod.path_counts_by_l == ref.path_counts_by_l
    scales = B.path_normalisation_scales(ref.paths)
    assert np.allclose(mod.path_scales, scales)
