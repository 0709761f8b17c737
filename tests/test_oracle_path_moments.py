"""Pin the oracle's output normalisation against its definition (CPU, float64, exact).

The reference scales each path's CG tensor to 'component' normalisation
(||C||_F = sqrt(2 l3 + 1), ``ictd_irreps.py:136-142``) and then by the 'element' path
normalisation, 1 / sqrt(sum of num_elements over the paths into the same l3) with
num_elements = 1 for the channelwise owner (``ictd_irreps.py:101-133``, owner set-up
``:2183-2188``, applied in ``_get_cg_list`` ``:2218-2236``).  These are e3nn's
definitions, and they are statements about second moments: for features with iid
unit-variance components, harmonics of a uniformly random direction and unit gates,

* every output component k of path p has E[out_{p,k}^2] = 1 / n(l3),
  n(l3) = the number of the owner's paths into degree l3;
* so the paths into each l3 sum to a unit second moment per component.

The moments are evaluated exactly, not sampled: the output is linear in the features,
so E_x[out_k^2] is the sum of the squared responses to the unit vectors e_i (channel c
carries e_c in every degree); the direction average is a product Gauss-Legendre (cos
theta) x uniform (phi) quadrature that is exact for polynomials of degree <= 15 on the
sphere (the integrand has degree 2 * edge_lmax).  A wrong path scale (1/n, n^-1/4,
none, 1/sqrt(2 l3 + 1)) or a wrong CG normalisation ('norm': ||C||_F = 1) fails it;
``test_planted_scale_errors_fail`` plants each of them in the oracle.
"""
import math

import numpy as np
import pytest
import torch

import oracle.ictc_basis as B
from oracle.tensor_product import TensorProductOracle, enumerate_paths


def _sphere_rule(m: int = 8, k: int = 16):
    """Directions and weights (summing to 1) of a product rule on the unit sphere."""
    z, wz = np.polynomial.legendre.leggauss(m)
    phi = 2.0 * math.pi * np.arange(k) / k
    zz, pp = np.meshgrid(z, phi, indexing="ij")
    s = np.sqrt(1.0 - zz ** 2)
    n = np.stack([s * np.cos(pp), s * np.sin(pp), zz], -1).reshape(-1, 3)
    w = (wz[:, None] / (2.0 * k) * np.ones((1, k))).reshape(-1)
    return torch.from_numpy(n), torch.from_numpy(w)


def path_component_moments(op: TensorProductOracle):
    """E[out_{p,k}^2] per path p (list of [2 l3 + 1] tensors) for iid unit-variance
    features, unit gates and a uniformly random direction, evaluated exactly."""
    n, w = _sphere_rule()
    q = n.shape[0]
    c = op.channels
    assert c >= 2 * op.input_lmax + 1
    blocks = {}
    for l in range(op.input_lmax + 1):
        v = torch.zeros(q, c, 2 * l + 1, dtype=torch.float64)
        for i in range(2 * l + 1):
            v[:, i, i] = 1.0            # channel i carries the unit vector e_i
        blocks[l] = v
    x = op.pack_input(blocks)
    y = B.direction_harmonics_packed(n, op.edge_lmax)
    gates = torch.ones(q, op.gate_width, dtype=torch.float64)
    out = op.unpack_output(op.forward(x, y, gates))
    moments = []
    for p, (_, _, l3) in enumerate(op.paths):
        c0 = op.path_offset[p] * c
        resp = out[l3][:, c0:c0 + c, :]                 # [q, channel = e_i, k]
        moments.append(torch.einsum("q,qck->k", w, resp ** 2))
    return moments


def _check_moments(op: TensorProductOracle, tol: float = 1e-12):
    moments = path_component_moments(op)
    counts = {}
    for _, _, l3 in op.paths:
        counts[l3] = counts.get(l3, 0) + 1
    for p, (l1, l2, l3) in enumerate(op.paths):
        err = (moments[p] - 1.0 / counts[l3]).abs().max().item()
        assert err <= tol, f"path {(l1, l2, l3)}: second moment off 1/{counts[l3]} by {err:.3e}"
    for l3, cnt in counts.items():
        total = sum(moments[p] for p, path in enumerate(op.paths) if path[2] == l3)
        err = (total - 1.0).abs().max().item()
        assert err <= tol * cnt, f"l3 = {l3}: paths sum to second moment {total.tolist()}"


@pytest.mark.parametrize("lin,le,lout", [(2, 2, 2), (3, 3, 3), (0, 3, 3), (1, 2, 3), (3, 1, 0), (4, 4, 4)])
def test_path_second_moments(lin, le, lout):
    op = TensorProductOracle(2 * lin + 1, lin, le, lout)
    _check_moments(op)


def test_path_second_moments_on_a_path_subset():
    """n(l3) counts only the owner's paths (the scale follows its path list)."""
    full = enumerate_paths(3, 3, 3)
    subset = [p for i, p in enumerate(full) if i % 3 != 1]
    op = TensorProductOracle(7, 3, 3, 3, paths=subset)
    assert op.num_paths == len(subset) < len(full)
    _check_moments(op)


def test_quadrature_is_exact_on_the_harmonics():
    """The rule integrates the harmonics' Gram matrix to the identity (component
    normalisation and orthogonality) and odd moments to zero."""
    n, w = _sphere_rule()
    y = B.direction_harmonics_packed(n, 4)
    gram = torch.einsum("q,qa,qb->ab", w, y, y)
    assert (gram - torch.eye(gram.shape[0], dtype=torch.float64)).abs().max() < 1e-13
    assert abs(float((w * n[:, 0] ** 3 * n[:, 2]).sum())) < 1e-15


_PLANTED = {
    "scale 1/n": lambda cnt, l3: 1.0 / cnt,
    "scale n^-1/4": lambda cnt, l3: cnt ** -0.25,
    "no scale": lambda cnt, l3: 1.0,
    "scale 1/sqrt(2 l3 + 1)": lambda cnt, l3: 1.0 / math.sqrt(2 * l3 + 1),
}


@pytest.mark.parametrize("name", sorted(_PLANTED))
def test_planted_scale_errors_fail(monkeypatch, name):
    rule = _PLANTED[name]

    def wrong(paths):
        counts = {}
        for p in paths:
            counts[p[2]] = counts.get(p[2], 0) + 1
        return [rule(counts[p[2]], p[2]) for p in paths]

    monkeypatch.setattr(B, "path_normalisation_scales", wrong)
    op = TensorProductOracle(7, 3, 3, 3)
    with pytest.raises(AssertionError):
        _check_moments(op)


def test_planted_cg_normalisation_error_fails(monkeypatch):
    monkeypatch.setattr(B, "cg_component_normalised", lambda c, l3: c / c.norm())
    op = TensorProductOracle(7, 3, 3, 3)
    with pytest.raises(AssertionError):
        _check_moments(op)
