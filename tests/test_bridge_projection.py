"""Bridge-U symmetric contraction on the CPU: the restated e3nn conventions, the folded U
tensors, and the projection of a module's U buffers onto the coupling chains the HIP kernels
evaluate (ictc_o3/ops/factorized_contraction.py; reference ops/factorized_contraction.py:51-149).

Pins:
* SU(2) Clebsch-Gordan values from standard tables and their orthogonality;
* e3nn's real coupling tensors are equivariant under the same rotation matrices that carry the
  restated e3nn harmonics (fitted from the harmonics themselves), with D_1(R) = R, the l = 1
  couplings proportional to delta and epsilon, and the harmonics' component normalisation;
* the folded bridge U equals the pure-ICTC chain U column by column up to a sign;
* projection: for U = U_chain A with a random invertible A (columns permuted and sign-flipped),
  the contraction with (U, W) equals the oracle's contraction with (U_chain, A_fit W) at 1e-12,
  and a U with a component outside the chains' span is refused by the 4e-6 gate.
"""
import math

import numpy as np
import pytest
import torch

from ictc_o3.basis import e3nn_convention as E
from ictc_o3.basis import symmetric_u as S
from ictc_o3.ops import factorized_contraction as FC
from oracle.symmetric_contraction import SymmetricContractionOracle


@pytest.mark.parametrize("args,value", [
    ((1, 1, 1, -1, 0, 0), 1 / math.sqrt(3)), ((1, 0, 1, 0, 0, 0), -1 / math.sqrt(3)),
    ((1, 1, 1, 0, 2, 1), 1 / math.sqrt(2)), ((1, 1, 1, 1, 2, 2), 1.0), ((1, 0, 1, 0, 2, 0), math.sqrt(2 / 3)),
    ((1, 1, 1, 0, 1, 1), 1 / math.sqrt(2)), ((1, 0, 1, 1, 1, 1), -1 / math.sqrt(2)),
    ((2, 0, 1, 0, 1, 0), -math.sqrt(2 / 5)), ((1, 1, 1, -1, 1, 0), 1 / math.sqrt(2))])
def test_su2_table_values(args, value):
    assert abs(E.su2_clebsch_gordan_coefficient(*args) - value) < 1e-14


@pytest.mark.parametrize("j1,j2", [(1, 1), (2, 1), (2, 3), (3, 3)])
def test_su2_orthogonality(j1, j2):
    rows = []
    for j3 in range(abs(j1 - j2), j1 + j2 + 1):
        c = E.su2_clebsch_gordan(j1, j2, j3)
        rows.extend(c[..., m] for m in range(2 * j3 + 1))
    gram = np.stack([r.ravel() for r in rows]) @ np.stack([r.ravel() for r in rows]).T
    assert np.abs(gram - np.eye(len(rows))).max() < 1e-13


def _rotation(seed):
    q, _ = np.linalg.qr(np.random.default_rng(seed).normal(size=(3, 3)))
    return q * np.sign(np.linalg.det(q))


def test_e3nn_harmonics_and_couplings_share_one_representation():
    rng = np.random.default_rng(1)
    n = rng.normal(size=(6000, 3))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    lmax = 4
    y = E.spherical_harmonics(lmax, n)
    assert np.abs(y[:, 1:4] - math.sqrt(3) * n).max() < 1e-14
    x_, y_, z_ = n.T
    s3 = math.sqrt(3)
    l2 = math.sqrt(5) * np.stack([s3 * x_ * z_, s3 * x_ * y_, y_ * y_ - 0.5 * (x_ * x_ + z_ * z_), s3 * y_ * z_,
                                  s3 / 2 * (z_ * z_ - x_ * x_)], -1)
    assert np.abs(y[:, 4:9] - l2).max() < 1e-13
    # every component has unit mean square (exact for a degree <= 2*lmax quadrature: use many points)
    assert np.abs((y ** 2).mean(0) - 1).max() < 0.06
    r = _rotation(2)
    yr = E.spherical_harmonics(lmax, n @ r.T)
    d = {}
    for l in range(lmax + 1):
        a, b = y[:, l * l:(l + 1) ** 2], yr[:, l * l:(l + 1) ** 2]
        dl = np.linalg.lstsq(a, b, rcond=None)[0].T
        assert np.abs(a @ dl.T - b).max() < 1e-11
        assert np.abs(dl @ dl.T - np.eye(2 * l + 1)).max() < 1e-11
        d[l] = dl
    assert np.abs(d[1] - r).max() < 1e-13
    for l1 in range(lmax + 1):
        for l2_ in range(lmax + 1):
            for l3 in range(abs(l1 - l2_), min(lmax, l1 + l2_) + 1):
                c = E.wigner_3j(l1, l2_, l3)
                assert abs(np.linalg.norm(c) - 1) < 1e-13
                rot = np.einsum("ijk,ia,jb,kc->abc", c, d[l1], d[l2_], d[l3])
                assert np.abs(rot - c).max() < 1e-10, (l1, l2_, l3)
    assert np.abs(E.wigner_3j(1, 1, 0)[:, :, 0] - np.eye(3) / math.sqrt(3)).max() < 1e-14
    eps = np.zeros((3, 3, 3))
    for i, j, k in ((0, 1, 2), (1, 2, 0), (2, 0, 1)):
        eps[i, j, k], eps[j, i, k] = 1, -1
    assert np.abs(np.abs(E.wigner_3j(1, 1, 1)) - np.abs(eps) / math.sqrt(6)).max() < 1e-14
    assert np.abs(E.wigner_3j(1, 1, 1) - np.sign(E.wigner_3j(1, 1, 1)[0, 1, 2]) * eps / math.sqrt(6)).max() < 1e-14


@pytest.mark.parametrize("lmax,l_out,order", [(3, 0, 3), (3, 1, 3), (2, 2, 2), (3, 1, 1), (1, 1, 3)])
def test_folded_bridge_u_is_the_chain_u_up_to_column_signs(lmax, l_out, order):
    qs = E.basis_bridge(lmax)
    ub = E.fold_u(E.u_matrix_real(lmax, l_out, order), qs, lmax, l_out, order)
    uc = S.u_matrix(lmax, l_out, order)
    assert ub.shape == uc.shape
    for k in range(ub.shape[-1]):
        a, b = ub[..., k].ravel(), uc[..., k].ravel()
        assert abs(abs(a @ b) - b @ b) < 1e-12 * max(1.0, b @ b)
        assert np.abs(a - np.sign(a @ b) * b).max() < 1e-12


def _oracle_with(u, weights, lmax, target, corr, channels, species_count):
    ref = SymmetricContractionOracle(species_count, channels, lmax, target, corr, seed=0)
    ref.u = {k: torch.as_tensor(v, dtype=torch.float64) for k, v in u.items()}
    ref.weights = {k: torch.as_tensor(v, dtype=torch.float64) for k, v in weights.items()}
    return ref


@pytest.mark.parametrize("lmax,target,corr", [(3, 1, 3), (2, 2, 3), (2, 1, 2)])
def test_projection_of_mixed_columns(lmax, target, corr):
    """U_module = U_chain A (A random, columns permuted and sign-flipped): the oracle contraction
    with the module's U and weights equals the one with the chain U and the projected weights."""
    rng = np.random.default_rng(lmax * 100 + target * 10 + corr)
    species_count, channels = 3, 5
    u_mod, w_mod, u_chain, w_chain = {}, {}, {}, {}
    for lo in range(target + 1):
        for nu in range(corr, 0, -1):
            uc = S.u_matrix(lmax, lo, nu)
            k = uc.shape[-1]
            a = rng.normal(size=(k, k)) + 3 * np.eye(k)
            a = a[:, rng.permutation(k)] * rng.choice([-1.0, 1.0], size=k)
            u_mod[(lo, nu)] = np.einsum("...p,pk->...k", uc, a)
            w_mod[(lo, nu)] = rng.normal(size=(species_count, k, channels))
            fit, rel = FC.projection(u_mod[(lo, nu)], lmax, lo, nu, 2e-11)
            assert fit is not None and rel < 1e-12
            u_chain[(lo, nu)] = uc
            w_chain[(lo, nu)] = np.einsum("pk,skc->spc", fit, w_mod[(lo, nu)])
    x = torch.randn(7, channels * (lmax + 1) ** 2, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    species = torch.tensor([0, 2, 1, 1, 0, 2, 2])
    got = _oracle_with(u_chain, w_chain, lmax, target, corr, channels, species_count).forward(x, species)
    expect = _oracle_with(u_mod, w_mod, lmax, target, corr, channels, species_count).forward(x, species)
    assert (got - expect).abs().max() / expect.abs().max() < 1e-12


def test_gate_refuses_components_outside_the_chain_span():
    rng = np.random.default_rng(5)
    uc = S.u_matrix(3, 1, 2)
    noise = rng.normal(size=uc.shape) * 1e-3 * np.abs(uc).max()
    fit, rel = FC.projection(uc + noise, 3, 1, 2, 4e-6)
    assert fit is None and rel > 4e-6
    fit, rel = FC.projection(uc + noise * 1e-7, 3, 1, 2, 4e-6)      # float32-level noise passes
    assert fit is not None


def test_module_plan_on_cpu_matches_the_dense_contraction():
    """The bridge module's own buffers and weights through the projection plan (CPU tensors: the
    plan is host arithmetic) against the oracle recursion on the module's U."""
    from ictc_o3.ops.symmetric_contraction import ICTDBridgeUSymmetricContractionSO3
    torch.manual_seed(0)
    mod = ICTDBridgeUSymmetricContractionSO3(num_elements=3, channels=4, lmax=2, target_lmax=1, correlation=3)
    names = dict(mod.named_buffers())
    assert "basis_bridge.q_2" in names and "symmetric_contractions.contractions.1.U_matrix_3" in names
    assert "symmetric_contractions.contractions.0.weights_0_zeroed" in names
    params = [n for n, _ in mod.named_parameters()]
    assert params == ["symmetric_contractions.contractions.0.weights_max",
                      "symmetric_contractions.contractions.0.weights.0",
                      "symmetric_contractions.contractions.0.weights.1",
                      "symmetric_contractions.contractions.1.weights_max",
                      "symmetric_contractions.contractions.1.weights.0",
                      "symmetric_contractions.contractions.1.weights.1"]
    x = torch.randn(6, 4 * 9, dtype=torch.float64)
    table = mod.weight_table(x.float())
    species = torch.tensor([0, 1, 2, 2, 1, 0])
    u_mod = {(lo, nu): con.U_tensors(nu).double() for lo, con in enumerate(mod.symmetric_contractions.contractions)
             for nu in range(1, 4)}
    w_mod = {(lo, nu): w.detach().double() for lo, con in enumerate(mod.symmetric_contractions.contractions)
             for nu, w in zip((3, 2, 1), con.columns())}
    expect = _oracle_with(u_mod, w_mod, 2, 1, 3, 4, 3).forward(x, species)
    u_chain, w_chain, col = {}, {}, 0
    for lo in range(2):
        for nu in (3, 2, 1):
            uc = S.u_matrix(2, lo, nu)
            u_chain[(lo, nu)] = uc
            w_chain[(lo, nu)] = table[:, col:col + uc.shape[-1]].detach()
            col += uc.shape[-1]
    got = _oracle_with(u_chain, w_chain, 2, 1, 3, 4, 3).forward(x, species)
    assert (got - expect).abs().max() / expect.abs().max() < 2e-6      # float32 U buffers
