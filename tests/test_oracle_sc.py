"""Pin the symmetric-contraction oracle and the product's chain tables (CPU).

* U tensors: the product's chain-assembled U (ictc_o3/basis/symmetric_u.py, numpy)
  equals the oracle's restatement of the reference's coupled basis
  (ictd_irreps.py:1387-1517) for every (lmax, l_out, order) used;
* U is an intertwiner: rotating every input leg by D(R) equals rotating the output
  leg (wrong CG, index or transposition fails);
* the intertwiners match the independent polynomial CG up to sign where both exist;
* the recursion (_forward_selected_elements) equals the explicit polynomial
  sum_p W_p U_p[x,x,x] on a tiny case, and species selection picks the weight rows.
"""
import numpy as np
import pytest
import torch

from oracle import ictc_basis as B
from oracle import symmetric_contraction as O


@pytest.mark.parametrize("lmax", [1, 2, 3])
def test_product_chain_u_equals_oracle_u(lmax):
    from ictc_o3.basis import symmetric_u as S
    for lo in range(lmax + 1):
        for nu in (1, 2, 3):
            a, b = S.u_matrix(lmax, lo, nu), O.u_matrix(lmax, lo, nu).numpy()
            assert a.shape == b.shape
            assert np.abs(a - b).max() < 1e-12


def test_u_is_equivariant():
    lmax = 2
    om = torch.tensor([0.3, -0.9, 0.5], dtype=torch.float64)
    d = torch.block_diag(*[B.wigner_d(l, om) for l in range(lmax + 1)])
    for lo in (0, 1, 2):
        u = O.u_matrix(lmax, lo, 3)
        if lo == 0:
            u = u.unsqueeze(0)
        rot = torch.einsum("ai,bj,ck,mijkp->mabcp", d, d, d, u)
        dout = B.wigner_d(lo, om)
        assert (rot - torch.einsum("nm,mabcp->nabcp", dout.T, u)).abs().max() < 1e-10


@pytest.mark.parametrize("l1,l2,l3", [(1, 1, 2), (2, 2, 2), (1, 2, 3), (3, 3, 2)])
def test_intertwiner_matches_polynomial_cg_up_to_sign(l1, l2, l3):
    a = B.cg_tensor(l1, l2, l3)
    b = B.full_cg_tensor(l1, l2, l3)
    a = a / a.norm()
    assert min((a - b).abs().max(), (a + b).abs().max()) < 1e-10


def test_recursion_equals_explicit_polynomial():
    lmax, lo = 1, 1
    sc = O.SymmetricContractionOracle(3, 2, lmax, 1, 3, seed=1)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 2 * (lmax + 1) ** 2, generator=g, dtype=torch.float64)
    species = torch.tensor([0, 2, 1, 2])
    out = sc.contract(x, species, lo)
    xb = sc.input_blocks(x)                         # [N, C, D]
    expect = torch.zeros(4, 2, 3, dtype=torch.float64)
    for order in (1, 2, 3):
        u = sc.u[(lo, order)]
        w = sc.weights[(lo, order)][species]        # [N, K, C]
        if order == 1:
            expect += torch.einsum("mip,nci,npc->ncm", u, xb, w)
        elif order == 2:
            expect += torch.einsum("mijp,nci,ncj,npc->ncm", u, xb, xb, w)
        else:
            expect += torch.einsum("mijkp,nci,ncj,nck,npc->ncm", u, xb, xb, xb, w)
    assert torch.allclose(out, expect.reshape(4, -1), atol=1e-12)
