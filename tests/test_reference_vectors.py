"""The oracle against vectors written by the reference's own CPU tensor product
(``tests/golden/make_tp_fixture.py``: ``EdgeWeightedPathPreservingTensorProduct`` of
``ictc_o3/basis/ictd_irreps.py:2501-2794``, ``direction_harmonics_all`` :1113-1168 and the
packing of ``EdgeTensorProduct._pack_output``, ``ictc_o3/operators.py:107-115``; float64).

Pins what no closed form fixes: the owner's path order, ``path_offset``, the per-degree
path counts and the packed output layout in both layouts, and, beside them, the normalised
and path-scaled CG tensors, the harmonics, the forward, the VJP to features / harmonics /
gates and the mixed second derivatives (gradients of a VJP contraction), all at 1e-12.
"""
import os

import numpy as np
import pytest
import torch

from oracle import ictc_basis as B
from oracle.tensor_product import TensorProductOracle

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tp_reference_vectors.npz")
CASES = ["l222", "l333", "l033", "l123", "l333_subset"]


def load_case(name):
    data = np.load(FIXTURE)
    return {k[len(name) + 1:]: torch.from_numpy(data[k]) for k in data.files if k.startswith(name + "/")}


def case_oracle(case, layout="ir_mul"):
    c, lin, le, lout = (int(v) for v in case["meta"])
    paths = [tuple(int(v) for v in p) for p in case["paths"]]
    return TensorProductOracle(c, lin, le, lout, layout=layout, paths=paths)


@pytest.mark.parametrize("name", CASES)
def test_paths_offsets_and_cg_match_reference(name):
    case = load_case(name)
    op = case_oracle(case)
    assert op.paths == [tuple(int(v) for v in p) for p in case["paths"]]
    assert op.path_offset == case["path_offset"].tolist()
    assert [op.path_counts_by_l.get(l, 0) for l in range(op.lmax + 1)] == case["path_counts"].tolist()
    for p in range(op.num_paths):
        assert (op.cg[p] - case[f"cg{p}"]).abs().max() < 1e-12, op.paths[p]


@pytest.mark.parametrize("name", CASES)
def test_harmonics_match_reference(name):
    case = load_case(name)
    le = int(case["meta"][2])
    y = B.direction_harmonics_packed(case["directions"], le)
    assert (y - case["harmonics"]).abs().max() < 1e-12


@pytest.mark.parametrize("layout", ["ir_mul", "mul_ir"])
@pytest.mark.parametrize("name", CASES)
def test_forward_vjp_and_second_derivatives_match_reference(name, layout):
    case = load_case(name)
    op = case_oracle(case, layout)
    leaves = [case[k].clone().requires_grad_() for k in ("x", "harmonics", "gates")]
    out = op.forward(*leaves)
    assert (out - case[f"{layout}/out"]).abs().max() < 1e-12
    grads = torch.autograd.grad(out, leaves, case["cotangent"], create_graph=True)
    for tag, g in zip(("dx", "dy", "dg"), grads):
        assert (g - case[f"{layout}/{tag}"]).abs().max() < 1e-12, tag
    s = sum((g * case[h]).sum() for g, h in zip(grads, ("hx", "hy", "hg")))
    second = torch.autograd.grad(s, leaves, allow_unused=True)
    for tag, g, like in zip(("ddx", "ddy", "ddg"), second, leaves):
        g = torch.zeros_like(like) if g is None else g
        assert (g - case[f"{layout}/{tag}"]).abs().max() < 1e-12, tag
