"""The HIP tensor product (through the C ABI) against vectors written by the reference's
own CPU tensor product (``tests/golden/make_tp_fixture.py``; float64 reference values,
float32 inputs here): forward, VJP to features / harmonics / gates and mixed second
derivatives in both layouts, for full path sets, a scalar-l1 set and a path subset, at the
fp32 bar (1e-5 relative to the largest reference entry)."""
import pytest
import torch

from conftest import assert_rel
from test_reference_vectors import CASES, load_case

pytestmark = pytest.mark.gpu


def _hip_op(case, layout, device):
    from ictc_o3 import EdgeTensorProduct
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    c, lin, le, lout = (int(v) for v in case["meta"])
    paths = [tuple(int(v) for v in p) for p in case["paths"]]
    tp = EdgeWeightedPathPreservingTensorProduct(c, max(lin, le, lout), allowed_paths=paths,
                                                 internal_compute_dtype=torch.float32).to(device)
    with torch.no_grad():
        tp.weight.fill_(1.)
    tp.weight.requires_grad_(False)
    return EdgeTensorProduct(tp, input_lmax=lin, edge_lmax=le, layout=layout)


@pytest.mark.parametrize("layout", ["ir_mul", "mul_ir"])
@pytest.mark.parametrize("name", CASES)
def test_hip_matches_reference_vectors(gpu, name, layout):
    print(f"reference vectors: {name} {layout}", flush=True)
    case = load_case(name)
    op = _hip_op(case, layout, gpu)
    assert [tuple(p) for p in op.paths] == [tuple(int(v) for v in p) for p in case["paths"]]
    leaves = [case[k].float().to(gpu).requires_grad_() for k in ("x", "harmonics", "gates")]
    out = op(*leaves)
    assert_rel(out, case[f"{layout}/out"], what="forward")
    grads = torch.autograd.grad(out, leaves, case["cotangent"].float().to(gpu), create_graph=True)
    for tag, g in zip(("dx", "dy", "dg"), grads):
        assert_rel(g, case[f"{layout}/{tag}"], what=tag)
    s = sum((g * case[h].float().to(gpu)).sum() for g, h in zip(grads, ("hx", "hy", "hg")))
    second = torch.autograd.grad(s, leaves, allow_unused=True)
    for tag, g, like in zip(("ddx", "ddy", "ddg"), second, leaves):
        g = torch.zeros_like(like) if g is None else g
        assert_rel(g, case[f"{layout}/{tag}"], what=tag)
