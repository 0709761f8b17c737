"""Pin the oracle's tensor product and graph message (CPU, float64).

* brute force: the grouped projector forward equals a direct quadruple loop
  over (path, i, j, k) with the normalised CG on tiny inputs;
* O(3) covariance: rotating x and the edge direction rotates each output block;
* trilinearity in (x, Y, gates) and the packed<->dict layout round trips;
* gradcheck / gradgradcheck of the autograd derivatives used as VJP references;
* graph message equals an explicit per-edge loop; empty graphs give zeros that
  keep the graph live (reference tensor_product.py:196-199).
"""
import math

import pytest
import torch

from oracle import ictc_basis as B
from oracle.tensor_product import TensorProductOracle


def _inputs(op, rows, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, op.input_width, generator=g, dtype=dtype)
    n = torch.nn.functional.normalize(torch.randn(rows, 3, generator=g, dtype=torch.float64), dim=-1)
    y = B.direction_harmonics_packed(n, op.edge_lmax).to(dtype)
    gates = torch.randn(rows, op.gate_width, generator=g, dtype=dtype) / math.sqrt(op.num_paths)
    return x, y, gates, n


@pytest.mark.parametrize("lin,le,lout,layout", [(2, 2, 2, "ir_mul"), (3, 3, 3, "ir_mul"),
                                                (1, 2, 3, "mul_ir"), (0, 3, 3, "ir_mul")])
def test_forward_matches_brute_force(lin, le, lout, layout):
    op = TensorProductOracle(3, lin, le, lout, layout=layout)
    x, y, gates, _ = _inputs(op, 5, 0)
    out = op.unpack_output(op.forward(x, y, gates))
    xb, yb = op.blocks(x), op.harmonics(y)
    g3 = gates.reshape(5, op.num_paths, 3)
    scales = B.path_normalisation_scales(op.paths)
    for p, (l1, l2, l3) in enumerate(op.paths):
        c = B.cg_component_normalised(B.cg_tensor(l1, l2, l3), l3) * scales[p]
        expect = torch.zeros(5, 3, 2 * l3 + 1, dtype=torch.float64)
        for e in range(5):
            for ch in range(3):
                for i in range(2 * l1 + 1):
                    for j in range(2 * l2 + 1):
                        for k in range(2 * l3 + 1):
                            expect[e, ch, k] += xb[l1][e, ch, i] * yb[l2][e, 0, j] * c[i, j, k]
        expect = expect * g3[:, p, :, None]
        c0 = op.path_offset[p] * 3
        assert torch.allclose(out[l3][:, c0:c0 + 3], expect, atol=1e-12)


@pytest.mark.parametrize("lin,le,lout", [(2, 2, 2), (3, 3, 3)])
def test_forward_rotation_covariant(lin, le, lout):
    op = TensorProductOracle(4, lin, le, lout)
    x, y, gates, n = _inputs(op, 6, 1)
    om = torch.tensor([0.4, -1.3, 0.2], dtype=torch.float64)
    flip = torch.eye(3, dtype=torch.float64).flip(0)
    rot = flip @ B.wigner_d(1, om) @ flip
    xb = op.blocks(x)
    xr = op.pack_input({l: xb[l] @ B.wigner_d(l, om).T for l in xb})
    yr = B.direction_harmonics_packed(n @ rot.T, le)
    out0, out1 = op.unpack_output(op.forward(x, y, gates)), op.unpack_output(op.forward(xr, yr, gates))
    for l in out0:
        assert torch.allclose(out1[l], out0[l] @ B.wigner_d(l, om).T, atol=1e-11)


def test_forward_trilinear_and_layout_roundtrip():
    op = TensorProductOracle(5, 2, 2, 2)
    x, y, g, _ = _inputs(op, 4, 2)
    x2, y2, g2, _ = _inputs(op, 4, 3)
    a, b = 0.7, -1.9
    f = op.forward
    assert torch.allclose(f(a * x + b * x2, y, g), a * f(x, y, g) + b * f(x2, y, g), atol=1e-12)
    assert torch.allclose(f(x, a * y + b * y2, g), a * f(x, y, g) + b * f(x, y2, g), atol=1e-12)
    assert torch.allclose(f(x, y, a * g + b * g2), a * f(x, y, g) + b * f(x, y, g2), atol=1e-12)
    out = f(x, y, g)
    assert torch.equal(op.pack_output(op.unpack_output(out)), out)
    assert torch.equal(op.pack_input(op.blocks(x)), x)


def test_gradcheck_and_gradgradcheck():
    op = TensorProductOracle(2, 2, 2, 2)
    x, y, g, _ = _inputs(op, 3, 4)
    args = tuple(t.clone().requires_grad_() for t in (x, y, g))
    assert torch.autograd.gradcheck(op.forward, args)
    assert torch.autograd.gradgradcheck(op.forward, args)


def test_graph_message_matches_edge_loop_and_empty_graph():
    op = TensorProductOracle(3, 2, 2, 2)
    nodes, edges = 6, 14
    gen = torch.Generator().manual_seed(5)
    feats = torch.randn(nodes, op.input_width, generator=gen, dtype=torch.float64)
    src = torch.randint(0, nodes, (edges,), generator=gen)
    dst = torch.randint(0, nodes, (edges,), generator=gen)
    _, y, g, _ = _inputs(op, edges, 6)
    mask = (torch.rand(edges, generator=gen) > 0.3).double()
    out = op.graph_message(feats, y, g, src, dst, mask, edge_chunk_size=4)
    expect = torch.zeros_like(out)
    for e in range(edges):
        expect[dst[e]] += mask[e] * op.forward(feats[src[e]][None], y[e][None], g[e][None])[0]
    assert torch.allclose(out, expect, atol=1e-12)
    # empty graph: zero output that still depends on the inputs
    f = feats.clone().requires_grad_()
    empty = op.graph_message(f, y[:0], g[:0], src[:0], dst[:0])
    assert empty.shape == (nodes, op.output_width) and empty.abs().max() == 0
    assert empty.requires_grad
