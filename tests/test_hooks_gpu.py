"""The reference's hook entry points, called with the reference's own argument forms, against the
float64 oracle:

* ``backends.hip.tensor_product.tensor_product(owner, features, harmonics, gates=None)``
  (reference ``backends/ascend/tensor_product.py:89``) with dict blocks, a live (non-unit)
  owner weight, gates as [E,P*C] and [E,P,C] and no gates at all, and missing degree blocks;
* ``backends.hip.tensor_product.graph_message(owner, features, harmonics, gates, src, dst,
  mask=None, *, edge_chunk_size=16384)`` (reference ``:159``) with a mask, owned destinations
  and an empty graph;
* ``ictc_o3.channel_linear`` / ``species_channel_linear`` (reference
  ``backends/ascend/linear.py:8-52``) against the reference's eager formulas, values and first
  and second derivatives, and their validation rules.
"""
import math

import pytest
import torch

from conftest import RTOL, assert_rel
from oracle import ictc_basis as B
from oracle.tensor_product import TensorProductOracle

pytestmark = pytest.mark.gpu


def _owner(gpu, channels, lmax, paths, weight):
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    tp = EdgeWeightedPathPreservingTensorProduct(channels, lmax, allowed_paths=paths,
                                                 internal_compute_dtype=torch.float32).to(gpu)
    with torch.no_grad():
        tp.weight.copy_(weight.reshape(tp.weight.shape))
    return tp


def _blocks(rows, channels, lmax, gen):
    return {l: torch.randn(rows, channels, 2 * l + 1, generator=gen, dtype=torch.float64) for l in range(lmax + 1)}


def _harm(rows, lmax, gen):
    n = torch.nn.functional.normalize(torch.randn(rows, 3, generator=gen, dtype=torch.float64), dim=-1)
    y = B.direction_harmonics_packed(n, lmax)
    return {l: y[:, l * l:(l + 1) ** 2].unsqueeze(1) for l in range(lmax + 1)}


@pytest.mark.parametrize("gate_form", ["flat", "path_major", "none"])
def test_tensor_product_hook(gpu, gate_form):
    from ictc_o3.backends.hip.tensor_product import tensor_product
    gen = torch.Generator().manual_seed(11)
    c, rows = 24, 50
    paths = [(a, b, k) for a in range(3) for b in range(3) for k in range(3)
             if abs(a - b) <= k <= a + b and (a + b + k) % 2 == 0 and k <= 1]
    ref = TensorProductOracle(c, 2, 2, 2, paths=paths)
    weight = 1.0 + 0.3 * torch.randn(ref.num_paths, c, generator=gen, dtype=torch.float64)
    ref.weight = weight
    owner = _owner(gpu, c, 2, paths, weight.float())
    x = _blocks(rows, c, 2, gen)
    del x[1]                                             # a missing degree block contributes nothing
    y = _harm(rows, 2, gen)
    g = torch.randn(rows, ref.num_paths, c, generator=gen, dtype=torch.float64) / math.sqrt(ref.num_paths)
    gates = {"flat": g.reshape(rows, -1), "path_major": g, "none": None}[gate_form]
    x_full = {**x, 1: torch.zeros(rows, c, 3, dtype=torch.float64)}
    expect = ref.forward_blocks(x_full, y, torch.ones_like(g) if gates is None else gates)
    got = tensor_product(owner, {l: v.float().to(gpu) for l, v in x.items()},
                         {l: v.float().to(gpu) for l, v in y.items()},
                         None if gates is None else gates.float().to(gpu))
    assert sorted(got) == list(range(owner.lmax + 1))
    for l in expect:
        assert got[l].shape == expect[l].shape
        assert_rel(got[l], expect[l], what=f"tensor_product hook l={l} ({gate_form})")


def test_graph_message_hook(gpu):
    from ictc_o3.backends.hip.tensor_product import graph_message
    gen = torch.Generator().manual_seed(12)
    c, nodes, edges = 32, 30, 200
    ref = TensorProductOracle(c, 2, 2, 2)
    weight = 1.0 + 0.2 * torch.randn(ref.num_paths, c, generator=gen, dtype=torch.float64)
    ref.weight = weight
    owner = _owner(gpu, c, 2, ref.paths, weight.float())
    owner._ascend_destination_nodes = 22               # owned destinations of a larger halo
    x = _blocks(nodes, c, 2, gen)
    y = _harm(edges, 2, gen)
    g = torch.randn(edges, ref.num_paths * c, generator=gen, dtype=torch.float64) / math.sqrt(ref.num_paths)
    src = torch.randint(0, nodes, (edges,), generator=gen)
    dst = torch.randint(0, 22, (edges,), generator=gen)
    mask = (torch.rand(edges, 1, generator=gen) > 0.2).double()
    expect = ref.graph_message_blocks(x, y, g, src, dst, mask, nodes=22)
    got = graph_message(owner, {l: v.float().to(gpu) for l, v in x.items()},
                        {l: v.float().to(gpu) for l, v in y.items()}, g.float().to(gpu), src.to(gpu),
                        dst.to(gpu), mask.float().to(gpu), edge_chunk_size=64)
    for l in expect:
        assert got[l].shape == expect[l].shape
        assert_rel(got[l], expect[l], what=f"graph_message hook l={l}")
    # empty graph: zeros that keep the autograd graph live (reference tensor_product.py:196-199)
    xs = {l: v.float().to(gpu).requires_grad_() for l, v in x.items()}
    empty = graph_message(owner, xs, {l: v[:0].float().to(gpu) for l, v in y.items()},
                          g[:0].float().to(gpu), src[:0].to(gpu), dst[:0].to(gpu))
    assert all(float(v.detach().abs().sum()) == 0.0 for v in empty.values())
    total = sum(v.sum() for v in empty.values())
    grads = torch.autograd.grad(total, list(xs.values()), allow_unused=True)
    assert all(gr is None or float(gr.abs().sum()) == 0.0 for gr in grads)
    with pytest.raises(ValueError):
        graph_message(owner, {l: v.float().to(gpu) for l, v in x.items()},
                      {l: v.float().to(gpu) for l, v in y.items()}, g.float().to(gpu), src.to(gpu),
                      dst.to(gpu), edge_chunk_size=0)


def _channel_linear_reference(features, weight, bias=None):
    """backends/ascend/linear.py:23-25 (the eager branch)."""
    angular = features.movedim(-2, -1).contiguous()
    result = torch.nn.functional.linear(angular.reshape(-1, weight.shape[1]), weight, bias)
    return result.reshape(*angular.shape[:-1], weight.shape[0]).movedim(-1, -2)


def _species_linear_reference(features, weight, species, bias=None):
    """backends/ascend/linear.py:41-52 (the eager branch)."""
    angular = features.transpose(1, 2).contiguous()
    flat = angular.reshape(-1, angular.shape[-1])
    result = None
    for s in range(weight.shape[0]):
        value = torch.nn.functional.linear(flat, weight[s], None if bias is None else bias[s]).reshape(
            features.shape[0], features.shape[2], weight.shape[1])
        selected = torch.where(species[:, None, None] == s, value, 0.)
        result = selected if result is None else result + selected
    return result.transpose(1, 2)


def _first_and_second(fn, args, cot, hess):
    """value, d<cot, fn>/d args, and d/d args of <hess, d<cot, fn>/d args[0]>."""
    leaves = [a.clone().requires_grad_() for a in args]
    out = fn(*leaves)
    grads = torch.autograd.grad(out, leaves, cot, create_graph=True)
    second = torch.autograd.grad((grads[0] * hess).sum(), leaves[1:], allow_unused=True)
    return out, grads, second


@pytest.mark.parametrize("m,with_bias", [(1, True), (5, False), (7, False)])
def test_channel_linear(gpu, m, with_bias):
    from ictc_o3 import channel_linear
    gen = torch.Generator().manual_seed(13 + m)
    x = torch.randn(3, 41, 16, m, generator=gen, dtype=torch.float64)
    w = torch.randn(24, 16, generator=gen, dtype=torch.float64) / 4
    args = [x, w] + ([torch.randn(24, generator=gen, dtype=torch.float64)] if with_bias else [])
    cot = torch.randn(3, 41, 24, m, generator=gen, dtype=torch.float64)
    hess = torch.randn_like(x)
    expect = _first_and_second(_channel_linear_reference, args, cot, hess)
    got = _first_and_second(channel_linear, [a.float().to(gpu) for a in args], cot.float().to(gpu),
                            hess.float().to(gpu))
    assert_rel(got[0], expect[0], what="channel_linear")
    for a, b in zip(got[1], expect[1]):
        assert_rel(a, b, what="channel_linear first derivative")
    for a, b in zip(got[2], expect[2]):
        if b is not None:
            assert_rel(a, b, what="channel_linear second derivative")


@pytest.mark.parametrize("m,with_bias", [(1, True), (3, False)])
def test_species_channel_linear(gpu, m, with_bias):
    from ictc_o3 import species_channel_linear
    gen = torch.Generator().manual_seed(17 + m)
    n, i, o, s = 57, 16, 12, 4
    x = torch.randn(n, i, m, generator=gen, dtype=torch.float64)
    w = torch.randn(s, o, i, generator=gen, dtype=torch.float64) / 4
    species = torch.randint(0, s, (n,), generator=gen)
    bias = torch.randn(s, o, generator=gen, dtype=torch.float64) if with_bias else None
    cot = torch.randn(n, o, m, generator=gen, dtype=torch.float64)
    hess = torch.randn_like(x)

    def ref(xx, ww, *b):
        return _species_linear_reference(xx, ww, species, *b)

    def hip(xx, ww, *b):
        return species_channel_linear(xx, ww, species.to(gpu), *b)
    args = [x, w] + ([bias] if with_bias else [])
    expect = _first_and_second(ref, args, cot, hess)
    got = _first_and_second(hip, [a.float().to(gpu) for a in args], cot.float().to(gpu), hess.float().to(gpu))
    assert_rel(got[0], expect[0], what="species_channel_linear")
    for a, b in zip(got[1], expect[1]):
        assert_rel(a, b, what="species_channel_linear first derivative")
    for a, b in zip(got[2], expect[2]):
        if b is not None:
            assert_rel(a, b, rtol=RTOL, what="species_channel_linear second derivative")


def test_linear_validation(gpu):
    from ictc_o3 import channel_linear, species_channel_linear
    x = torch.randn(4, 8, 3, device=gpu)
    w = torch.randn(5, 8, device=gpu)
    with pytest.raises(ValueError):
        channel_linear(x, torch.randn(5, 7, device=gpu))
    with pytest.raises(ValueError):
        channel_linear(x, w, torch.randn(5, device=gpu))          # bias on a non-scalar block
    with pytest.raises(ValueError):
        channel_linear(x.double(), w.double())                     # precision is never changed
    ws = torch.randn(2, 5, 8, device=gpu)
    with pytest.raises(ValueError):
        species_channel_linear(x, ws, torch.tensor([0, 1, 2, 0], device=gpu))   # species out of range
    with pytest.raises(ValueError):
        species_channel_linear(x, ws, torch.zeros(4, dtype=torch.float32, device=gpu))
    with pytest.raises(ValueError):
        species_channel_linear(x, ws, torch.zeros(4, dtype=torch.int64, device=gpu), torch.randn(2, 5, device=gpu))
