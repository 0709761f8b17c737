"""ictc_hip_message_edge_grad_static (the entry point that allocates nothing; its chunk partials
live in a library-owned static device array) against ictc_hip_message_edge_grad followed by the
sum over the chunk axis, through the C ABI.

Each configuration runs two calls in a row on one GPU, the second on a smaller graph, so rows
the first call left in the shared array must not leak into the second call's result.  Channel
counts cover one chunk (the kernel writes the sums itself), two chunks (the cfg-4 width; the
two-term sum is exact in either order) and three chunks.  Sizes beyond the array are refused
before any launch.
"""
import ctypes
import math

import pytest
import torch

from conftest import assert_rel
from oracle import ictc_basis as B

pytestmark = pytest.mark.gpu


def _plan(c, lmax):
    from ictc_o3.backends.hip.tensor_product import TensorProductPlan
    from ictc_o3.basis.ictd_irreps import triangle_paths
    return TensorProductPlan(triangle_paths(lmax, lmax, lmax), c, lmax, lmax)


def _inputs(plan, nodes, edges, seed, dev):
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, nodes, (edges,), generator=g)
    dst = torch.randint(0, nodes - 1, (edges,), generator=g)        # the last node receives nothing
    x = torch.randn(nodes, plan.x_width, generator=g)
    n = torch.nn.functional.normalize(torch.randn(edges, 3, generator=g, dtype=torch.float64), dim=-1)
    y = B.direction_harmonics_packed(n, plan.edge_lmax).float()
    gates = torch.randn(edges, plan.full_gate_width, generator=g) / math.sqrt(plan.desc.num_paths)
    go = torch.randn(nodes, plan.full_out_width, generator=g)
    return [t.to(dev) for t in (src, dst, x, y, gates, go)]


def _edge_grads(plan, nodes, edges, seed, dev):
    from ictc_o3 import _lib
    from ictc_o3.backends.hip.graph_message import message_graph
    lib = _lib.lib()
    src, dst, x, y, gates, go = _inputs(plan, nodes, edges, seed, dev)
    graph = message_graph(src, dst, nodes, nodes)
    stream = _lib.stream_of(dev)
    chunks = lib.ictc_hip_message_chunks(plan.channels)
    ny = plan.y_width
    common = (ctypes.byref(plan.desc), x.data_ptr(), y.data_ptr(), gates.data_ptr(), go.data_ptr(),
              graph.src.data_ptr(), graph.rowptr_dst.data_ptr(), _lib.ptr(graph.perm_dst))
    dyp = torch.empty(edges, chunks, ny, device=dev)
    dg = torch.empty(edges, plan.full_gate_width, device=dev)
    dxe = torch.empty(edges, plan.x_width, device=dev)
    _lib.check(lib.ictc_hip_message_edge_grad(*common, dyp.data_ptr(), dg.data_ptr(), dxe.data_ptr(), nodes,
                                              nodes, edges, 0, stream), "ictc_hip_message_edge_grad")
    dy2 = torch.full((edges, ny), float("nan"), device=dev)
    dg2 = torch.full_like(dg, float("nan"))
    dxe2 = torch.full_like(dxe, float("nan"))
    print(f"static edge grad: C={plan.channels} lmax={plan.edge_lmax} nodes={nodes} edges={edges}", flush=True)
    _lib.check(lib.ictc_hip_message_edge_grad_static(*common, dy2.data_ptr(), dg2.data_ptr(), dxe2.data_ptr(),
                                                     nodes, nodes, edges, stream),
               "ictc_hip_message_edge_grad_static")
    torch.cuda.synchronize(dev)
    return (dyp.sum(1) if chunks > 1 else dyp[:, 0]), dg, dxe, dy2, dg2, dxe2, chunks


@pytest.mark.parametrize("c,lmax", [(128, 3), (192, 2), (64, 2)])
def test_static_edge_grad_matches_allocating_entry_point(gpu, c, lmax):
    plan = _plan(c, lmax)
    for nodes, edges, seed in ((300, 4000, 1), (40, 500, 2)):        # second call smaller
        dy, dg, dxe, dy2, dg2, dxe2, chunks = _edge_grads(plan, nodes, edges, seed, gpu)
        assert torch.equal(dg2, dg) and torch.equal(dxe2, dxe)
        if chunks <= 2:
            assert torch.equal(dy2, dy)
        else:
            assert_rel(dy2, dy, rtol=1e-6, what="chunk sums")
        assert bool(torch.isfinite(dy2).all())


def test_static_edge_grad_refuses_beyond_capacity(gpu):
    from ictc_o3 import _lib
    lib = _lib.lib()
    plan = _plan(128, 3)
    capacity = 4194304 // (2 * 16)
    fake = ctypes.c_void_p(256)   # never dereferenced: the size check comes before any launch
    args = (ctypes.byref(plan.desc),) + (fake,) * 10
    assert lib.ictc_hip_message_edge_grad_static(*args, 8, 8, capacity + 1, None) == 5
    assert lib.ictc_hip_status_string(5) == b"input exceeds the static scratch capacity"


def test_static_edge_grad_under_graph_capture(gpu):
    """The entry point captured into a HIP graph (after ictc_hip_message_static_prepare resolved
    the array's address, so the capture records launches only), replayed three times on inputs
    changed in place, with eager work in between: every replay equals the allocating entry point
    on the same inputs."""
    from ictc_o3 import _lib
    from ictc_o3.backends.hip.graph_message import message_graph
    lib = _lib.lib()
    plan = _plan(128, 3)
    nodes, edges = 200, 3000
    src, dst, x, y, gates, go = _inputs(plan, nodes, edges, 5, gpu)
    graph = message_graph(src, dst, nodes, nodes)
    assert lib.ictc_hip_message_static_prepare() == 0
    ny = plan.y_width
    dy = torch.empty(edges, ny, device=gpu)
    dg = torch.empty(edges, plan.full_gate_width, device=gpu)
    dxe = torch.empty(edges, plan.x_width, device=gpu)

    def call(stream):
        return lib.ictc_hip_message_edge_grad_static(
            ctypes.byref(plan.desc), x.data_ptr(), y.data_ptr(), gates.data_ptr(), go.data_ptr(),
            graph.src.data_ptr(), graph.rowptr_dst.data_ptr(), _lib.ptr(graph.perm_dst), dy.data_ptr(),
            dg.data_ptr(), dxe.data_ptr(), nodes, nodes, edges, stream)

    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        assert call(side.cuda_stream) == 0                          # warm-up outside the capture
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize(gpu)
    g = torch.cuda.CUDAGraph()
    print("static edge grad: capture", flush=True)
    with torch.cuda.graph(g):
        assert call(_lib.stream_of(gpu)) == 0
    gen = torch.Generator(device=gpu).manual_seed(9)
    for replay in range(3):
        with torch.no_grad():
            x.copy_(torch.randn(x.shape, device=gpu, generator=gen))
            go.copy_(torch.randn(go.shape, device=gpu, generator=gen))
        g.replay()
        torch.cuda.synchronize(gpu)
        chunks = lib.ictc_hip_message_chunks(plan.channels)
        dyp = torch.empty(edges, chunks, ny, device=gpu)
        dg_ref = torch.empty_like(dg)
        dxe_ref = torch.empty_like(dxe)
        _lib.check(lib.ictc_hip_message_edge_grad(
            ctypes.byref(plan.desc), x.data_ptr(), y.data_ptr(), gates.data_ptr(), go.data_ptr(),
            graph.src.data_ptr(), graph.rowptr_dst.data_ptr(), _lib.ptr(graph.perm_dst), dyp.data_ptr(),
            dg_ref.data_ptr(), dxe_ref.data_ptr(), nodes, nodes, edges, 0, _lib.stream_of(gpu)),
            "ictc_hip_message_edge_grad")
        torch.cuda.synchronize(gpu)
        assert torch.equal(dg, dg_ref) and torch.equal(dxe, dxe_ref), f"replay {replay}"
        assert torch.equal(dy, dyp.sum(1)), f"replay {replay}"
