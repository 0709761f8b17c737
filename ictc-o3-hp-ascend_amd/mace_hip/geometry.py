"""Edge geometry with a deterministic adjoint.

``edge_vectors(pos, src, dst)`` = pos[dst] - pos[src] (the edge geometry of reference
``mace_ictc/models/pure_cartesian_ictd_fix.py:2930-2933`` before the periodic shift).  Its
adjoint, grad_pos[n] = sum over in-edges minus sum over out-edges of grad_vec, runs on
``ictc_hip_edge_vector_grad`` over the message graph's receiver and source CSR in a fixed
order, where ``index_select``'s own backward accumulates through atomics: forces and their
training gradients are bit-identical from run to run.  The two maps are each other's adjoint,
so every derivative order stays deterministic.
"""
from __future__ import annotations

import torch

from ictc_o3 import _lib
from ictc_o3.backends.hip.graph_message import MessageGraph, message_graph


def _gather_difference(values: torch.Tensor, graph: MessageGraph) -> torch.Tensor:
    return values.index_select(0, graph.dst) - values.index_select(0, graph.src)


def _scatter_difference(grad_vec: torch.Tensor, graph: MessageGraph) -> torch.Tensor:
    grad_vec = grad_vec.contiguous()
    out = torch.empty(graph.nodes_src, 3, device=grad_vec.device, dtype=grad_vec.dtype)
    if graph.edges == 0:
        return out.zero_()
    dtype = {torch.float32: 0, torch.float64: 1}[grad_vec.dtype]
    _lib.check(_lib.lib().ictc_hip_edge_vector_grad(
        dtype, grad_vec.data_ptr(), graph.rowptr_dst.data_ptr(), _lib.ptr(graph.perm_dst), graph.rowptr_src.data_ptr(),
        _lib.ptr(graph.perm_src), out.data_ptr(), graph.nodes_src, _lib.stream_of(grad_vec.device)),
        "ictc_hip_edge_vector_grad")
    return out


class _EdgeVectors(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pos, graph):
        ctx.graph = graph
        return _gather_difference(pos, graph)

    @staticmethod
    def backward(ctx, grad_vec):
        return _EdgeVectorAdjoint.apply(grad_vec, ctx.graph), None


class _EdgeVectorAdjoint(torch.autograd.Function):
    @staticmethod
    def forward(ctx, grad_vec, graph):
        ctx.graph = graph
        return _scatter_difference(grad_vec, graph)

    @staticmethod
    def backward(ctx, grad_pos):
        return _EdgeVectors.apply(grad_pos, ctx.graph), None


def edge_vectors(pos: torch.Tensor, src: torch.Tensor, dst: torch.Tensor) -> torch.Tensor:
    """pos [N, 3] float32/float64 on the GPU, src/dst int64 [E] -> pos[dst] - pos[src] [E, 3]."""
    if pos.ndim != 2 or pos.shape[1] != 3 or pos.dtype not in (torch.float32, torch.float64):
        raise ValueError("positions must be a float32/float64 [N,3] tensor")
    graph = message_graph(src, dst, pos.shape[0], pos.shape[0])
    return _EdgeVectors.apply(pos, graph)


def one_hot_rows(index: torch.Tensor, classes: int, dtype=torch.float32) -> torch.Tensor:
    """[N, classes] indicator rows built by comparison (no device-side range check, so no host
    synchronisation and nothing that prevents graph capture)."""
    return (index.view(-1, 1) == torch.arange(classes, device=index.device)).to(dtype)
