"""Graph message on the HIP kernels: out[n] = sum_{dst(e)=n} TP(x[src(e)], Y[e], g[e]).

Reference semantics: ``backends/ascend/tensor_product.py:189-218`` (gather -> TP ->
index_add) and ``channel_message.py:35-216`` (the published performance path).

The map is trilinear in (node features x, edge harmonics Y, edge gates g) for a
fixed graph, so its VJP and every mixed derivative reuse the same three kernels
with substituted operands (as for the plain TP):

    bonds     : msg_bond     (per-edge bond matrices from Y, once per edge; forward only)
    forward   : msg_forward  (receiver CSR, per-node register accumulation)
    dY, dg    : msg_edge_grad (receiver CSR, dout[n] contracted with the CG tensors once
                per receiver, x[src] gathered, Y read per edge)
    dx        : msg_edge_grad writes each edge's feature adjoint, msg_node_grad sums
                them per source node (source CSR), so dout is never gathered per edge

Graph preprocessing (CSR over receivers and over sources, stable order, index range
validation) runs once per (src, dst) pair and is cached.
"""
from __future__ import annotations

import contextlib
import ctypes
from typing import Optional

import torch

from ... import _lib
from ...autograd.adjoint_requirements import required_gradients
from .tensor_product import TensorProductPlan


class MessageGraph:
    """Receiver and source CSR of an edge list (stable order: ties keep edge order)."""

    def __init__(self, src: torch.Tensor, dst: torch.Tensor, nodes_src: int, nodes_dst: int):
        if src.ndim != 1 or dst.ndim != 1 or src.dtype != torch.int64 or dst.dtype != torch.int64:
            raise ValueError("Graph indices must be int64 vectors")
        if src.shape != dst.shape:
            raise ValueError("Source and destination index shapes must match")
        self.src, self.dst = src.contiguous(), dst.contiguous()
        self.edges = int(src.numel())
        self.nodes_src, self.nodes_dst = int(nodes_src), int(nodes_dst)
        if self.edges:
            lo = torch.stack([self.src.min(), self.dst.min()]).cpu()
            hi = torch.stack([self.src.max(), self.dst.max()]).cpu()
            if int(lo.min()) < 0 or int(hi[0]) >= self.nodes_src or int(hi[1]) >= self.nodes_dst:
                raise ValueError("Graph indices are out of range")
        self.rowptr_dst, self.perm_dst = self._csr(self.dst, self.nodes_dst)
        self.rowptr_src, self.perm_src = self._csr(self.src, self.nodes_src)

    def _csr(self, index: torch.Tensor, nodes: int):
        dev = index.device
        counts = torch.bincount(index, minlength=nodes) if self.edges else torch.zeros(
            nodes, dtype=torch.int64, device=dev)
        rowptr = torch.zeros(nodes + 1, dtype=torch.int64, device=dev)
        torch.cumsum(counts, 0, out=rowptr[1:])
        if self.edges and bool((index[1:] >= index[:-1]).all()):
            return rowptr, None                      # already sorted: identity permutation
        perm = torch.sort(index, stable=True).indices if self.edges else None
        return rowptr, perm


_GRAPH_CACHE: dict = {}
_PIN_LISTS: list = []          # open pin_graphs() scopes


@contextlib.contextmanager
def pin_graphs():
    """Collect every MessageGraph handed out inside the scope into the yielded list.

    A HIP graph captured inside the scope records the raw device addresses of those graphs'
    CSR tensors; the cache below evicts entries, so whoever replays the capture must keep
    the list (and with it the tensors) alive for as long as the capture exists."""
    held: list = []
    _PIN_LISTS.append(held)
    try:
        yield held
    finally:
        # by identity: two open scopes may hold equal lists
        del _PIN_LISTS[next(i for i, h in enumerate(_PIN_LISTS) if h is held)]


def message_graph(src: torch.Tensor, dst: torch.Tensor, nodes_src: int, nodes_dst: int) -> MessageGraph:
    """Cached CSR build; the key includes tensor identity and version counters."""
    key = (src.data_ptr(), dst.data_ptr(), src._version, dst._version, src.numel(), str(src.device),
           int(nodes_src), int(nodes_dst))
    graph = _GRAPH_CACHE.get(key)
    if graph is None or graph.src.data_ptr() != src.data_ptr():
        if len(_GRAPH_CACHE) > 8:
            _GRAPH_CACHE.clear()
        graph = MessageGraph(src, dst, nodes_src, nodes_dst)
        _GRAPH_CACHE[key] = graph
    for held in _PIN_LISTS:
        if not any(g is graph for g in held):
            held.append(graph)
    return graph


def _p(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def bond_width(plan: TensorProductPlan) -> int:
    width = getattr(plan, "_bond_width", None)
    if width is None:
        width = _lib.lib().ictc_hip_message_bond_width(ctypes.byref(plan.desc))
        if width < 0:
            raise ValueError("invalid tensor-product descriptor")
        plan._bond_width = width
    return width


def _bonds(plan: TensorProductPlan, graph: MessageGraph, y) -> Optional[torch.Tensor]:
    """Per-edge bond matrices [E, NB] of harmonics y (None for an empty graph).  For degree
    sets whose kernels build the bond rows themselves (bond width 0) this is y itself."""
    if graph.edges == 0:
        return None
    if bond_width(plan) == 0:
        return y
    out = torch.empty(graph.edges, bond_width(plan), device=y.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_message_bonds(
        ctypes.byref(plan.desc), y.data_ptr(), out.data_ptr(), graph.edges, _lib.stream_of(y.device)),
        "ictc_hip_message_bonds")
    return out


def _forward_raw(plan: TensorProductPlan, graph: MessageGraph, x, y, g, bonds=None) -> torch.Tensor:
    if bonds is None:
        bonds = _bonds(plan, graph, y)
    out = torch.empty(graph.nodes_dst, plan.full_out_width, device=x.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_message_forward(
        ctypes.byref(plan.desc), x.data_ptr(), _p(bonds), _p(g), graph.src.data_ptr(),
        graph.rowptr_dst.data_ptr(), _p(graph.perm_dst), out.data_ptr(), graph.nodes_src,
        graph.nodes_dst, graph.edges, _lib.stream_of(x.device)), "ictc_hip_message_forward")
    return out


def _backward_raw(plan: TensorProductPlan, graph: MessageGraph, need, x, y, g, go, dg_into=None):
    """First-order adjoints; the edge kernels read the harmonics y (not bond rows).  dg_into: a gate
    gradient [E, P*C] already computed for the same gates, which the kernel adds this one into (the
    returned dg is then that buffer)."""
    dev = go.device
    lib = _lib.lib()
    stream = _lib.stream_of(dev)
    dx = dy = dg = None
    dyp = dxe = None
    if graph.edges:
        nch = lib.ictc_hip_message_chunks(plan.channels)
        if need[1]:
            dyp = torch.empty(graph.edges, nch, plan.y_width, device=dev, dtype=torch.float32)
        if need[2]:
            dg = dg_into if dg_into is not None else torch.empty(graph.edges, plan.full_gate_width, device=dev,
                                                                 dtype=torch.float32)
        if need[0]:
            dxe = torch.empty(graph.edges, plan.x_width, device=dev, dtype=torch.float32)
        if need[0] or need[1] or need[2]:
            xp = x.data_ptr() if (need[1] or need[2]) else None
            _lib.check(lib.ictc_hip_message_edge_grad(
                ctypes.byref(plan.desc), xp, _p(y), _p(g), go.data_ptr(), graph.src.data_ptr(),
                graph.rowptr_dst.data_ptr(), _p(graph.perm_dst), _p(dyp), _p(dg), _p(dxe), graph.nodes_src,
                graph.nodes_dst, graph.edges, int(dg_into is not None and need[2]), stream),
                "ictc_hip_message_edge_grad")
        if dyp is not None:
            dy = dyp[:, 0] if nch == 1 else dyp.sum(1)
    else:
        if need[1]:
            dy = torch.empty(0, plan.y_width, device=dev, dtype=torch.float32)
        if need[2]:
            dg = torch.empty(0, plan.full_gate_width, device=dev, dtype=torch.float32)
    if need[0]:
        dx = torch.empty(graph.nodes_src, plan.x_width, device=dev, dtype=torch.float32)
        _lib.check(lib.ictc_hip_message_node_grad(
            ctypes.byref(plan.desc), _p(dxe), graph.rowptr_src.data_ptr(), _p(graph.perm_src), dx.data_ptr(),
            graph.nodes_src, graph.edges, stream), "ictc_hip_message_node_grad")
    return dx, dy, dg


def _second_order_raw(plan: TensorProductPlan, graph: MessageGraph, need, x, y, g, go, tx, ty, tg, bonds=None):
    """Mixed second derivatives of the message for the tangent (tx, ty, tg) with go fixed:
    (gx, gy, gg, ggo) = the directional derivatives of (node_grad(dxe), dY, dg) and of the
    forward, each summed over the three one-argument substitutions; two tangent kernel
    passes and one node_grad instead of a forward and a VJP per tangent argument."""
    nx, ny, ng, no = (bool(n) for n in need)
    dev = go.device
    lib = _lib.lib()
    stream = _lib.stream_of(dev)
    gx = gy = gg = ggo = None
    if no:   # the forward tangent reads bond rows, the edge tangent pass the harmonics
        if bonds is None:
            bonds = _bonds(plan, graph, y)
        tbonds = _bonds(plan, graph, ty)
        ggo = torch.empty(graph.nodes_dst, plan.full_out_width, device=dev, dtype=torch.float32)
        _lib.check(lib.ictc_hip_message_forward_tangent(
            ctypes.byref(plan.desc), x.data_ptr(), _p(bonds), _p(g), tx.data_ptr(), _p(tbonds), _p(tg),
            graph.src.data_ptr(), graph.rowptr_dst.data_ptr(), _p(graph.perm_dst), ggo.data_ptr(),
            graph.nodes_src, graph.nodes_dst, graph.edges, stream), "ictc_hip_message_forward_tangent")
    nch = lib.ictc_hip_message_chunks(plan.channels)
    dyp = torch.empty(graph.edges, nch, plan.y_width, device=dev, dtype=torch.float32) if ny else None
    gg = torch.empty(graph.edges, plan.full_gate_width, device=dev, dtype=torch.float32) if ng else None
    dxe = torch.empty(graph.edges, plan.x_width, device=dev, dtype=torch.float32) if nx else None
    if nx or ny or ng:
        _lib.check(lib.ictc_hip_message_edge_grad_tangent(
            ctypes.byref(plan.desc), x.data_ptr(), _p(y), _p(g), tx.data_ptr(), _p(ty), _p(tg),
            go.data_ptr(), graph.src.data_ptr(), graph.rowptr_dst.data_ptr(), _p(graph.perm_dst), _p(dyp),
            _p(gg), _p(dxe), graph.nodes_src, graph.nodes_dst, graph.edges, stream),
            "ictc_hip_message_edge_grad_tangent")
    if dyp is not None:
        gy = dyp[:, 0] if nch == 1 else dyp.sum(1)
    if nx:
        gx = torch.empty(graph.nodes_src, plan.x_width, device=dev, dtype=torch.float32)
        _lib.check(lib.ictc_hip_message_node_grad(
            ctypes.byref(plan.desc), dxe.data_ptr(), graph.rowptr_src.data_ptr(), _p(graph.perm_src),
            gx.data_ptr(), graph.nodes_src, graph.edges, stream), "ictc_hip_message_node_grad")
    return gx, gy, gg, ggo


# The double backward uses the fused tangent kernels when no further derivative is recorded
# (grad mode off inside backward), all three tangents are present and the degrees have them
# (every degree <= 3); otherwise it applies the differentiable one-argument substitutions.
# Tests switch this off to compare the two.
FUSED_SECOND_ORDER = True


def _add(acc, value):
    if value is None:
        return acc
    return value if acc is None else acc + value


class _GateGradSlot:
    """Hand-over of a gate gradient between the two autograd nodes that both produce a gradient
    for the same message gates in a force-loss double backward: the message forward's node (the
    energy path) and the node of its VJP (the force path, recorded when the forces are taken with
    create_graph).  Without it the engine sums the two [E, P*C] gradients with one more pass over
    three such tensors.  When the VJP's node runs first and the forward's node is still to run and
    will produce a gate gradient, the VJP's node leaves its gate gradient here and returns none;
    the forward's node then has the edge kernel add its own gradient into that buffer
    (``ictc_hip_message_edge_grad`` accumulate mode) and returns the sum.  In any other order
    both return their gradients and the engine adds them as usual."""
    __slots__ = ("stash", "forward_done")

    def __init__(self):
        self.stash = None            # a gate gradient deferred to the forward's node
        self.forward_done = False    # the forward's node ran in a backward that records nothing


# The hand-over of _GateGradSlot (tests switch it off to compare: the results are bit-identical,
# a float add being commutative).
GATE_GRAD_HANDOVER = True


def _defer_gate_grad(ctx, plan: TensorProductPlan, graph: MessageGraph, g) -> bool:
    """Whether the VJP node (ctx) hands its gate gradient to the message forward's node."""
    slot, fwd = getattr(ctx, "slot", None), getattr(ctx, "forward_node", None)
    if (not GATE_GRAD_HANDOVER or torch.is_grad_enabled() or slot is None or fwd is None or slot.stash is not None
            or slot.forward_done):
        return False
    if plan.generic or graph.edges == 0 or not fwd.needs_input_grad[4]:
        return False
    query = getattr(torch._C, "_will_engine_execute_node", None)
    if query is None:
        return False
    try:
        return bool(query(fwd)) and required_gradients((g,), (True,))[0]
    except (RuntimeError, AttributeError, AssertionError):
        return False


class _Forward(torch.autograd.Function):
    """bonds: the bond rows of y when the caller has them (derived data, not an input)."""

    @staticmethod
    def forward(ctx, plan, graph, x, y, g, bonds=None):
        ctx.plan, ctx.graph = plan, graph
        if bonds is None:
            bonds = _bonds(plan, graph, y)
        ctx.bonds = bonds
        ctx.slot = _GateGradSlot()
        ctx.save_for_backward(x, y, g)
        return _forward_raw(plan, graph, x, y, g, bonds)

    @staticmethod
    def backward(ctx, go):
        x, y, g = ctx.saved_tensors
        stash = None
        if not torch.is_grad_enabled():          # a backward that records nothing (the last one)
            stash, ctx.slot.stash = ctx.slot.stash, None
            ctx.slot.forward_done = True
        need = required_gradients((x, y, g), ctx.needs_input_grad[2:5])
        if go is None or not any(need):
            return None, None, None, None, stash, None
        if stash is not None and need[2] and not ctx.plan.generic and ctx.graph.edges:
            # add this gate gradient into the one the VJP's node deferred here (inside the kernel)
            dx, dy, dg = _backward_raw(ctx.plan, ctx.graph, need, x, y, g, go.contiguous(), dg_into=stash)
        else:
            dx, dy, dg = vjp(ctx.plan, ctx.graph, need, x, y, g, go.contiguous(), ctx.bonds, slot=ctx.slot,
                             forward_node=ctx)
            if stash is not None:
                dg = stash if dg is None else dg + stash
        return None, None, dx, dy, dg, None


class _Backward(torch.autograd.Function):
    @staticmethod
    def forward(ctx, plan, graph, need, x, y, g, go, bonds=None, slot=None, forward_node=None):
        ctx.plan, ctx.graph, ctx.need = plan, graph, need
        ctx.slot, ctx.forward_node = slot, forward_node   # see _GateGradSlot
        ctx.set_materialize_grads(False)
        ctx.bonds = bonds   # for the forward passes of the double backward (formed there if None)
        ctx.save_for_backward(x, y, g, go)
        outs = _backward_raw(plan, graph, need, x, y, g, go)
        empty = go.new_empty(0)
        outs = tuple(t if t is not None else empty for t in outs)
        for t, n in zip(outs, need):
            if not n:
                ctx.mark_non_differentiable(t)
        return outs

    @staticmethod
    def backward(ctx, hx, hy, hg):
        plan, graph, need_out = ctx.plan, ctx.graph, ctx.need
        x, y, g, go = ctx.saved_tensors
        bonds = ctx.bonds
        hx = hx if need_out[0] else None
        hy = hy if need_out[1] else None
        hg = hg if need_out[2] else None
        nx, ny, ng, no = required_gradients((x, y, g, go), ctx.needs_input_grad[3:7])
        if (FUSED_SECOND_ORDER and not plan.generic and not torch.is_grad_enabled() and graph.edges > 0
                and hx is not None and hy is not None and hg is not None and (nx or ny or ng or no)):
            gx, gy, gg, ggo = _second_order_raw(plan, graph, (nx, ny, ng, no), x, y, g, go, hx.contiguous(),
                                                hy.contiguous(), hg.contiguous(), bonds)
            if gg is not None and _defer_gate_grad(ctx, plan, graph, g):
                ctx.slot.stash, gg = gg, None
            return None, None, None, gx, gy, gg, ggo, None, None, None
        gx = gy = gg = ggo = None
        if hx is not None:
            hx = hx.contiguous()
            if ny or ng:
                _, a, b = vjp(plan, graph, (False, ny, ng), hx, y, g, go, bonds)
                gy, gg = _add(gy, a), _add(gg, b)
            if no:
                ggo = _add(ggo, _Forward.apply(plan, graph, hx, y, g, bonds))
        if hy is not None:
            hy = hy.contiguous()
            if nx or ng:
                a, _, b = vjp(plan, graph, (nx, False, ng), x, hy, g, go)
                gx, gg = _add(gx, a), _add(gg, b)
            if no:
                ggo = _add(ggo, _Forward.apply(plan, graph, x, hy, g))
        if hg is not None:
            hg = hg.contiguous()
            if nx or ny:
                a, b, _ = vjp(plan, graph, (nx, ny, False), x, y, hg, go, bonds)
                gx, gy = _add(gx, a), _add(gy, b)
            if no:
                ggo = _add(ggo, _Forward.apply(plan, graph, x, y, hg, bonds))
        if gg is not None and _defer_gate_grad(ctx, plan, graph, g):
            ctx.slot.stash, gg = gg, None
        return None, None, None, gx, gy, gg, ggo, None, None, None


def vjp(plan, graph, need, x, y, g, go, bonds=None, slot=None, forward_node=None):
    need = tuple(bool(n) for n in need)
    if not any(need):
        return None, None, None
    if not torch.is_grad_enabled():       # nothing recorded: skip the autograd Function
        return _backward_raw(plan, graph, need, x, y, g, go)
    outs = _Backward.apply(plan, graph, need, x, y, g, go, bonds, slot, forward_node)
    return tuple(o if n else None for o, n in zip(outs, need))


def message_bonds(plan: TensorProductPlan, harmonics: torch.Tensor) -> Optional[torch.Tensor]:
    """The bond rows the message forward derives from the harmonics [E, (L_e+1)^2] (the harmonics
    themselves for degree sets whose kernels build them in-kernel; None without edges), for a
    caller that issues them ahead, e.g. on another stream, and passes them to
    ``packed_graph_message``."""
    edges = harmonics.shape[0]
    if edges == 0:
        return None
    y = harmonics.contiguous()
    if bond_width(plan) == 0:
        return y
    out = torch.empty(edges, bond_width(plan), device=y.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_message_bonds(ctypes.byref(plan.desc), y.data_ptr(), out.data_ptr(), edges,
                                                 _lib.stream_of(y.device)), "ictc_hip_message_bonds")
    return out


def packed_graph_message(plan: TensorProductPlan, features: torch.Tensor, harmonics: torch.Tensor,
                         gates: torch.Tensor, src: torch.Tensor, dst: torch.Tensor, *,
                         nodes_dst: Optional[int] = None, mask: Optional[torch.Tensor] = None,
                         bonds: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Packed ir_mul message: features [N_src, C(L_in+1)^2], harmonics [E,(L_e+1)^2],
    gates [E, P*C] (path weights folded in), src/dst int64 [E] -> [N_dst, NOC*C].  bonds: the
    harmonics' ``message_bonds`` for this plan when the caller has them (derived data: the
    harmonics stay the differentiated input)."""
    nodes_src = features.shape[0]
    nodes_dst = nodes_src if nodes_dst is None else int(nodes_dst)
    graph = message_graph(src, dst, nodes_src, nodes_dst)
    rows, c = gates.shape[0], plan.channels
    if mask is not None:
        gates = gates * mask.reshape(rows, 1).to(gates.dtype)
    if not plan.is_full:
        slots = torch.tensor(plan.slot_of_path, device=gates.device)
        gates = gates.new_zeros(rows, len(plan.full_paths), c).index_copy(
            1, slots, gates.reshape(rows, plan.num_paths, c)).reshape(rows, len(plan.full_paths) * c)
    out = _Forward.apply(plan, graph, features.contiguous(), harmonics.contiguous(), gates.contiguous(), bonds)
    if not plan.is_full:
        keep = torch.tensor(plan.output_rows, device=gates.device)
        out = out.reshape(nodes_dst, -1, c).index_select(1, keep).reshape(nodes_dst, len(plan.output_rows) * c)
    return out
