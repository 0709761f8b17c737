"""Radial-streaming graph message: the gates of the message are the output of a dense radial
projection ``gates = hidden @ W^T + b`` (the last Linear of the radial MLP), produced one
receiver range at a time instead of as one ``[E, P*C]`` tensor (reference
``ictc_o3/backends/ascend/capacity_message.py:109-179``, ``capacity_adjoint.py:5-148``).

Schedule (edges in receiver-CSR slot order; for a dst-sorted edge list that is the edge order):

* the receivers are cut into contiguous ranges holding at most ``edge_chunk_size`` edges each
  (a receiver with more edges forms its own range), from the receiver CSR once per graph;
* forward, per range: gates_r = hidden_r @ W^T + b (one GEMM into a range-sized buffer), the bond
  rows of the range's harmonics, then the fused message kernel over the range's receivers only,
  writing their node rows.  Peak scratch: one range's gates and bonds instead of the whole
  graph's;
* first-order backward (grad mode off, as for forces at inference and for the first backward of
  any first-order use), per range: the gates again, the per-edge adjoint kernel over the range
  (harmonics gradient, gate adjoint, edge feature adjoints), then d hidden_r = dg_r @ W,
  dW += dg_r^T hidden_r, db += sum(dg_r), and the range's node-feature gradient by the
  source-CSR segmented sum restricted to the range's edges, added to dx.  Every sum has a fixed
  order: the result is the same on every run;
* a backward that is itself differentiated (force-loss training) materialises the full gates
  differentiably and takes the ordinary message adjoint, as the reference keeps its native
  recursive schedule for higher derivatives (``capacity_message.py:36-48``).

Two ranges are in flight: consecutive ranges alternate between the caller's stream and a second
(default-priority) stream, each stream with its own range buffers and, in the backward, its own
node-gradient and weight-gradient accumulators (added once at the end), so one range's GEMM and
kernels run beside the other's.  A single range at a time leaves most of the GPU idle at these sizes:
a 16,384-edge range launches ~600 receiver blocks per message kernel.  Peak scratch is two ranges'
buffers.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Tuple

import numpy as np
import torch

from ... import _lib
from ...autograd.adjoint_requirements import required_gradients
from .graph_message import MessageGraph, bond_width, message_graph, vjp
from .linear import mm, sgemm_into
from .tensor_product import TensorProductPlan


class RangePlan:
    """Receiver ranges of one graph for one range size, with the slot-ordered source indices,
    each range's shifted receiver row pointers and its own source CSR (cached on the graph)."""

    def __init__(self, graph: MessageGraph, edge_chunk_size: int):
        rowptr = graph.rowptr_dst.cpu().numpy()
        self.ranges: List[Tuple[int, int, int, int]] = []
        n0 = 0
        while n0 < graph.nodes_dst:
            # the most receivers from n0 on whose edges fit, at least one
            n1 = int(np.searchsorted(rowptr, rowptr[n0] + edge_chunk_size, side="right")) - 1
            n1 = min(max(n1, n0 + 1), graph.nodes_dst)
            self.ranges.append((n0, n1, int(rowptr[n0]), int(rowptr[n1])))
            n0 = n1
        dev = graph.src.device
        self.src_sorted = (graph.src if graph.perm_dst is None else graph.src.index_select(0, graph.perm_dst)).contiguous()
        self.rowptr = [graph.rowptr_dst[n0:n1 + 1] - s0 for n0, n1, s0, _ in self.ranges]
        self.source_csr = []
        for _, _, s0, s1 in self.ranges:
            src_r = self.src_sorted[s0:s1]
            counts = torch.bincount(src_r, minlength=graph.nodes_src) if s1 > s0 else torch.zeros(
                graph.nodes_src, dtype=torch.int64, device=dev)
            rp = torch.zeros(graph.nodes_src + 1, dtype=torch.int64, device=dev)
            torch.cumsum(counts, 0, out=rp[1:])
            perm = torch.sort(src_r, stable=True).indices if s1 > s0 else None
            self.source_csr.append((rp, perm))
        self.max_rows = max([1] + [s1 - s0 for _, _, s0, s1 in self.ranges])


def range_plan(graph: MessageGraph, edge_chunk_size: int) -> RangePlan:
    plans = graph.__dict__.setdefault("_range_plans", {})
    plan = plans.get(int(edge_chunk_size))
    if plan is None:
        plan = RangePlan(graph, int(edge_chunk_size))
        plans[int(edge_chunk_size)] = plan
    return plan


def _slot_order(t: Optional[torch.Tensor], graph: MessageGraph) -> Optional[torch.Tensor]:
    if t is None or graph.perm_dst is None:
        return t
    return t.index_select(0, graph.perm_dst)


def _range_gates_into(out, hidden, weight, bias, mask, s0, s1):
    """The range's gates hidden[s0:s1] @ W^T (+ b) (* mask) into a stream's range buffer."""
    g = sgemm_into(hidden[s0:s1], weight.t(), out[:s1 - s0])
    if bias is not None:
        g += bias
    if mask is not None:
        g *= mask[s0:s1].unsqueeze(1)
    return g


def _range_bonds(plan: TensorProductPlan, y, s0, s1, out):
    yr = y[s0:s1]
    if bond_width(plan) == 0:
        return yr
    _lib.check(_lib.lib().ictc_hip_message_bonds(ctypes.byref(plan.desc), yr.data_ptr(), out.data_ptr(), s1 - s0,
                                                 _lib.stream_of(y.device)), "ictc_hip_message_bonds")
    return out


_SIDE: dict = {}


def _streams(device: torch.device):
    """(the caller's stream, this module's second stream on the device, created once)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    side = _SIDE.get(index)
    if side is None:
        side = _SIDE[index] = torch.cuda.Stream(device=index)
    return torch.cuda.current_stream(device), side


class _TwoStreams:
    """Fork onto the second stream (it waits for the caller's work so far), mark the inputs it reads,
    and join it back at the end: the caller's stream then holds every range's results."""

    def __init__(self, device, reads):
        self.main, self.side = _streams(device)
        self.reads = [t for t in reads if t is not None]

    def __enter__(self):
        self.side.wait_stream(self.main)
        for t in self.reads:
            t.record_stream(self.side)
        return (self.main, self.side)

    def __exit__(self, *exc):
        self.main.wait_stream(self.side)
        return False


def _forward_raw(plan, graph, ranges: RangePlan, x, y, hidden, weight, bias, mask):
    """x [N_src, NX*C]; y, hidden, mask in slot order."""
    lib, dev = _lib.lib(), x.device
    width = plan.full_out_width
    out = torch.empty(graph.nodes_dst, width, device=dev, dtype=torch.float32)
    rows = ranges.max_rows
    # one gate (and bond) buffer per stream, reused by that stream's ranges in its own order
    gbuf = [torch.empty(rows, plan.full_gate_width, device=dev, dtype=torch.float32) for _ in range(2)]
    bw = bond_width(plan)
    bbuf = [torch.empty(rows, bw, device=dev, dtype=torch.float32) if bw else None for _ in range(2)]
    with _TwoStreams(dev, (x, y, hidden, weight, bias, mask, out, gbuf[1], bbuf[1])) as streams:
        for i, ((n0, n1, s0, s1), rowptr) in enumerate(zip(ranges.ranges, ranges.rowptr)):
            k = i % 2
            with torch.cuda.stream(streams[k]):
                if s1 == s0:
                    out[n0:n1].zero_()
                    continue
                g = _range_gates_into(gbuf[k], hidden, weight, bias, mask, s0, s1)
                bonds = _range_bonds(plan, y, s0, s1, bbuf[k])
                _lib.check(lib.ictc_hip_message_forward(
                    ctypes.byref(plan.desc), x.data_ptr(), bonds.data_ptr(), g.data_ptr(),
                    ranges.src_sorted[s0:s1].data_ptr(), rowptr.data_ptr(), None, out[n0:n1].data_ptr(),
                    graph.nodes_src, n1 - n0, s1 - s0, _lib.stream_of(dev)), "ictc_hip_message_forward")
    return out


def _backward_raw(plan, graph, ranges: RangePlan, need, x, y, hidden, weight, bias, mask, go):
    """First-order adjoints (dx, dy, dhidden, dweight, dbias), y/hidden/dy/dhidden in slot order."""
    nx, ny, nh, nw, nb = need
    lib = _lib.lib()
    dev = x.device
    need_dg = nh or nw or nb
    nch = lib.ictc_hip_message_chunks(plan.channels)
    dy = torch.empty(y.shape[0], plan.y_width, device=dev, dtype=torch.float32) if ny else None
    dyp = torch.empty(y.shape[0], nch, plan.y_width, device=dev, dtype=torch.float32) if ny else None
    dh = torch.empty_like(hidden) if nh else None
    # the range products dg_r @ W read W column-major (copied once here, not per range): 47 vs
    # 130 us for a 16,384-row range of the cfg-4 shape
    weight_cm = weight.t().contiguous().t() if nh else None
    rows = ranges.max_rows

    def buffers():
        """One stream's range buffers and its node-, weight- and bias-gradient accumulators."""
        return dict(g=torch.empty(rows, plan.full_gate_width, device=dev, dtype=torch.float32),
                    dg=torch.empty(rows, plan.full_gate_width, device=dev, dtype=torch.float32) if need_dg else None,
                    dxe=torch.empty(rows, plan.x_width, device=dev, dtype=torch.float32) if nx else None,
                    part=torch.empty_like(x) if nx else None, dx=torch.zeros_like(x) if nx else None,
                    dw=torch.zeros_like(weight) if nw else None,
                    db=torch.zeros_like(bias) if (nb and bias is not None) else None)
    buf = [buffers(), buffers()]
    reads = (x, y, hidden, weight, bias, mask, go, weight_cm, dyp, dh, *buf[1].values())
    with _TwoStreams(dev, reads) as streams:
        for i, ((n0, n1, s0, s1), rowptr, (rp_src, perm_src)) in enumerate(
                zip(ranges.ranges, ranges.rowptr, ranges.source_csr)):
            r = s1 - s0
            if r == 0:
                continue
            bk = buf[i % 2]
            with torch.cuda.stream(streams[i % 2]):
                stream = _lib.stream_of(dev)
                g = _range_gates_into(bk["g"], hidden, weight, bias, mask, s0, s1)
                dg = bk["dg"][:r] if need_dg else None
                dxe = bk["dxe"][:r] if nx else None
                _lib.check(lib.ictc_hip_message_edge_grad(
                    ctypes.byref(plan.desc), x.data_ptr() if (ny or need_dg) else None, y[s0:s1].data_ptr(),
                    g.data_ptr(), go[n0:n1].data_ptr(), ranges.src_sorted[s0:s1].data_ptr(), rowptr.data_ptr(), None,
                    _lib.ptr(dyp[s0:s1] if ny else None), _lib.ptr(dg), _lib.ptr(dxe), graph.nodes_src, n1 - n0, r,
                    0, stream), "ictc_hip_message_edge_grad")
                if need_dg:
                    if mask is not None:
                        dg *= mask[s0:s1].unsqueeze(1)
                    if nh:
                        sgemm_into(dg, weight_cm, dh[s0:s1])
                    if nw:
                        bk["dw"] += mm(dg.t(), hidden[s0:s1])
                    if bk["db"] is not None:
                        bk["db"] += dg.sum(0)
                if nx:
                    _lib.check(lib.ictc_hip_message_node_grad(
                        ctypes.byref(plan.desc), dxe.data_ptr(), rp_src.data_ptr(), _lib.ptr(perm_src),
                        bk["part"].data_ptr(), graph.nodes_src, r, stream), "ictc_hip_message_node_grad")
                    bk["dx"] += bk["part"]
    if ny:   # channel-chunk partials of every range, summed once
        if nch == 1:
            dy.copy_(dyp[:, 0])
        else:
            torch.sum(dyp, 1, out=dy)
    # the two streams' partial sums, in a fixed order (the same on every run)
    dx = buf[0]["dx"] + buf[1]["dx"] if nx else None
    dw = buf[0]["dw"] + buf[1]["dw"] if nw else None
    db = buf[0]["db"] + buf[1]["db"] if buf[0]["db"] is not None else None
    return dx, dy, dh, dw, db


class _RadialMessage(torch.autograd.Function):
    @staticmethod
    def forward(ctx, plan, graph, ranges, x, y, hidden, weight, bias, mask):
        ctx.plan, ctx.graph, ctx.ranges = plan, graph, ranges
        ctx.has_bias = bias is not None
        ctx.save_for_backward(x, y, hidden, weight, bias, mask)
        return _forward_raw(plan, graph, ranges, x, y, hidden, weight, bias, mask)

    @staticmethod
    def backward(ctx, go):
        x, y, hidden, weight, bias, mask = ctx.saved_tensors
        need = list(required_gradients((x, y, hidden, weight, bias if ctx.has_bias else weight),
                                       ctx.needs_input_grad[3:8]))
        if not ctx.has_bias:
            need[4] = False
        if go is None or not any(need):
            return (None,) * 9
        go = go.contiguous()
        plan, graph = ctx.plan, ctx.graph
        if not torch.is_grad_enabled():
            dx, dy, dh, dw, db = _backward_raw(plan, graph, ctx.ranges, need, x, y, hidden, weight,
                                               bias, mask, go)
            return None, None, None, dx, dy, dh, dw, db, None
        # differentiated backward: full gates, ordinary (differentiable) message adjoint
        gates = mm(hidden, weight.t())
        if bias is not None:
            gates = gates + bias
        if mask is not None:
            gates = gates * mask.unsqueeze(1)
        sorted_graph = ctx.ranges.sorted_graph(graph)
        dx, dy, dg = vjp(plan, sorted_graph, (need[0], need[1], need[2] or need[3] or need[4]), x, y,
                         gates.contiguous(), go)
        dh = dw = db = None
        if dg is not None:
            if mask is not None:
                dg = dg * mask.unsqueeze(1)
            dh = mm(dg, weight) if need[2] else None
            dw = mm(dg.t(), hidden) if need[3] else None
            db = dg.sum(0) if need[4] else None
        return None, None, None, dx, dy, dh, dw, db, None


def _sorted_graph(self, graph: MessageGraph) -> MessageGraph:
    """The graph with its edges renumbered in slot order (dst-sorted: no receiver permutation)."""
    sg = getattr(self, "_sorted", None)
    if sg is None:
        dst_sorted = graph.dst if graph.perm_dst is None else graph.dst.index_select(0, graph.perm_dst)
        sg = MessageGraph(self.src_sorted, dst_sorted.contiguous(), graph.nodes_src, graph.nodes_dst)
        self._sorted = sg
    return sg


RangePlan.sorted_graph = _sorted_graph


def packed_radial_graph_message(plan: TensorProductPlan, features: torch.Tensor, harmonics: torch.Tensor,
                                hidden: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                                src: torch.Tensor, dst: torch.Tensor, *, nodes_dst: Optional[int] = None,
                                mask: Optional[torch.Tensor] = None, edge_chunk_size: int = 16384) -> torch.Tensor:
    """Packed ir_mul message whose gates are ``hidden @ weight^T + bias`` (``weight`` [P_full*C, H],
    rows in the kernels' full path order with any path weights folded in), produced one receiver
    range of at most ``edge_chunk_size`` edges at a time.  features [N_src, C(L_in+1)^2],
    harmonics [E, (L_e+1)^2], hidden [E, H], src/dst int64 [E], mask [E] -> [N_dst, NOC*C]."""
    if not isinstance(edge_chunk_size, int) or isinstance(edge_chunk_size, bool) or edge_chunk_size < 1:
        raise ValueError("Edge chunk size must be positive")
    nodes_src = features.shape[0]
    nodes_dst = nodes_src if nodes_dst is None else int(nodes_dst)
    edges = src.numel()
    if hidden.ndim != 2 or hidden.shape[0] != edges or weight.shape != (plan.full_gate_width, hidden.shape[1]):
        raise ValueError("Expected hidden [E,H] and weight [P*C,H]")
    if bias is not None and bias.shape != (plan.full_gate_width,):
        raise ValueError("Expected bias [P*C]")
    graph = message_graph(src, dst, nodes_src, nodes_dst)
    ranges = range_plan(graph, edge_chunk_size)
    m = None if mask is None else _slot_order(mask.reshape(edges).to(torch.float32), graph).contiguous()
    y = _slot_order(harmonics, graph).contiguous()
    h = _slot_order(hidden, graph).contiguous()
    return _RadialMessage.apply(plan, graph, ranges, features.contiguous(), y, h, weight.contiguous(),
                                None if bias is None else bias.contiguous(), m)


def fold_projection(owner, plan: TensorProductPlan, weight: torch.Tensor, bias: Optional[torch.Tensor]):
    """A radial projection's weight [P*C, H] and bias [P*C] (owner path order) with the owner's
    path weights folded in and the rows moved to the kernels' full path order (zero rows for
    paths the owner leaves out), as the gates the message kernels read."""
    c, p = owner.channels, owner.num_paths
    weight = weight.reshape(p, c, -1)
    bias = None if bias is None else bias.reshape(p, c)
    w = owner.weight              # always folded (a [P, C, H] product), so every change is seen
    weight = weight * w[:, :, None]
    bias = None if bias is None else bias * w
    if not plan.is_full:
        slots = torch.tensor(plan.slot_of_path, device=weight.device)
        full = len(plan.full_paths)
        weight = weight.new_zeros(full, c, weight.shape[2]).index_copy(0, slots, weight)
        bias = None if bias is None else bias.new_zeros(full, c).index_copy(0, slots, bias)
    return weight.reshape(-1, weight.shape[2]), None if bias is None else bias.reshape(-1)


def radial_graph_message(owner, features, harmonics, radial, edge_features, src, dst, mask=None, *,
                         edge_chunk_size=None):
    """The reference's radial-streaming message hook (``capacity_message.py:109-179``, called from
    the interaction block at ``pure_cartesian_ictd_fix.py:1787-1793``): ``radial`` is the radial MLP
    (an ``nn.Sequential`` ending in an ``nn.Linear`` with P*C outputs); its prefix runs once and
    its last Linear is produced one receiver range (at most ``edge_chunk_size`` edges, default
    16,384) at a time inside the message, so the ``[E, P*C]`` gates never exist whole.  Returns
    {l: [N_dst, count_l*C, 2l+1]}, or None (not handled: the caller computes the gates and calls
    ``graph_message``) for an empty graph, a radial module of another form, a mask that needs a
    gradient, or hooks on the radial modules."""
    from .runtime import require_gpu_fp32
    from .tensor_product import (check_message_operands, destination_nodes, owner_degrees, pack_features,
                                 pack_harmonics, packed_to_blocks)
    if not src.numel():
        return None
    if (type(radial) is not torch.nn.Sequential or not len(radial) or "forward" in radial.__dict__
            or type(radial[-1]) is not torch.nn.Linear):
        return None
    projection = radial[-1]
    if (mask is not None and mask.requires_grad) or projection.out_features != owner.num_paths * owner.channels:
        return None
    if any(m._forward_hooks or m._forward_pre_hooks or m._backward_hooks or m._backward_pre_hooks
           for m in (radial, projection)):
        return None
    sample = next(iter(features.values()))
    nodes = sample.shape[0]
    edges = check_message_operands(owner, sample.device, [v.shape[0] for v in harmonics.values()], None,
                                   src, dst, mask, edge_chunk_size)
    require_gpu_fp32(owner.weight, projection.weight, edge_features, *features.values(), *harmonics.values())
    hidden = edge_features
    for layer in list(radial.children())[:-1]:
        hidden = layer(hidden)
    if hidden.ndim != 2 or hidden.shape != (edges, projection.in_features):
        raise ValueError("Radial prefix must return one hidden-feature row per edge")
    x = pack_features(owner, features, nodes)
    y = pack_harmonics(owner, harmonics, edges, sample)
    plan = owner.hip_plan(*owner_degrees(owner))
    weight, bias = fold_projection(owner, plan, projection.weight, projection.bias)
    out = packed_radial_graph_message(plan, x, y, hidden, weight, bias, src, dst,
                                      nodes_dst=destination_nodes(owner, nodes), mask=mask,
                                      edge_chunk_size=16384 if edge_chunk_size is None else edge_chunk_size)
    if not plan.is_full:
        keep = torch.tensor(plan.output_rows, device=out.device)
        out = out.reshape(out.shape[0], -1, plan.channels).index_select(1, keep).reshape(out.shape[0], -1)
    return packed_to_blocks(plan, out)
