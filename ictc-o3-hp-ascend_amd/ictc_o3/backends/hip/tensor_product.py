"""Channelwise path-preserving tensor product on the HIP kernels, with autograd to
any order.

The map out = F(x, Y, g) is trilinear in (features x, harmonics Y, gates g), so
its VJP (Gx, GY, Gg) is trilinear as well and every mixed derivative is one of
the same two kernels with an operand substituted -- the bilinear-substitution
scheme of the reference's structured adjoint (``backends/ascend/structured_product.py:97-183``):

    <hx, Gx(Y,g,o)> : d/dY = GY(hx,g,o),  d/dg = Gg(hx,Y,o),  d/do = F(hx,Y,g)
    <hY, GY(x,g,o)> : d/dx = Gx(hY,g,o),  d/dg = Gg(x,hY,o),  d/do = F(x,hY,g)
    <hg, Gg(x,Y,o)> : d/dx = Gx(Y,hg,o),  d/dY = GY(x,hg,o),  d/do = F(x,Y,hg)

Both Functions call each other through ``.apply``, so ``create_graph=True`` chains
to third and higher order with no separate code path.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Optional, Sequence, Tuple

import torch

from ... import _lib
from ...autograd.adjoint_requirements import required_gradients
from ...basis.ictd_irreps import PathPlan, triangle_paths


MAX_DEGREE = 6            # degree-generic kernels (run-time path tables)
COMPILED_MAX_DEGREE = 3   # per-degree kernels


def _canonical_layout(full):
    """First output component of each full-set path: ascending l3, enumeration order
    within one l3 (the owner's path_offset order)."""
    offsets, acc = [0] * len(full), 0
    for l in range(max(p[2] for p in full) + 1):
        for i, p in enumerate(full):
            if p[2] == l:
                offsets[i] = acc
                acc += 2 * l + 1
    return offsets, acc


class TensorProductPlan:
    """Immutable launch description of one owner (paths, channels, degrees).

    The kernels run the full triangle/parity path set of (input_lmax, edge_lmax,
    output_lmax).  An owner with a path subset runs the full set with zero gates on the
    absent paths and keeps only its own output rows.  Degrees up to 3 run the per-degree
    kernels; a degree of 4 to 6 runs the degree-generic ones (``generic``), which have no
    fused message tangent kernels."""

    def __init__(self, paths: Sequence[Tuple[int, int, int]], channels: int, input_lmax: int,
                 edge_lmax: int, lmax: Optional[int] = None):
        paths = [tuple(int(v) for v in p) for p in paths]
        if not paths:
            raise ValueError("a tensor product needs at least one path")
        self.channels, self.input_lmax, self.edge_lmax = int(channels), int(input_lmax), int(edge_lmax)
        self.output_lmax = max(p[2] for p in paths)
        self.lmax = max(lmax if lmax is not None else 0, self.input_lmax, self.edge_lmax, self.output_lmax)
        if any(i > self.input_lmax or j > self.edge_lmax for i, j, _ in paths):
            raise ValueError("Declared input degrees must cover every tensor-product path")
        if max(self.input_lmax, self.edge_lmax, self.output_lmax) > MAX_DEGREE:
            raise ValueError(f"the HIP tensor-product kernels support degrees up to {MAX_DEGREE}")
        self.generic = max(self.input_lmax, self.edge_lmax, self.output_lmax) > COMPILED_MAX_DEGREE
        self.plan = PathPlan(paths, channels)
        self.plan.path_counts_by_l = {l: self.plan.path_counts_by_l.get(l, 0) for l in range(self.lmax + 1)}
        self.paths = self.plan.paths
        full = triangle_paths(self.input_lmax, self.edge_lmax, self.output_lmax)
        missing = set(paths) - set(full)
        if missing:
            raise ValueError(f"paths {sorted(missing)} violate the triangle/parity rule")
        index = {p: i for i, p in enumerate(paths)}
        offsets, noc = _canonical_layout(full)
        desc = _lib.TpDesc()
        desc.channels = self.channels
        desc.input_lmax, desc.edge_lmax, desc.output_lmax = self.input_lmax, self.edge_lmax, self.output_lmax
        desc.num_paths = len(full)
        desc.out_components = noc
        for s, p in enumerate(full):
            desc.gate_index[s] = s
            desc.out_offset[s] = offsets[s]
            desc.scale[s] = self.plan.scales[index[p]] if p in index else 0.0
        self.desc = desc
        self.num_paths = len(paths)
        self.full_paths = full
        self.is_full = paths == full
        self.x_width = self.channels * (self.input_lmax + 1) ** 2
        self.y_width = (self.edge_lmax + 1) ** 2
        self.gate_width = self.num_paths * self.channels
        self.out_width = self.plan.output_components * self.channels
        self.full_gate_width = len(full) * self.channels
        self.full_out_width = noc * self.channels
        if not self.is_full:
            # owner path i -> full slot; owner output rows -> full output rows
            self.slot_of_path = [full.index(p) for p in paths]
            rows = []
            for l in range(self.output_lmax + 1):
                for s, p in enumerate(full):
                    if p[2] == l and p in index:
                        rows.extend(range(offsets[s], offsets[s] + 2 * l + 1))
            self.output_rows = rows

    def set_scale(self, path_index: int, value: float) -> None:
        self.desc.scale[self.full_paths.index(self.paths[path_index])] = float(value)


def _forward_raw(plan: TensorProductPlan, x, y, g) -> torch.Tensor:
    rows = x.shape[0]
    out = torch.empty(rows, plan.full_out_width, device=x.device, dtype=torch.float32)
    _lib.check(_lib.lib().ictc_hip_tp_forward(ctypes.byref(plan.desc), x.data_ptr(), y.data_ptr(),
                                               g.data_ptr(), out.data_ptr(), rows,
                                               _lib.stream_of(x.device)), "ictc_hip_tp_forward")
    return out


def _backward_raw(plan: TensorProductPlan, need, x, y, g, go):
    rows = go.shape[0]
    dev = go.device
    dx = torch.empty(rows, plan.x_width, device=dev, dtype=torch.float32) if need[0] else None
    dy = torch.empty(rows, plan.y_width, device=dev, dtype=torch.float32) if need[1] else None
    dg = torch.empty(rows, plan.full_gate_width, device=dev, dtype=torch.float32) if need[2] else None
    if any(need):
        _lib.check(_lib.lib().ictc_hip_tp_backward(
            ctypes.byref(plan.desc), x.data_ptr(), y.data_ptr(),
            g.data_ptr(), go.data_ptr(), _lib.ptr(dx), _lib.ptr(dy), _lib.ptr(dg), rows,
            _lib.stream_of(dev)), "ictc_hip_tp_backward")
    return dx, dy, dg


def _add(acc, value):
    if value is None:
        return acc
    return value if acc is None else acc + value


class _Forward(torch.autograd.Function):
    @staticmethod
    def forward(ctx, plan, x, y, g):
        ctx.plan = plan
        ctx.save_for_backward(x, y, g)
        return _forward_raw(plan, x, y, g)

    @staticmethod
    def backward(ctx, go):
        x, y, g = ctx.saved_tensors
        need = required_gradients((x, y, g), ctx.needs_input_grad[1:])
        if go is None or not any(need):
            return None, None, None, None
        dx, dy, dg = vjp(ctx.plan, need, x, y, g, go.contiguous())
        return None, dx, dy, dg


class _Backward(torch.autograd.Function):
    """(dx, dY, dg) = VJP(x, Y, g; go); outputs not requested are empty placeholders."""

    @staticmethod
    def forward(ctx, plan, need, x, y, g, go):
        ctx.plan, ctx.need = plan, need
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(x, y, g, go)
        dx, dy, dg = _backward_raw(plan, need, x, y, g, go)
        empty = go.new_empty(0)
        outs = tuple(t if t is not None else empty for t in (dx, dy, dg))
        for t, n in zip(outs, need):
            if not n:
                ctx.mark_non_differentiable(t)
        return outs

    @staticmethod
    def backward(ctx, hx, hy, hg):
        plan, need_out = ctx.plan, ctx.need
        x, y, g, go = ctx.saved_tensors
        hx = hx if need_out[0] else None
        hy = hy if need_out[1] else None
        hg = hg if need_out[2] else None
        nx, ny, ng, no = required_gradients((x, y, g, go), ctx.needs_input_grad[2:])
        gx = gy = gg = ggo = None
        if hx is not None:
            hx = hx.contiguous()
            if ny or ng:
                _, a, b = vjp(plan, (False, ny, ng), hx, y, g, go)
                gy, gg = _add(gy, a), _add(gg, b)
            if no:
                ggo = _add(ggo, _Forward.apply(plan, hx, y, g))
        if hy is not None:
            hy = hy.contiguous()
            if nx or ng:
                a, _, b = vjp(plan, (nx, False, ng), x, hy, g, go)
                gx, gg = _add(gx, a), _add(gg, b)
            if no:
                ggo = _add(ggo, _Forward.apply(plan, x, hy, g))
        if hg is not None:
            hg = hg.contiguous()
            if nx or ny:
                a, b, _ = vjp(plan, (nx, ny, False), x, y, hg, go)
                gx, gy = _add(gx, a), _add(gy, b)
            if no:
                ggo = _add(ggo, _Forward.apply(plan, x, y, hg))
        return None, None, gx, gy, gg, ggo


def vjp(plan, need, x, y, g, go):
    """(dx, dY, dg) with None for entries not in ``need``; differentiable."""
    need = tuple(bool(n) for n in need)
    if not any(need):
        return None, None, None
    if not torch.is_grad_enabled():       # nothing recorded: skip the autograd Function
        return _backward_raw(plan, need, x, y, g, go)
    outs = _Backward.apply(plan, need, x, y, g, go)
    return tuple(o if n else None for o, n in zip(outs, need))


def packed_tensor_product(plan: TensorProductPlan, features: torch.Tensor, harmonics: torch.Tensor,
                          gates: torch.Tensor) -> torch.Tensor:
    """Packed ir_mul TP: features [E, C(L_in+1)^2], harmonics [E,(L_e+1)^2],
    gates [E, P*C] (path weights already folded in) -> [E, NOC*C]."""
    if plan.is_full:
        return _Forward.apply(plan, features.contiguous(), harmonics.contiguous(), gates.contiguous())
    rows, c = gates.shape[0], plan.channels
    slots = torch.tensor(plan.slot_of_path, device=gates.device)
    full_gates = gates.new_zeros(rows, len(plan.full_paths), c).index_copy(
        1, slots, gates.reshape(rows, plan.num_paths, c))
    out = _Forward.apply(plan, features.contiguous(), harmonics.contiguous(),
                         full_gates.reshape(rows, len(plan.full_paths) * c))
    keep = torch.tensor(plan.output_rows, device=gates.device)
    return out.reshape(rows, -1, c).index_select(1, keep).reshape(rows, len(plan.output_rows) * c)


def blocks_to_packed(blocks: Dict[int, torch.Tensor], lmax: int) -> torch.Tensor:
    """{l: [E,C,2l+1]} -> ir_mul packed [E, C(lmax+1)^2]."""
    rows = next(iter(blocks.values())).shape[0]
    return torch.cat([blocks[l].transpose(1, 2).reshape(rows, blocks[l].shape[1] * (2 * l + 1))
                      for l in range(lmax + 1)], -1)


def packed_to_blocks(plan: TensorProductPlan, out: torch.Tensor) -> Dict[int, torch.Tensor]:
    """ir_mul packed output -> {l: [E, count_l*C, 2l+1]} (owner dict layout)."""
    result, off, rows, c = {}, 0, out.shape[0], plan.channels
    for l in range(plan.lmax + 1):
        count, width = plan.plan.path_counts_by_l.get(l, 0), 2 * l + 1
        span = count * c * width
        result[l] = out[:, off:off + span].reshape(rows, count, width, c).transpose(2, 3).reshape(
            rows, count * c, width)
        off += span
    return result


# ----------------------------------------------------------------------------- reference hooks
def owner_degrees(owner) -> Tuple[int, int]:
    """(input lmax, edge lmax) the owner's paths need."""
    return max(p[0] for p in owner.paths), max(p[1] for p in owner.paths)


def pack_features(owner, features: Dict[int, torch.Tensor], rows: int) -> torch.Tensor:
    """{l: [rows, C, 2l+1]} -> packed ir_mul [rows, C(L_in+1)^2]; degrees the dict leaves out are
    zero (the reference skips their paths)."""
    if not features:
        raise ValueError("Feature blocks must not be empty")
    c = owner.channels
    for l, value in features.items():
        if value.ndim != 3 or value.shape != (rows, c, 2 * l + 1):
            raise ValueError("Feature blocks must have shape [N,C,2l+1]")
    sample = next(iter(features.values()))
    input_lmax = owner_degrees(owner)[0]
    return blocks_to_packed({l: features[l] if l in features else sample.new_zeros(rows, c, 2 * l + 1)
                             for l in range(input_lmax + 1)}, input_lmax)


def pack_harmonics(owner, harmonics: Dict[int, torch.Tensor], rows: int, like: torch.Tensor) -> torch.Tensor:
    """{l: [rows, 1, 2l+1]} -> [rows, (L_e+1)^2]; left-out degrees are zero."""
    for l, value in harmonics.items():
        if value.shape not in ((rows, 1, 2 * l + 1), (rows, 2 * l + 1)):
            raise ValueError("Harmonic blocks must have shape [E,1,2l+1]")
    edge_lmax = owner_degrees(owner)[1]
    return torch.cat([harmonics[l].reshape(rows, 2 * l + 1) if l in harmonics else like.new_zeros(rows, 2 * l + 1)
                      for l in range(edge_lmax + 1)], -1)


def tensor_product(owner, features, harmonics, gates=None):
    """The reference's TP hook (``backends/ascend/tensor_product.py:89-125``, called from the owner's
    forward, ``ictd_irreps.py:2773-2775``): owner = EdgeWeightedPathPreservingTensorProduct,
    features {l: [E,C,2l+1]}, harmonics {l: [E,1,2l+1]}, gates [E,P*C], [E,P,C] or None (the
    owner's weight alone) -> {l: [E, count_l*C, 2l+1]} for every l <= owner.lmax."""
    from .runtime import require_gpu_fp32
    sample = next(iter(features.values()))
    rows, channels = sample.shape[0], owner.channels
    if gates is not None and gates.shape not in ((rows, owner.num_paths * channels),
                                                 (rows, owner.num_paths, channels)):
        raise ValueError("External gates must have shape [E,P*C] or [E,P,C]")
    require_gpu_fp32(owner.weight, *features.values(), *harmonics.values(), *(() if gates is None else (gates,)))
    x = pack_features(owner, features, rows)
    y = pack_harmonics(owner, harmonics, rows, sample)
    plan = owner.hip_plan(*owner_degrees(owner))
    return packed_to_blocks(plan, packed_tensor_product(plan, x, y, owner.effective_gates(gates, rows)))


def destination_nodes(owner, source_nodes: int) -> int:
    """Owned destinations of a larger source halo (reference ``tensor_product.py:151-156``):
    ``owner._ascend_destination_nodes`` (or ``_destination_nodes``), default all source nodes."""
    nodes = getattr(owner, "_destination_nodes", getattr(owner, "_ascend_destination_nodes", source_nodes))
    if not isinstance(nodes, int) or isinstance(nodes, bool) or not 0 <= nodes <= source_nodes:
        raise ValueError("Destination node count must be between zero and the source node count")
    return nodes


def check_message_operands(owner, device, harmonics_rows, gates, src, dst, mask, edge_chunk_size):
    """Shared argument checks of the message hooks (reference ``tensor_product.py:159-218``,
    ``ascendc/graph.py:7-19``)."""
    from .runtime import require_gpu_fp32
    if edge_chunk_size is not None and (not isinstance(edge_chunk_size, int) or isinstance(edge_chunk_size, bool)
                                        or edge_chunk_size < 1):
        raise ValueError("Edge chunk size must be positive")
    for value in (src, dst):
        if value.ndim != 1 or value.dtype != torch.int64 or value.device != device:
            raise ValueError("Graph indices must be int64 vectors on the GPU")
    if dst.shape != src.shape:
        raise ValueError("Source and destination index shapes must match")
    edges = src.numel()
    if any(rows != edges for rows in harmonics_rows):
        raise ValueError("Harmonic row counts must match graph edges")
    if gates is not None:
        if gates.shape not in ((edges, owner.num_paths * owner.channels), (edges, owner.num_paths, owner.channels)):
            raise ValueError("External gates must have shape [E,P*C] or [E,P,C]")
        require_gpu_fp32(gates)
    if mask is not None:
        if mask.shape not in ((edges,), (edges, 1)) or mask.device != device:
            raise ValueError("Expected an edge mask [E] or [E,1] on the feature device")
        require_gpu_fp32(mask)
    return edges


def message_gates(owner, gates: Optional[torch.Tensor], edges: int):
    """(gates [E, P*C], receiver-row weight or None) for the message kernels.  The owner's
    per-(path, channel) weight is applied to the message's receiver rows
    (``owner.output_weight_rows``, always, so every change of the weight is seen) rather than
    folded into every edge's gates; ``gates=None`` means the weight alone."""
    if gates is None:
        return owner.effective_gates(None, edges), None
    return gates.reshape(edges, owner.num_paths * owner.channels), owner.output_weight_rows()


def graph_message(owner, features, harmonics, gates, src, dst, mask=None, *, edge_chunk_size=16384):
    """The reference's message hook (``backends/ascend/tensor_product.py:159-218``, called by the
    interaction block at ``pure_cartesian_ictd_fix.py:1787-1800``):
    node_out[n] = sum_{e: dst(e) = n} mask_e TP(features[src e], harmonics[e], gates[e]) as
    {l: [N_dst, count_l*C, 2l+1]}.  One fused HIP kernel family (receiver CSR, no atomics, no
    per-edge messages in HBM); ``edge_chunk_size`` is validated and otherwise unused."""
    from .graph_message import packed_graph_message
    from .runtime import require_gpu_fp32
    sample = next(iter(features.values()))
    nodes = sample.shape[0]
    edges = check_message_operands(owner, sample.device, [v.shape[0] for v in harmonics.values()], gates,
                                   src, dst, mask, edge_chunk_size)
    require_gpu_fp32(owner.weight, *features.values(), *harmonics.values())
    x = pack_features(owner, features, nodes)
    y = pack_harmonics(owner, harmonics, edges, sample)
    plan = owner.hip_plan(*owner_degrees(owner))
    gates, row_weight = message_gates(owner, gates, edges)
    out = packed_graph_message(plan, x, y, gates, src, dst, nodes_dst=destination_nodes(owner, nodes), mask=mask)
    return packed_to_blocks(plan, out if row_weight is None else out * row_weight)
