"""Public ictc_o3 operators on MI355X (gfx950) HIP kernels.

Same names, signatures, layouts and autograd semantics as the reference's
``ictc_o3/operators.py`` (``__all__`` at ``:232-234``); the device is a ROCm GPU
(torch device type ``"cuda"``) instead of an Ascend NPU.  Every operator runs its
arithmetic in ``libictc_hip.so``; there is no CPU or eager fallback.
"""
from __future__ import annotations

import torch

from ictc_o3.backends.hip.linear import channel_linear, species_channel_linear
from ictc_o3.backends.hip.runtime import require_gpu_fp32, strict_fp32


def _degree(value, name):
    if not isinstance(value, int) or isinstance(value, bool) or value < 0:
        raise ValueError(f"{name} must be a nonnegative integer")


def _positive_integer(value, name):
    if not isinstance(value, int) or isinstance(value, bool) or value < 1:
        raise ValueError(f"{name} must be a positive integer")


def _require_gpu_device(device) -> torch.device:
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("This operator factory requires a ROCm GPU device")
    return device


class EdgeTensorProduct(torch.nn.Module):
    """Path-preserving TP with live external gates (reference ``operators.py:19-139``).

    ``layout="ir_mul"`` stores each degree as [angular, channel] (channel-contiguous,
    the kernels' native layout); ``"mul_ir"`` stores [channel, angular] and is
    transposed around the kernels.  Output multiplicities keep the owner's path order.
    """

    def __init__(self, tp, *, input_lmax, edge_lmax, layout="ir_mul"):
        super().__init__()
        from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
        if not isinstance(tp, EdgeWeightedPathPreservingTensorProduct):
            raise TypeError("Expected an ICTC path-preserving tensor product")
        _degree(input_lmax, "input_lmax")
        _degree(edge_lmax, "edge_lmax")
        require_gpu_fp32(tp.weight)
        if layout not in ("ir_mul", "mul_ir"):
            raise ValueError("layout must be ir_mul or mul_ir")
        if tp.internal_compute_dtype != torch.float32:
            raise ValueError("Tensor-product internal compute dtype must be FP32")
        if not tp.paths or any(i > input_lmax or j > edge_lmax for i, j, _ in tp.paths):
            raise ValueError("Declared input degrees must cover every tensor-product path")
        strict_fp32()
        self.tp, self.input_lmax, self.edge_lmax, self.layout = tp, input_lmax, edge_lmax, layout
        self.plan = tp.hip_plan(input_lmax, edge_lmax)

    @classmethod
    def create(cls, *, channels=64, input_lmax=2, edge_lmax=2, output_lmax=None, layout="ir_mul",
               device="cuda"):
        _positive_integer(channels, "channels")
        _degree(input_lmax, "input_lmax")
        _degree(edge_lmax, "edge_lmax")
        output_lmax = input_lmax if output_lmax is None else output_lmax
        _degree(output_lmax, "output_lmax")
        device = _require_gpu_device(device)
        from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
        paths = [(i, j, k) for i in range(input_lmax + 1) for j in range(edge_lmax + 1)
                 for k in range(output_lmax + 1) if abs(i - j) <= k <= i + j and (i + j + k) % 2 == 0]
        tp = EdgeWeightedPathPreservingTensorProduct(
            channels=channels, lmax=max(input_lmax, edge_lmax, output_lmax), allowed_paths=paths,
            internal_compute_dtype=torch.float32).to(device=device, dtype=torch.float32)
        with torch.no_grad():
            tp.weight.fill_(1.)
        tp.weight.requires_grad_(False)
        return cls(tp, input_lmax=input_lmax, edge_lmax=edge_lmax, layout=layout)

    @property
    def paths(self):
        return tuple(tuple(p) for p in self.tp.paths)

    @property
    def gate_width(self):
        return self.tp.num_paths * self.tp.channels

    @property
    def output_width(self):
        return sum(count * self.tp.channels * (2 * l + 1) for l, count in self.tp.path_counts_by_l.items())

    def pack_input(self, blocks):
        parts = []
        for l in range(self.input_lmax + 1):
            value = blocks[l]
            if value.shape[1:] != (self.tp.channels, 2 * l + 1):
                raise ValueError("Input block must have shape [E,C,2*l+1]")
            if self.layout == "ir_mul":
                value = value.transpose(1, 2)
            parts.append(value.reshape(value.shape[0], self.tp.channels * (2 * l + 1)))
        return torch.cat(parts, -1)

    def unpack_output(self, output):
        result, offset = {}, 0
        for l in range(self.tp.lmax + 1):
            count, width = self.tp.path_counts_by_l.get(l, 0), 2 * l + 1
            span = count * self.tp.channels * width
            value = output[:, offset:offset + span]
            if self.layout == "ir_mul":
                value = value.reshape(output.shape[0], count, width, self.tp.channels).transpose(2, 3)
            result[l] = value.reshape(output.shape[0], count * self.tp.channels, width)
            offset += span
        return result

    # -------------------------------------------------------------- layout helpers
    def _to_ir_mul_features(self, features):
        if self.layout == "ir_mul":
            return features.contiguous()
        rows, c, parts, off = features.shape[0], self.tp.channels, [], 0
        for l in range(self.input_lmax + 1):
            width = c * (2 * l + 1)
            parts.append(features[:, off:off + width].reshape(rows, c, 2 * l + 1).transpose(1, 2)
                         .reshape(rows, width))
            off += width
        return torch.cat(parts, -1)

    def _from_ir_mul_output(self, out):
        if self.layout == "ir_mul":
            return out
        rows, c, parts, off = out.shape[0], self.tp.channels, [], 0
        for l in range(self.tp.lmax + 1):
            count, width = self.tp.path_counts_by_l.get(l, 0), 2 * l + 1
            span = count * c * width
            parts.append(out[:, off:off + span].reshape(rows, count, width, c).transpose(2, 3)
                         .reshape(rows, span))
            off += span
        return torch.cat(parts, -1)

    def _check(self, features, harmonics, gates):
        require_gpu_fp32(features, harmonics, self.tp.weight, *(() if gates is None else (gates,)))
        if features.ndim != 2 or features.shape[1] != self.tp.channels * (self.input_lmax + 1) ** 2:
            raise ValueError("Packed features must have shape [E,C*(L_in+1)^2]")
        rows = features.shape[0]
        if harmonics.shape != (rows, (self.edge_lmax + 1) ** 2):
            raise ValueError("Harmonics must have shape [E,(L_edge+1)^2]")
        if gates is not None and gates.shape not in ((rows, self.gate_width),
                                                     (rows, self.tp.num_paths, self.tp.channels)):
            raise ValueError("External gates must have shape [E,P*C] or [E,P,C]")
        return rows

    def forward(self, features, harmonics, gates):
        from ictc_o3.backends.hip.tensor_product import packed_tensor_product
        rows = self._check(features, harmonics, gates)
        if not rows:
            zero = sum(v.sum() * 0 for v in (features, harmonics, self.tp.weight,
                                             *(() if gates is None else (gates,))))
            return features.new_empty(0, self.output_width) + zero
        out = packed_tensor_product(self.plan, self._to_ir_mul_features(features), harmonics,
                                    self.tp.effective_gates(gates, rows))
        return self._from_ir_mul_output(out)


class PackedGraphMessage(EdgeTensorProduct):
    """Packed node gather, per-edge TP and receiver segmented sum in one HIP kernel
    family (reference ``operators.py:141-163``).

    ``forward(features [N,C(L_in+1)^2], harmonics [E,(L_e+1)^2], gates [E,P*C] or
    [E,P,C], src, dst int64 [E], mask [E] or [E,1] | None) -> [N_dst, output_width]``.
    ``edge_chunk_size`` is accepted for API compatibility; the kernels never
    materialise per-edge messages, so no chunking is needed.  ``N_dst`` defaults to
    the node count and can be lowered through ``tp._destination_nodes`` (owned
    destinations of a larger source halo, reference tensor_product.py:151-156)."""

    def __init__(self, *args, edge_chunk_size=16384, **kwargs):
        super().__init__(*args, **kwargs)
        _positive_integer(edge_chunk_size, "edge_chunk_size")
        self.edge_chunk_size = edge_chunk_size

    @classmethod
    def create(cls, *, edge_chunk_size=16384, **kwargs):
        op = EdgeTensorProduct.create(**kwargs)
        return cls(op.tp, input_lmax=op.input_lmax, edge_lmax=op.edge_lmax,
                   layout=op.layout, edge_chunk_size=edge_chunk_size)

    def _message(self, features, harmonics, gates, src, dst, mask):
        from ictc_o3.backends.hip.graph_message import packed_graph_message
        from ictc_o3.backends.hip.tensor_product import check_message_operands, destination_nodes, message_gates
        edges = check_message_operands(self.tp, features.device, [harmonics.shape[0]], gates, src, dst, mask,
                                       self.edge_chunk_size)
        require_gpu_fp32(features, harmonics, self.tp.weight)
        if features.ndim != 2 or features.shape[1] != self.tp.channels * (self.input_lmax + 1) ** 2:
            raise ValueError("Packed features must have shape [E,C*(L_in+1)^2]")
        if harmonics.shape != (edges, (self.edge_lmax + 1) ** 2):
            raise ValueError("Harmonics must have shape [E,(L_edge+1)^2]")
        nodes = destination_nodes(self.tp, features.shape[0])
        gates, row_weight = message_gates(self.tp, gates, edges)
        out = packed_graph_message(self.plan, self._to_ir_mul_features(features), harmonics, gates, src, dst,
                                   nodes_dst=nodes, mask=mask)
        return out if row_weight is None else out * row_weight

    def forward(self, features, harmonics, gates, src, dst, mask=None):
        return self._from_ir_mul_output(self._message(features, harmonics, gates, src, dst, mask))


class GraphMessage(PackedGraphMessage):
    """Dictionary block interface for the same message map (reference ``operators.py:166-170``):
    features {l: [N,C,2l+1]}, harmonics {l: [E,1,2l+1]} -> {l: [N_dst, count_l*C, 2l+1]}, through
    the ``graph_message`` hook as in the reference."""

    def forward(self, features, harmonics, gates, src, dst, mask=None):
        from ictc_o3.backends.hip.tensor_product import graph_message
        return graph_message(self.tp, features, harmonics, gates, src, dst, mask,
                             edge_chunk_size=self.edge_chunk_size)


def direction_harmonics(directions, lmax, *, policy="auto"):
    """Direction harmonics Y_0..Y_lmax in the ICTC basis, returned as a list of
    [..., 2l+1] tensors (reference ``operators.py:173-186``).  Computed by the HIP
    harmonics kernel, with analytic first and second derivatives."""
    _degree(lmax, "lmax")
    if policy not in ("auto", "generated", "reference"):
        raise ValueError("policy must be auto, generated or reference")
    require_gpu_fp32(directions)
    from ictc_o3.backends.hip.harmonics import direction_harmonics_packed
    packed = direction_harmonics_packed(directions, lmax)
    return [packed[..., l * l:(l + 1) ** 2] for l in range(lmax + 1)]


def configure_symmetric_contraction(module, *, policy="auto", training=False):
    """Select the HIP contraction for a module (reference ``operators.py:189-201``): the bridge-U
    module the factory returns, or the pure-ICTC variant.  Checks the compiled configuration and,
    for the bridge-U module, that its U buffers pass the reconstruction gate."""
    from ictc_o3.ops.symmetric_contraction import (ICTDBridgeUSymmetricContractionSO3,
                                                   ICTDPureUSymmetricContractionSO3)
    if not isinstance(module, (ICTDBridgeUSymmetricContractionSO3, ICTDPureUSymmetricContractionSO3)):
        raise TypeError("Expected an ICTC bridge-U symmetric contraction")
    if policy not in ("auto", "generated", "reference"):
        raise ValueError("policy must be auto, generated or reference")
    if policy == "reference":
        raise ValueError("the reference (eager CPU) contraction is not part of this library")
    require_gpu_fp32(*module.parameters())
    if module.correlation not in (1, 2, 3):
        raise ValueError("symmetric contraction supports correlation 1, 2 and 3")
    strict_fp32()
    module.plan  # compiled configuration check
    if isinstance(module, ICTDBridgeUSymmetricContractionSO3):
        module.weight_table(next(module.parameters()))   # reconstruction gate
    module._ascend_hp = True
    return {"backend": "hip", "selected": "generated"}


def create_symmetric_contraction(*, num_elements, lmax, target_lmax=None, channels=64, correlation=3,
                                 device="cuda", policy="generated", training=False):
    """Factory (reference ``operators.py:204-218``): the bridge-U contraction (U tensors of the
    e3nn generalized coupling folded into the ICTC basis) on the HIP kernels."""
    for value, name in ((num_elements, "num_elements"), (channels, "channels"), (correlation, "correlation")):
        _positive_integer(value, name)
    if correlation not in (1, 2, 3):
        raise ValueError("symmetric contraction supports correlation 1, 2 and 3")
    _degree(lmax, "lmax")
    target_lmax = lmax if target_lmax is None else target_lmax
    _degree(target_lmax, "target_lmax")
    device = _require_gpu_device(device)
    from ictc_o3.ops.symmetric_contraction import ICTDBridgeUSymmetricContractionSO3
    module = ICTDBridgeUSymmetricContractionSO3(num_elements=num_elements, channels=channels, lmax=lmax,
                                                target_lmax=target_lmax, correlation=correlation
                                                ).to(device=device, dtype=torch.float32)
    configure_symmetric_contraction(module, policy=policy, training=training)
    return module


def normalized_silu(features, scale=1.):
    require_gpu_fp32(features)
    if not isinstance(scale, (int, float)) or isinstance(scale, bool):
        raise TypeError("scale must be a fixed numeric scalar")
    return torch.nn.functional.silu(features) * float(scale)


__all__ = ["EdgeTensorProduct", "PackedGraphMessage", "GraphMessage", "direction_harmonics",
           "create_symmetric_contraction", "configure_symmetric_contraction",
           "channel_linear", "species_channel_linear", "normalized_silu", "strict_fp32"]
