"""Oracle: path-preserving channelwise CG tensor product and graph message (CPU).

Restates the reference's CPU path:

* path enumeration  -- ``ictc_o3/operators.py:54-55`` and the ordering filter of
  ``HarmonicPathWeightedTensorProduct.__init__`` (``ictd_irreps.py:2161-2212``);
* path bookkeeping  -- ``EdgeWeightedPathPreservingTensorProduct.__init__``
  (``ictd_irreps.py:2504-2526``);
* CG list / group projectors -- ``_get_cg_list`` / ``_get_proj_group_list``
  (``ictd_irreps.py:2218-2262``);
* forward           -- ``_forward_index_add`` (``ictd_irreps.py:2669-2748``);
* packed layouts    -- ``EdgeTensorProduct.pack_input/_blocks/_harmonics/
  _pack_output/unpack_output`` (``operators.py:77-127``);
* graph message     -- ``graph_message`` CPU semantics
  (``backends/ascend/tensor_product.py:189-218``).

All derivatives (VJP, mixed second order, ...) come from torch autograd
through these eager expressions, as in the reference CPU backend.
Test infrastructure only.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import ictc_basis as basis


def enumerate_paths(input_lmax: int, edge_lmax: int, output_lmax: int) -> List[Tuple[int, int, int]]:
    """Triangle + parity paths (``operators.py:54-55``) in the owner's order
    (l1, l2, l3 ascending; ``ictd_irreps.py:2161-2175``)."""
    lmax = max(input_lmax, edge_lmax, output_lmax)
    allowed = {(i, j, k) for i in range(input_lmax + 1) for j in range(edge_lmax + 1)
               for k in range(output_lmax + 1) if abs(i - j) <= k <= i + j and (i + j + k) % 2 == 0}
    ordered = []
    for l1 in range(lmax + 1):
        for l2 in range(lmax + 1):
            for l3 in range(abs(l1 - l2), min(l1 + l2, lmax) + 1):
                if (l1 + l2 + l3) % 2 == 0 and (l1, l2, l3) in allowed:
                    ordered.append((l1, l2, l3))
    return ordered


class TensorProductOracle:
    """CPU restatement of ``EdgeWeightedPathPreservingTensorProduct`` wrapped by
    ``EdgeTensorProduct`` (``operators.py:19-139``)."""

    def __init__(self, channels: int, input_lmax: int, edge_lmax: int,
                 output_lmax: Optional[int] = None, *, layout: str = "ir_mul",
                 paths: Optional[Sequence[Tuple[int, int, int]]] = None,
                 weight: Optional[torch.Tensor] = None, dtype=torch.float64):
        output_lmax = input_lmax if output_lmax is None else output_lmax
        self.channels, self.layout, self.dtype = int(channels), layout, dtype
        self.input_lmax, self.edge_lmax, self.output_lmax = input_lmax, edge_lmax, output_lmax
        self.lmax = max(input_lmax, edge_lmax, output_lmax)
        full = enumerate_paths(input_lmax, edge_lmax, output_lmax)
        self.paths = full if paths is None else [p for p in full if p in set(map(tuple, paths))]
        self.num_paths = len(self.paths)
        # tp.weight is filled with 1 and frozen by EdgeTensorProduct.create (operators.py:60-62)
        self.weight = (torch.ones(self.num_paths, self.channels, dtype=dtype) if weight is None
                       else weight.to(dtype))
        # groups by (l1,l2), segments in path order (ictd_irreps.py:2194-2212)
        groups: Dict[Tuple[int, int], List[Tuple[int, int]]] = {}
        for p, (l1, l2, l3) in enumerate(self.paths):
            groups.setdefault((l1, l2), []).append((p, l3))
        self.groups = []
        for (l1, l2), items in sorted(groups.items()):
            segs, start = [], 0
            for p, l3 in items:
                segs.append((p, l3, start, start + 2 * l3 + 1))
                start += 2 * l3 + 1
            self.groups.append((l1, l2, segs, start))
        # path_l3 / path_offset / path_counts_by_l (ictd_irreps.py:2514-2526)
        self.path_offset = [0] * self.num_paths
        self.path_counts_by_l = {l: 0 for l in range(self.lmax + 1)}
        for l1, l2, segs, _ in self.groups:
            for p, l3, _, _ in segs:
                self.path_offset[p] = self.path_counts_by_l[l3]
                self.path_counts_by_l[l3] += 1
        scales = basis.path_normalisation_scales(self.paths)
        self.cg = [basis.cg_component_normalised(basis.cg_tensor(*p), p[2]) * scales[i]
                   for i, p in enumerate(self.paths)]
        self.proj = []
        for l1, l2, segs, k_total in self.groups:
            u = torch.zeros((2 * l1 + 1) * (2 * l2 + 1), k_total, dtype=torch.float64)
            for p, l3, s, e in segs:
                u[:, s:e] = self.cg[p].reshape(-1, e - s)
            self.proj.append(u)

    # ------------------------------------------------------------------ sizes
    @property
    def gate_width(self) -> int:
        return self.num_paths * self.channels

    @property
    def output_width(self) -> int:
        return sum(c * self.channels * (2 * l + 1) for l, c in self.path_counts_by_l.items())

    @property
    def input_width(self) -> int:
        return self.channels * (self.input_lmax + 1) ** 2

    # ------------------------------------------------------------------ forward (dict blocks)
    def forward_blocks(self, x1: Dict[int, torch.Tensor], x2: Dict[int, torch.Tensor],
                       gates: Optional[torch.Tensor]) -> Dict[int, torch.Tensor]:
        """``_forward_index_add`` (``ictd_irreps.py:2669-2748``).

        x1[l]: [E,C,2l+1]; x2[l]: [E,1,2l+1]; gates [E,P,C] or [E,P*C]."""
        sample = next(iter(x1.values()))
        rows, dt = sample.shape[0], sample.dtype
        if gates is not None and gates.shape[-1] == self.num_paths * self.channels:
            gates = gates.reshape(rows, self.num_paths, self.channels)
        w = self.weight.to(dt)
        seg_by_l: Dict[int, list] = {l: [] for l in range(self.lmax + 1)}
        idx_by_l: Dict[int, list] = {l: [] for l in range(self.lmax + 1)}
        for g, (l1, l2, segs, _) in enumerate(self.groups):
            a, b = x1.get(l1), x2.get(l2)
            if a is None or b is None:
                continue
            pair = (a.unsqueeze(-1) * b.unsqueeze(-2)).reshape(rows, self.channels, -1)
            y = pair @ self.proj[g].to(dt)  # _project_group (ictd_irreps.py:2264-2268)
            for p, l3, s, e in segs:
                seg = y[..., s:e] * w[p].view(1, self.channels, 1)
                if gates is not None:
                    seg = seg * gates[:, p, :].unsqueeze(-1)
                c0 = self.path_offset[p] * self.channels
                seg_by_l[l3].append(seg)
                idx_by_l[l3].append(torch.arange(c0, c0 + self.channels))
        out = {}
        for l in range(self.lmax + 1):
            base = torch.zeros(rows, self.channels * self.path_counts_by_l[l], 2 * l + 1, dtype=dt)
            if seg_by_l[l]:
                base = base.index_add(-2, torch.cat(idx_by_l[l]), torch.cat(seg_by_l[l], -2))
            out[l] = base
        return out

    # ------------------------------------------------------------------ packed layouts
    def blocks(self, features: torch.Tensor) -> Dict[int, torch.Tensor]:
        """``EdgeTensorProduct._blocks`` (``operators.py:88-99``)."""
        out, off = {}, 0
        for l in range(self.input_lmax + 1):
            width = self.channels * (2 * l + 1)
            v = features[:, off:off + width]
            out[l] = (v.reshape(-1, 2 * l + 1, self.channels).transpose(1, 2) if self.layout == "ir_mul"
                      else v.reshape(-1, self.channels, 2 * l + 1))
            off += width
        return out

    def harmonics(self, harmonics: torch.Tensor) -> Dict[int, torch.Tensor]:
        """``EdgeTensorProduct._harmonics`` (``operators.py:101-105``)."""
        return {l: harmonics[:, l * l:(l + 1) ** 2].unsqueeze(1) for l in range(self.edge_lmax + 1)}

    def pack_output(self, blocks: Dict[int, torch.Tensor]) -> torch.Tensor:
        """``EdgeTensorProduct._pack_output`` (``operators.py:107-115``)."""
        rows, parts = next(iter(blocks.values())).shape[0], []
        for l in range(self.lmax + 1):
            count, width = self.path_counts_by_l.get(l, 0), 2 * l + 1
            v = blocks[l].reshape(rows, count, self.channels, width)
            if self.layout == "ir_mul":
                v = v.transpose(2, 3)
            parts.append(v.reshape(rows, count * self.channels * width))
        return torch.cat(parts, -1)

    def unpack_output(self, output: torch.Tensor) -> Dict[int, torch.Tensor]:
        """``EdgeTensorProduct.unpack_output`` (``operators.py:117-127``)."""
        result, off = {}, 0
        for l in range(self.lmax + 1):
            count, width = self.path_counts_by_l.get(l, 0), 2 * l + 1
            span = count * self.channels * width
            v = output[:, off:off + span]
            if self.layout == "ir_mul":
                v = v.reshape(output.shape[0], count, width, self.channels).transpose(2, 3)
            result[l] = v.reshape(output.shape[0], count * self.channels, width)
            off += span
        return result

    def pack_input(self, blocks: Dict[int, torch.Tensor]) -> torch.Tensor:
        """``EdgeTensorProduct.pack_input`` (``operators.py:77-86``)."""
        parts = []
        for l in range(self.input_lmax + 1):
            v = blocks[l]
            if self.layout == "ir_mul":
                v = v.transpose(1, 2)
            parts.append(v.reshape(v.shape[0], self.channels * (2 * l + 1)))
        return torch.cat(parts, -1)

    def forward(self, features: torch.Tensor, harmonics: torch.Tensor,
                gates: Optional[torch.Tensor]) -> torch.Tensor:
        """``EdgeTensorProduct.forward`` reference branch (``operators.py:136-138``)."""
        return self.pack_output(self.forward_blocks(self.blocks(features), self.harmonics(harmonics), gates))

    # ------------------------------------------------------------------ graph message
    def graph_message_blocks(self, features: Dict[int, torch.Tensor], harmonics: Dict[int, torch.Tensor],
                             gates: torch.Tensor, src: torch.Tensor, dst: torch.Tensor,
                             mask: Optional[torch.Tensor] = None, *, nodes: Optional[int] = None,
                             edge_chunk_size: int = 16384) -> Dict[int, torch.Tensor]:
        """Chunked gather -> TP -> mask -> index_add (``tensor_product.py:189-218``)."""
        sample = next(iter(features.values()))
        nodes = sample.shape[0] if nodes is None else nodes
        output = {l: sample.new_zeros(nodes, self.path_counts_by_l.get(l, 0) * self.channels, 2 * l + 1)
                  for l in range(self.lmax + 1)}
        if src.numel() == 0:
            zero = self.weight.sum() * 0 + gates.sum() * 0
            zero = zero + sum(v.sum() * 0 for v in (*features.values(), *harmonics.values()))
            return {l: v + zero for l, v in output.items()}
        for begin in range(0, src.numel(), edge_chunk_size):
            end = min(begin + edge_chunk_size, src.numel())
            ef = {l: v.index_select(0, src[begin:end]) for l, v in features.items()}
            eh = {l: v[begin:end] for l, v in harmonics.items()}
            value = self.forward_blocks(ef, eh, gates[begin:end])
            for l, block in value.items():
                if mask is not None:
                    block = block * mask[begin:end].reshape(-1, 1, 1)
                output[l] = output[l].index_add(0, dst[begin:end], block)
        return output

    def graph_message(self, features: torch.Tensor, harmonics: torch.Tensor, gates: torch.Tensor,
                      src: torch.Tensor, dst: torch.Tensor, mask: Optional[torch.Tensor] = None,
                      **kw) -> torch.Tensor:
        """``PackedGraphMessage.forward`` (``operators.py:154-163``)."""
        return self.pack_output(self.graph_message_blocks(
            self.blocks(features), self.harmonics(harmonics), gates, src, dst, mask, **kw))
