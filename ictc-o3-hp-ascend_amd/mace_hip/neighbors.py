"""Periodic radius graph on the GPU (HIP cell list), ordered for the message kernels.

Mirrors reference ``mace_ictc/utils/graph_utils.py``: ``pbc_image_nmax`` (:192-214, image
bound from the cell's face heights) and ``radius_graph_pbc_gpu`` (:217-297, same
arguments and returns: ``(edge_src, edge_dst, edge_shifts float64)`` with
``vec = pos[dst] - pos[src] + shift @ cell``, self pairs excluded, optional saturation flag).
The reference runs one torch_cluster radius query per lattice image, each capped at
``max_num_neighbors``; here one exact search over binned atoms runs on HIP
(``ictc_hip_radius_graph_count`` / ``_fill_sorted``), nothing is truncated, and the edges come
out ordered by (dst, src, shift): the receiver order the message kernels use, with ties
resolved deterministically.  ``saturated`` reports whether any receiver has at least
``max_num_neighbors`` neighbours (where the reference's per-image queries could truncate).

Host steps (device tensors): fractional coordinates, wrap along periodic axes, bins at
least one cutoff wide along every face normal (fewer bins and a wider reach when the cell
is narrower than the cutoff, so every image is enumerated exactly once), atoms grouped by
bin, count pass (one wave per receiver), exclusive scan, one device-to-host read of the edge
count and the longest row, then the sorted fill: one wave per receiver writes its row already
ordered by (src, shift), with dst and the float64 shifts.  A row longer than the kernel's LDS
key capacity (1,024 edges) takes the unsorted fill and two stable sorts here instead.
"""
from __future__ import annotations

import ctypes
import math

import torch

from ictc_o3 import _lib
from ictc_o3.backends.hip.runtime import is_gpu

MAX_BINS_PER_AXIS = 256


def _pbc_flags(pbc):
    if pbc is None:
        return [True, True, True]
    flags = [bool(v) for v in (torch.as_tensor(pbc).reshape(-1).tolist())]
    if len(flags) == 1:
        flags = flags * 3
    if len(flags) != 3:
        raise ValueError(f"pbc must have length 3, got {len(flags)}")
    return flags


def _face_heights(cell64_cpu: torch.Tensor) -> list:
    a0, a1, a2 = cell64_cpu
    volume = abs(float(torch.linalg.det(cell64_cpu)))
    areas = [float(torch.linalg.cross(a1, a2).norm()), float(torch.linalg.cross(a2, a0).norm()),
             float(torch.linalg.cross(a0, a1).norm())]
    if volume <= 1e-12 or min(areas) <= 1e-12:
        raise ValueError("cell is singular")
    return [volume / s for s in areas]


def pbc_image_nmax(cell: torch.Tensor, cutoff: float, pbc=None) -> torch.Tensor:
    """ceil(cutoff / h_i) per periodic axis (h_i = volume / face area), 0 on open axes."""
    cell_mat = cell.squeeze(0) if cell.dim() == 3 else cell
    heights = _face_heights(cell_mat.detach().double().cpu())
    flags = _pbc_flags(pbc)
    return torch.tensor([max(1, math.ceil(float(cutoff) / h)) if f else 0 for h, f in zip(heights, flags)],
                        dtype=torch.long, device=cell_mat.device)


def _row_capacity() -> int:
    """Longest receiver row the sorted fill kernel orders in LDS."""
    return int(_lib.lib().ictc_hip_radius_graph_row_capacity())


@torch.no_grad()
def radius_graph_pbc_gpu(pos: torch.Tensor, r: float, cell: torch.Tensor, max_num_neighbors: int = 100, pbc=None,
                         return_saturation: bool = False):
    """-> (edge_src, edge_dst, edge_shifts [E,3] float64[, saturated]), ordered by (dst, src, shift)."""
    if not is_gpu(pos) or pos.ndim != 2 or pos.shape[1] != 3 or pos.dtype not in (torch.float32, torch.float64):
        raise ValueError("positions must be a float32/float64 [N,3] tensor on a ROCm GPU")
    r = float(r)
    if not r > 0.0:
        raise ValueError("cutoff must be positive")
    dev = pos.device
    cell_mat = cell.squeeze(0) if cell.dim() == 3 else cell
    if cell_mat.shape != (3, 3):
        raise ValueError("cell must be [3,3] or [1,3,3]")
    flags = _pbc_flags(pbc)
    n = pos.shape[0]
    empty = (torch.empty(0, dtype=torch.long, device=dev), torch.empty(0, dtype=torch.long, device=dev),
             torch.empty(0, 3, dtype=torch.float64, device=dev))
    if n == 0:
        return empty + (False,) if return_saturation else empty
    cell_cpu = cell_mat.detach().double().cpu()
    heights = _face_heights(cell_cpu)
    c64 = cell_cpu.to(dev)
    frac = pos.double() @ torch.linalg.inv(cell_cpu).to(dev)
    if all(flags):
        # every axis wraps into [0, 1): the binned region is the cell itself, known on the host
        n0 = torch.floor(frac)
        fw = frac - n0
        lo, span, span_host = None, None, [1.0, 1.0, 1.0]
    else:
        periodic = torch.tensor(flags, device=dev)
        n0 = torch.where(periodic, torch.floor(frac), torch.zeros_like(frac))
        fw = frac - n0
        lo = torch.where(periodic, torch.zeros(3, dtype=torch.float64, device=dev), fw.min(0).values)
        span = torch.where(periodic, torch.ones(3, dtype=torch.float64, device=dev),
                           (fw.max(0).values - lo).clamp_min(1e-12))
        span_host = span.cpu().tolist()
    extents = [span_host[a] * heights[a] for a in range(3)]   # perpendicular extent of the binned region
    bins = [int(min(MAX_BINS_PER_AXIS, max(1, math.floor(e / r)))) for e in extents]
    while bins[0] * bins[1] * bins[2] > max(64, 8 * n):          # sparse systems: coarser bins
        a = max(range(3), key=lambda i: bins[i])
        bins[a] = max(1, bins[a] // 2)
    reach = []
    for a in range(3):
        k = max(1, math.ceil(r / (extents[a] / bins[a])))         # bins of width extent / bins
        reach.append(min(k, bins[a] - 1) if not flags[a] else k)
    bins_t = torch.tensor(bins, dtype=torch.float64, device=dev)
    abin = torch.floor((fw if lo is None else (fw - lo) / span) * bins_t).clamp(min=0)
    abin = torch.minimum(abin, bins_t - 1).to(torch.int32).contiguous()
    wpos = (fw @ c64).contiguous()
    ab = abin.to(torch.int64)
    bin_id = (ab[:, 0] * bins[1] + ab[:, 1]) * bins[2] + ab[:, 2]
    nbins = bins[0] * bins[1] * bins[2]
    bin_atoms = torch.sort(bin_id, stable=True).indices.contiguous()
    bin_start = torch.zeros(nbins + 1, dtype=torch.int64, device=dev)
    torch.cumsum(torch.bincount(bin_id, minlength=nbins), 0, out=bin_start[1:])

    grid = _lib.CellGrid()
    for i, v in enumerate(cell_cpu.reshape(-1).tolist()):
        grid.cell[i] = v
    grid.cutoff_sq = r * r
    for a in range(3):
        grid.bins[a], grid.reach[a], grid.periodic[a] = bins[a], reach[a], int(flags[a])
    lib, stream = _lib.lib(), _lib.stream_of(dev)
    args = (ctypes.byref(grid), wpos.data_ptr(), abin.data_ptr(), bin_start.data_ptr(), bin_atoms.data_ptr(), n)
    counts = torch.empty(n, dtype=torch.int64, device=dev)
    _lib.check(lib.ictc_hip_radius_graph_count(*args, counts.data_ptr(), stream), "ictc_hip_radius_graph_count")
    rowptr = torch.zeros(n + 1, dtype=torch.int64, device=dev)
    torch.cumsum(counts, 0, out=rowptr[1:])
    edges, longest = torch.stack((rowptr[-1], counts.max())).tolist()   # one device-to-host read
    saturated = max_num_neighbors > 0 and longest >= int(max_num_neighbors)
    if edges == 0:
        return empty + (saturated,) if return_saturation else empty
    n0i = n0.to(torch.int64).contiguous()
    if longest <= _row_capacity():
        # rows written in (dst, src, shift) order by the kernel itself
        src = torch.empty(edges, dtype=torch.int64, device=dev)
        dst = torch.empty(edges, dtype=torch.int64, device=dev)
        shift = torch.empty(edges, 3, dtype=torch.float64, device=dev)
        _lib.check(lib.ictc_hip_radius_graph_fill_sorted(*args, rowptr.data_ptr(), n0i.data_ptr(), src.data_ptr(),
                                                         dst.data_ptr(), shift.data_ptr(), stream),
                   "ictc_hip_radius_graph_fill_sorted")
        result = (src, dst, shift)
        return result + (saturated,) if return_saturation else result
    # a row beyond the kernel's key capacity: fill in visiting order, then order the rows here
    src = torch.empty(edges, dtype=torch.int64, device=dev)
    images = torch.empty(edges, 3, dtype=torch.int32, device=dev)
    _lib.check(lib.ictc_hip_radius_graph_fill(*args, rowptr.data_ptr(), src.data_ptr(), images.data_ptr(), stream),
               "ictc_hip_radius_graph_fill")
    dst = torch.repeat_interleave(torch.arange(n, device=dev), counts)
    shift = images.to(torch.int64) - n0i[dst] + n0i[src]
    # rows are grouped by dst; order each row by (src, shift): stable sort by that key, then by dst
    smax = int(shift.abs().max())
    w = 2 * smax + 1
    code = ((shift[:, 0] + smax) * w + (shift[:, 1] + smax)) * w + (shift[:, 2] + smax)
    if n * w ** 3 >= 2 ** 62:
        raise ValueError("too many atoms or lattice images to order the edges")
    order = torch.sort(src * (w ** 3) + code, stable=True).indices
    order = order[torch.sort(dst[order], stable=True).indices]
    result = (src[order], dst[order], shift[order].to(torch.float64))
    return result + (saturated,) if return_saturation else result
