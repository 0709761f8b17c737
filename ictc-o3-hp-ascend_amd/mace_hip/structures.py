"""Synthetic periodic structures and their radius graphs (benchmark and test inputs).

* ``uniform_box``: atoms uniform in a cubic box of the given number density;
* ``sequential_insertion``: random sequential insertion with a minimum (minimum-image)
  separation, rejecting overlapping trial positions;
* ``radius_graph``: all directed pairs (src != dst) closer than the cutoff under the
  minimum-image convention, ordered by (dst, src).  Edge vectors follow the
  reference convention (``pure_cartesian_ictd_fix.py:2930-2933``):
      vec_e = pos[dst] - pos[src] + shift_e @ cell,   shift_e integer lattice coords.
  The minimum image is unique when every perpendicular cell width exceeds 2 cutoff,
  which is checked; it replaces the torch_cluster-based builder
  (``mace_ictc/utils/graph_utils.py:217-297``) for such cells.
Positions are generated on the host from a seeded numpy generator (bit-reproducible),
the graph is built on the device of ``positions``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class Structure:
    positions: torch.Tensor       # [N, 3]
    cell: torch.Tensor            # [3, 3] rows are lattice vectors
    species: torch.Tensor         # [N] int64 compact species index


def box_edge(n: int, density: float) -> float:
    return float((n / density) ** (1.0 / 3.0))


def uniform_box(n: int, density: float, *, num_species: int = 10, seed: int = 4,
                dtype=torch.float32) -> Structure:
    rng = np.random.default_rng(seed)
    edge = box_edge(n, density)
    pos = rng.random((n, 3)) * edge
    species = np.random.default_rng(seed + 1).integers(0, num_species, n)
    return Structure(torch.tensor(pos, dtype=dtype), torch.eye(3, dtype=dtype) * edge,
                     torch.tensor(species, dtype=torch.int64))


def sequential_insertion(n: int, density: float, *, min_separation: float = 1.5, num_species: int = 10,
                         seed: int = 4, max_trials: int = 1000000, dtype=torch.float32) -> Structure:
    rng = np.random.default_rng(seed)
    edge = box_edge(n, density)
    pos = np.empty((n, 3))
    count, trials = 0, 0
    while count < n:
        trials += 1
        if trials > max_trials:
            raise RuntimeError("random sequential insertion did not converge; lower the density or separation")
        p = rng.random(3) * edge
        if count:
            d = pos[:count] - p
            d -= edge * np.round(d / edge)
            if np.min(np.einsum("ij,ij->i", d, d)) < min_separation ** 2:
                continue
        pos[count] = p
        count += 1
    species = np.random.default_rng(seed + 1).integers(0, num_species, n)
    return Structure(torch.tensor(pos, dtype=dtype), torch.eye(3, dtype=dtype) * edge,
                     torch.tensor(species, dtype=torch.int64))


@torch.no_grad()
def radius_graph(positions: torch.Tensor, cell: torch.Tensor, cutoff: float, *, rows_per_chunk: int = 1024):
    """-> (src, dst, shifts [E,3] float lattice coords), ordered by (dst, src)."""
    cell64 = cell.double()
    widths = 1.0 / torch.linalg.norm(torch.linalg.inv(cell64), dim=0)   # perpendicular widths
    if bool((widths <= 2.0 * cutoff).any()):
        raise ValueError("radius_graph needs every perpendicular cell width > 2 * cutoff (minimum image)")
    pos = positions.double()
    inv = torch.linalg.inv(cell64)
    n = pos.shape[0]
    srcs, dsts, shifts = [], [], []
    for begin in range(0, n, rows_per_chunk):
        end = min(begin + rows_per_chunk, n)
        raw = pos[begin:end, None, :] - pos[None, :, :]              # pos[dst] - pos[src]
        frac = raw @ inv
        shift = -torch.round(frac)
        vec = raw + shift @ cell64
        dist2 = (vec * vec).sum(-1)
        keep = dist2 < cutoff * cutoff
        keep[torch.arange(end - begin), torch.arange(begin, end)] = False
        d, s = keep.nonzero(as_tuple=True)                           # row-major: (dst, src) order
        srcs.append(s)
        dsts.append(d + begin)
        shifts.append(shift[d, s])
    src = torch.cat(srcs).to(torch.int64)
    dst = torch.cat(dsts).to(torch.int64)
    return src, dst, torch.cat(shifts).to(positions.dtype)
