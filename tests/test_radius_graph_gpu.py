"""HIP periodic radius graph (mace_hip.neighbors.radius_graph_pbc_gpu) against a brute-force
search over every lattice image in reach, bit-exact in indices and shifts and in order.

The brute force enumerates all (dst, src, s) with |pos[dst] - pos[src] + s @ cell| < r,
s in [-nmax, nmax]^3 on periodic axes (0 on open ones), (src, s) != (dst, 0), in float64 on
the CPU, sorted by (dst, src, s): the semantics of reference
mace_ictc/utils/graph_utils.py:217-297 without its per-image neighbour cap.  Cases: cubic,
skewed triclinic, cells narrower than the cutoff (several images of one pair), an open
axis, empty and single-atom inputs, the cfg-4 structure against the minimum-image
builder the benchmarks also use, rows longer than the sorted fill kernel's key capacity, and
the host-ordered long-row path forced on small cases and checked against the sorted fill.
"""
import itertools
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _brute_force(pos, cell, r, pbc=(True, True, True)):
    pos, cell = pos.double().cpu(), cell.double().cpu()
    vol = abs(float(torch.linalg.det(cell)))
    a0, a1, a2 = cell
    areas = [torch.linalg.cross(a1, a2).norm(), torch.linalg.cross(a2, a0).norm(), torch.linalg.cross(a0, a1).norm()]
    nmax = [math.ceil(r / (vol / float(s))) + 1 if p else 0 for s, p in zip(areas, pbc)]
    rows = []
    for s in itertools.product(*[range(-k, k + 1) for k in nmax]):
        sv = torch.tensor(s, dtype=torch.float64)
        vec = pos[:, None, :] - pos[None, :, :] + sv @ cell          # [dst, src]
        keep = (vec * vec).sum(-1) < r * r
        if not any(s):
            keep.fill_diagonal_(False)
        d, src = keep.nonzero(as_tuple=True)
        for a, b in zip(d.tolist(), src.tolist()):
            rows.append((a, b) + tuple(s))
    rows.sort()
    if not rows:
        return torch.empty(0, dtype=torch.long), torch.empty(0, dtype=torch.long), torch.empty(0, 3)
    t = torch.tensor(rows, dtype=torch.long)
    return t[:, 1], t[:, 0], t[:, 2:].double()


def _check(gpu, pos, cell, r, pbc=None):
    from mace_hip import radius_graph_pbc_gpu
    src, dst, shifts = radius_graph_pbc_gpu(pos.to(gpu), r, cell.to(gpu), pbc=pbc)
    es, ed, esh = _brute_force(pos, cell, r, pbc if pbc is not None else (True, True, True))
    assert src.dtype == torch.long and dst.dtype == torch.long and shifts.dtype == torch.float64
    assert torch.equal(dst.cpu(), ed) and torch.equal(src.cpu(), es) and torch.equal(shifts.cpu(), esh)
    return src, dst, shifts


def _uniform(n, box, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(n, 3, generator=g, dtype=torch.float64) @ box


def test_cubic_and_minimum_image_agree(gpu):
    from mace_hip import radius_graph
    cell = torch.eye(3, dtype=torch.float64) * 17.0
    pos = _uniform(300, cell, 1) + torch.tensor([3.0, -40.0, 9.0], dtype=torch.float64)   # unwrapped input
    src, dst, shifts = _check(gpu, pos, cell, 5.0)
    s2, d2, sh2 = radius_graph(pos, cell, 5.0)
    assert torch.equal(src.cpu(), s2) and torch.equal(dst.cpu(), d2) and torch.equal(shifts.cpu(), sh2)


def test_skewed_triclinic_cell(gpu):
    cell = torch.tensor([[12.0, 0.0, 0.0], [5.0, 11.0, 0.0], [-3.0, 4.0, 13.0]], dtype=torch.float64)
    _check(gpu, _uniform(220, cell, 2), cell, 4.5)


@pytest.mark.parametrize("edge,atoms", [(4.0, 5), (2.5, 3), (7.0, 11)])
def test_cells_narrower_than_the_cutoff(gpu, edge, atoms):
    cell = torch.tensor([[edge, 0.0, 0.0], [0.3, edge, 0.0], [0.0, -0.4, edge * 1.1]], dtype=torch.float64)
    src, dst, shifts = _check(gpu, _uniform(atoms, cell, atoms), cell, 5.0)
    pairs = (dst * atoms + src).cpu()
    assert pairs.unique().numel() < pairs.numel()       # one pair under several images


def test_open_axis(gpu):
    cell = torch.eye(3, dtype=torch.float64) * 14.0
    pos = _uniform(180, cell, 3)
    pos[:, 2] = pos[:, 2] * 2.5 - 6.0                   # spread beyond the cell along the open axis
    src, dst, shifts = _check(gpu, pos, cell, 4.0, pbc=(True, True, False))
    assert bool((shifts[:, 2] == 0).all())


def test_empty_single_atom_and_float32(gpu):
    from mace_hip import radius_graph_pbc_gpu
    cell = torch.eye(3, dtype=torch.float64) * 10.0
    src, dst, shifts, sat = radius_graph_pbc_gpu(torch.empty(0, 3, device=gpu), 3.0, cell.to(gpu),
                                                 return_saturation=True)
    assert src.numel() == dst.numel() == shifts.shape[0] == 0 and sat is False
    small = torch.eye(3, dtype=torch.float64) * 3.0
    src, dst, shifts = _check(gpu, torch.tensor([[0.5, 1.0, 2.9]], dtype=torch.float64), small, 5.0)
    assert bool((src == 0).all()) and bool((dst == 0).all()) and bool((shifts.abs().sum(1) > 0).all())
    pos32 = _uniform(120, cell, 4).float()
    _check(gpu, pos32, cell, 3.5)


def test_sparse_system_in_a_large_cell(gpu):
    """Few atoms in a large cell: the bin grid is coarsened (bounded by the atom count) and the
    result is still exact."""
    cell = torch.tensor([[400.0, 0.0, 0.0], [0.0, 300.0, 0.0], [20.0, 0.0, 350.0]], dtype=torch.float64)
    g = torch.Generator().manual_seed(9)
    centers = torch.rand(6, 3, generator=g, dtype=torch.float64) @ cell
    pos = (centers[:, None, :] + 3.0 * torch.randn(6, 7, 3, generator=g, dtype=torch.float64)).reshape(-1, 3)
    _check(gpu, pos, cell, 5.0)


def test_saturation_flag(gpu):
    from mace_hip import radius_graph_pbc_gpu
    cell = torch.eye(3, dtype=torch.float64) * 8.0
    pos = _uniform(200, cell, 5).to(gpu)
    *_, sat = radius_graph_pbc_gpu(pos, 4.0, cell.to(gpu), max_num_neighbors=10, return_saturation=True)
    assert sat is True
    *_, sat = radius_graph_pbc_gpu(pos, 4.0, cell.to(gpu), max_num_neighbors=10_000, return_saturation=True)
    assert sat is False


def test_cfg4_structure_matches_minimum_image_builder(gpu):
    from mace_hip import radius_graph, radius_graph_pbc_gpu, sequential_insertion
    st = sequential_insertion(2048, 0.1, min_separation=1.5, num_species=10, seed=4)
    pos, cell = st.positions.to(gpu), st.cell.to(gpu)
    src, dst, shifts = radius_graph_pbc_gpu(pos, 5.0, cell)
    s2, d2, sh2 = radius_graph(pos, cell, 5.0)
    assert src.numel() > 100_000
    assert torch.equal(src, s2) and torch.equal(dst, d2) and torch.equal(shifts.to(sh2.dtype), sh2)


def test_rows_beyond_the_sorted_fill_capacity(gpu):
    """A dense cell (~1,200 neighbours per atom, above the sorted fill's 1,024-key rows) takes the
    unsorted fill and host-side ordering; still exact against the brute force."""
    from mace_hip.neighbors import _row_capacity
    cell = torch.eye(3, dtype=torch.float64) * 10.0
    src, dst, shifts = _check(gpu, _uniform(400, cell, 6), cell, 9.0)
    assert int(torch.bincount(dst).max()) > _row_capacity()


@pytest.mark.parametrize("case", ["triclinic", "narrow", "open"])
def test_unsorted_fill_path(gpu, monkeypatch, case):
    """The long-row path forced on small cases (capacity patched to 2 keys), against the brute force."""
    from mace_hip import neighbors
    monkeypatch.setattr(neighbors, "_row_capacity", lambda: 2)
    if case == "triclinic":
        cell = torch.tensor([[12.0, 0.0, 0.0], [5.0, 11.0, 0.0], [-3.0, 4.0, 13.0]], dtype=torch.float64)
        _check(gpu, _uniform(220, cell, 2), cell, 4.5)
    elif case == "narrow":
        cell = torch.tensor([[4.0, 0.0, 0.0], [0.3, 4.0, 0.0], [0.0, -0.4, 4.4]], dtype=torch.float64)
        _check(gpu, _uniform(5, cell, 5), cell, 5.0)
    else:
        cell = torch.eye(3, dtype=torch.float64) * 14.0
        pos = _uniform(180, cell, 3)
        pos[:, 2] = pos[:, 2] * 2.5 - 6.0
        _check(gpu, pos, cell, 4.0, pbc=(True, True, False))


def test_sorted_and_unsorted_fill_agree_on_cfg4(gpu, monkeypatch):
    from mace_hip import neighbors, sequential_insertion
    st = sequential_insertion(2048, 0.1, min_separation=1.5, num_species=10, seed=4)
    pos, cell = st.positions.to(gpu), st.cell.to(gpu)
    sorted_fill = neighbors.radius_graph_pbc_gpu(pos, 5.0, cell)
    monkeypatch.setattr(neighbors, "_row_capacity", lambda: 0)
    host_ordered = neighbors.radius_graph_pbc_gpu(pos, 5.0, cell)
    for a, b in zip(sorted_fill, host_ordered):
        assert a.dtype == b.dtype and torch.equal(a, b)
