"""The HIP tensor product's output normalisation at the full cfg-1 size (C = 128, lmax 3,
131,072 instances), checked against its definition rather than against the oracle.

With features x ~ N(0, 1) per component, harmonics of directions drawn uniformly on the
sphere and unit gates, the reference's 'component' CG normalisation and 'element' path
normalisation (``ictd_irreps.py:101-142``, applied at ``:2218-2236``) give every output
component of path p the second moment 1 / n(l3), n(l3) = the number of paths into l3 (4, 6,
7, 6 for l3 = 0..3 here), so the paths into each degree sum to 1.  The sample moments below
average 16.8 M (instance, channel) values per component.  A single component's moment
carries the sampling spread of the 131,072 directions (up to 1 % over three seeds in a
float64 simulation); a path's average over its components does not (the sum over the
components of a path's squared response is rotation invariant), leaving only the feature
sampling (~0.05 %).  A wrong path scale moves these moments by a factor of at least 1.17
(1/sqrt(2 l3 + 1) against 1/sqrt(n)) and the other plausible slips (1/n, n^-1/4, none) by
2 or more.
"""
import pytest
import torch

from oracle import ictc_basis as B

pytestmark = pytest.mark.gpu


def test_cfg1_path_second_moments(gpu):
    from ictc_o3 import EdgeTensorProduct
    c, lmax, rows = 128, 3, 131072
    print(f"path moments: C={c} lmax={lmax} rows={rows}", flush=True)
    op = EdgeTensorProduct.create(channels=c, input_lmax=lmax, edge_lmax=lmax, device=gpu)
    paths = [tuple(p) for p in op.paths]
    counts = {}
    for _, _, l3 in paths:
        counts[l3] = counts.get(l3, 0) + 1
    assert [counts[l] for l in range(4)] == [4, 6, 7, 6]
    g = torch.Generator(device=gpu).manual_seed(0)
    x = torch.randn(rows, c * (lmax + 1) ** 2, generator=g, device=gpu)
    gen = torch.Generator().manual_seed(1)
    n = torch.nn.functional.normalize(torch.randn(rows, 3, generator=gen, dtype=torch.float64), dim=-1)
    y = B.direction_harmonics_packed(n, lmax).float().to(gpu)
    gates = torch.ones(rows, op.gate_width, device=gpu)
    with torch.no_grad():
        out = op(x, y, gates)
    torch.cuda.synchronize()
    # ir_mul output: per degree l3, per path with that l3 (owner path_offset order), (2 l3 + 1) rows of C
    off, moment = 0, {}
    for l3 in range(lmax + 1):
        width = counts[l3] * (2 * l3 + 1) * c
        blk = out[:, off:off + width].view(rows, counts[l3], 2 * l3 + 1, c)
        ms = (blk * blk).sum(dim=(0, 3), dtype=torch.float64) / (rows * c)
        moment[l3] = ms.cpu()                        # [paths into l3, 2 l3 + 1]
        off += width
    assert off == op.output_width
    offsets = list(op.tp.path_offset)
    for p, (l1, l2, l3) in enumerate(paths):
        m = moment[l3][offsets[p]]
        want = 1.0 / counts[l3]
        comp = (m / want - 1.0).abs().max().item()
        mean = abs(m.mean().item() / want - 1.0)
        assert comp < 0.03 and mean < 0.005, (
            f"path {(l1, l2, l3)}: component moments {m.tolist()} vs 1/{counts[l3]} "
            f"(worst component {comp:.2%}, mean {mean:.2%})")
    for l3 in range(lmax + 1):
        total = moment[l3].sum(0)
        assert (total - 1.0).abs().max().item() < 0.03, f"l3 = {l3}: paths sum to {total.tolist()}"
        assert abs(total.mean().item() - 1.0) < 0.005
