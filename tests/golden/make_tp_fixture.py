"""Write ``tp_reference_vectors.npz``: float64 input/output vectors of the reference's own
CPU tensor product, for the conventions that no closed form fixes (path order,
``path_offset``, packed output layout), together with its CG tensors, harmonics, forward,
VJP and mixed second derivatives.

Run once, in the build container only, where the reference tree exists:

    python tests/golden/make_tp_fixture.py /root/reference

It imports the torch-only owner ``EdgeWeightedPathPreservingTensorProduct``
(``ictc_o3/basis/ictd_irreps.py:2501-2794``, CPU forward ``_forward_index_add`` :2669-2748
or the scalar-l1 branch :2575-2667), ``direction_harmonics_all`` (:1113-1168) and the packing
rule of ``EdgeTensorProduct._pack_output`` (``ictc_o3/operators.py:107-115``; the class itself
refuses non-NPU devices, so its method is applied to a stand-in holding ``tp`` and
``layout``).  The on-disk CG cache is switched off (``FSCETP_ICTD_CACHE=0``), so nothing is
written into the reference tree.  Only the resulting numbers are committed; the GPU box never
sees the reference.
"""
from __future__ import annotations

import os
import sys
import types

import numpy as np

CASES = [  # (name, channels, input_lmax, edge_lmax, output_lmax, keep every k-th path or None)
    ("l222", 3, 2, 2, 2, None),
    ("l333", 3, 3, 3, 3, None),
    ("l033", 3, 0, 3, 3, None),   # scalar-l1 paths (MACE layer 0)
    ("l123", 2, 1, 2, 3, None),
    ("l333_subset", 3, 3, 3, 3, 2),
]
ROWS = 5


def main(reference: str, out_path: str) -> None:
    os.environ["FSCETP_ICTD_CACHE"] = "0"
    sys.path.insert(0, reference)
    import torch
    from ictc_o3.basis.ictd_irreps import (EdgeWeightedPathPreservingTensorProduct,
                                           direction_harmonics_all)
    from ictc_o3.operators import EdgeTensorProduct

    torch.manual_seed(0)
    data = {}
    for name, c, lin, le, lout, keep in CASES:
        gen = torch.Generator().manual_seed(sum(map(ord, name)))
        paths = [(i, j, k) for i in range(lin + 1) for j in range(le + 1) for k in range(lout + 1)
                 if abs(i - j) <= k <= i + j and (i + j + k) % 2 == 0]
        if keep is not None:
            ordered = EdgeWeightedPathPreservingTensorProduct(
                channels=c, lmax=max(lin, le, lout), allowed_paths=paths,
                internal_compute_dtype=torch.float64).paths
            paths = [p for n, p in enumerate(ordered) if n % keep == 0]
        tp = EdgeWeightedPathPreservingTensorProduct(
            channels=c, lmax=max(lin, le, lout), allowed_paths=paths,
            internal_compute_dtype=torch.float64).double()
        with torch.no_grad():
            tp.weight.fill_(1.0)
        tp.weight.requires_grad_(False)
        n = torch.nn.functional.normalize(torch.randn(ROWS, 3, generator=gen, dtype=torch.float64), dim=-1)
        ys = direction_harmonics_all(n, le)
        y = torch.cat(ys, -1)
        x = torch.randn(ROWS, c * (lin + 1) ** 2, generator=gen, dtype=torch.float64)
        gates = torch.randn(ROWS, tp.num_paths * c, generator=gen, dtype=torch.float64)
        width = sum(cnt * c * (2 * l + 1) for l, cnt in tp.path_counts_by_l.items())
        cot = torch.randn(ROWS, width, generator=gen, dtype=torch.float64)
        hx, hy, hg = (torch.randn(ROWS, t.shape[1], generator=gen, dtype=torch.float64) for t in (x, y, gates))

        pre = f"{name}/"
        data[pre + "meta"] = np.array([c, lin, le, lout], dtype=np.int64)
        data[pre + "paths"] = np.array(tp.paths, dtype=np.int64).reshape(-1, 3)
        data[pre + "path_offset"] = np.array(tp.path_offset, dtype=np.int64)
        data[pre + "path_counts"] = np.array([tp.path_counts_by_l.get(l, 0) for l in range(tp.lmax + 1)],
                                             dtype=np.int64)
        for p, cg in enumerate(tp._get_cg_list(torch.device("cpu"), torch.float64)):
            data[pre + f"cg{p}"] = cg.numpy()
        data[pre + "directions"] = n.numpy()
        data[pre + "harmonics"] = y.numpy()
        data[pre + "x"], data[pre + "gates"], data[pre + "cotangent"] = x.numpy(), gates.numpy(), cot.numpy()
        data[pre + "hx"], data[pre + "hy"], data[pre + "hg"] = hx.numpy(), hy.numpy(), hg.numpy()
        for layout in ("ir_mul", "mul_ir"):
            packer = types.SimpleNamespace(tp=tp, layout=layout, input_lmax=lin, edge_lmax=le)
            leaves = [t.clone().requires_grad_() for t in (x, y, gates)]
            blocks = _blocks(packer, leaves[0])
            harm = {l: leaves[1][:, l * l:(l + 1) ** 2].unsqueeze(1) for l in range(le + 1)}
            out = EdgeTensorProduct._pack_output(packer, tp(blocks, harm, leaves[2]))
            grads = torch.autograd.grad(out, leaves, cot, create_graph=True)
            second = torch.autograd.grad(sum((g * h).sum() for g, h in zip(grads, (hx, hy, hg))),
                                         leaves, allow_unused=True)
            data[pre + f"{layout}/out"] = out.detach().numpy()
            for tag, g in zip(("dx", "dy", "dg"), grads):
                data[pre + f"{layout}/{tag}"] = g.detach().numpy()
            for tag, g, like in zip(("ddx", "ddy", "ddg"), second, (x, y, gates)):
                data[pre + f"{layout}/{tag}"] = (torch.zeros_like(like) if g is None else g).numpy()
    np.savez_compressed(out_path, **data)
    print(f"wrote {out_path}: {len(data)} arrays")


def _blocks(packer, features):
    """Packed features -> per-degree [E, C, 2l+1] blocks by the rule of
    ``EdgeTensorProduct._blocks`` (``operators.py:88-99``), whose device check refuses CPU."""
    result, offset = {}, 0
    c = packer.tp.channels
    for l in range(packer.input_lmax + 1):
        width = c * (2 * l + 1)
        value = features[:, offset:offset + width]
        result[l] = (value.reshape(features.shape[0], 2 * l + 1, c).transpose(1, 2)
                     if packer.layout == "ir_mul" else value.reshape(features.shape[0], c, 2 * l + 1))
        offset += width
    return result


if __name__ == "__main__":
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    main(ref, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tp_reference_vectors.npz"))
