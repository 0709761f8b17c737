"""Convert the reference's frozen ICTC harmonic-basis assets into plain npz data.

The reference ships 13 basis tensors ``B_l`` (monomial -> harmonic coordinates,
float64, shape ``[(l+2)(l+1)/2, 2l+1]``) as torch-serialised dicts under
``ictc_o3/basis/_ictd_basis/v1/harmonic_basis_l{l}.pt`` and pins each one by
the SHA-256 of its float64 bytes (``ictc_o3/basis/ictd_irreps.py:632-694``).

This script loads each asset with ``torch.load(weights_only=True)`` (data only,
nothing is executed from the file), checks the format fields and the SHA pin,
and writes the tensors as float64 arrays into two npz files:

* ``tests/golden/ictc_basis_v1.npz``   -- read by the CPU oracle;
* ``ictc-o3-hp-ascend_amd/ictc_o3/basis/data/ictc_basis_v1.npz`` -- read by
  the product's plan builder.

Both consumers re-verify the same SHA pins at load time, so a corrupted or
re-generated basis fails loudly.  Run from the repository root:

    python tests/golden/make_basis_fixture.py [/root/reference]
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

# SHA-256 of the float64 bytes of B_l, as pinned by the reference
# (ictc_o3/basis/ictd_irreps.py:633-647).
SHA256 = {
    0: "6c3c396ed6b5c36dcae172271f462051b1266b851e92df3deea8ac65478fd712",
    1: "1332df685c45a61a0ac008a6a653295b8c5655361c1d34b6304b22ec40235fb8",
    2: "0881fbfd2a1866b76334d823d216ec74773a91a5f77234c45bb956838df7c315",
    3: "a7440553d51231cc044287b305d35cb5cafc59f77d7528d8189956c51a52a9e0",
    4: "f89f4b7f49ed9be8cc7fbbcec5e1a8947442c612d239bd42ce36180c6c644225",
    5: "8cce9bfb0a710f2c19d50ca3bcf6a79593697b5bd129085f10422066c2030ea8",
    6: "01cc08fe54c00daaff6899a86c923b62433f1691b7f283b95643c7be78ce9a96",
    7: "bde0ef7cf352a8cc83b4df959405616a390d270cf0b10bd93eed01da80e1a531",
    8: "85cdd2180f8078d9016110556076bf0464d12985ef079f51fee6c8f2641acf28",
    9: "190d6891295881dd5db122b80442a8feea21d0d716c6ff97faddcb0720509c6b",
    10: "fed2be677a84dc357b0e9b27e14b5bbc4c8a110520f44e536e7bc11365d70586",
    11: "4708bb0367de5a1c0d8d6bb01de80cb1a9a84ce6e128bc1913fecceabdf834ec",
    12: "761c7af5c246722d57a910b32ffe82741ac39326d6cba627be7db3b14d4ab689",
}


def main(reference: str) -> None:
    root = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    src = os.path.join(reference, "ictc_o3", "basis", "_ictd_basis", "v1")
    arrays = {}
    for l in range(13):
        blob = torch.load(os.path.join(src, f"harmonic_basis_l{l}.pt"), map_location="cpu",
                          weights_only=True)
        tensor = blob["tensor"].detach().to(torch.float64).contiguous()
        sha = hashlib.sha256(tensor.numpy().tobytes()).hexdigest()
        if (blob.get("format") != "ictd-canonical-harmonic-basis" or blob.get("version") != "v1"
                or int(blob.get("l", -1)) != l or sha != SHA256[l] or blob.get("sha256") != sha
                or tuple(tensor.shape) != ((l + 2) * (l + 1) // 2, 2 * l + 1)):
            raise SystemExit(f"basis asset l={l} failed its integrity check")
        arrays[f"l{l}"] = tensor.numpy()
    for out in (os.path.join(root, "tests", "golden", "ictc_basis_v1.npz"),
                os.path.join(root, "ictc-o3-hp-ascend_amd", "ictc_o3", "basis", "data",
                             "ictc_basis_v1.npz")):
        np.savez(out, **arrays)
        print("wrote", out)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
