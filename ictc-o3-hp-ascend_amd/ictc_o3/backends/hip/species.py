"""Species-index validation, cached on the index tensor itself (counterpart of reference
``ictc_o3/backends/ascend/species.py:9-17``).

The result is stored as an attribute of the validated tensor object together with its
version counter, so a different tensor -- even one the caching allocator placed at the same
address -- is always checked again, and so is an in-place change of the validated one.  The
check reads two scalars back to the host, once per index tensor."""
from __future__ import annotations

import torch


def validate_species(index: torch.Tensor, count: int) -> None:
    key = (int(count), index._version)
    if getattr(index, "_ictc_hip_valid_species", None) == key:
        return
    if index.numel():
        lo, hi = torch.stack((index.amin(), index.amax())).cpu().tolist()
        if lo < 0 or hi >= count:
            raise ValueError("Species index is outside the weight bank")
    index._ictc_hip_valid_species = key
