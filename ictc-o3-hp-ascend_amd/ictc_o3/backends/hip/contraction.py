"""The reference's contraction hook (``backends/ascend/contraction.py:8-45``, called from the
module's forward at ``ops/symmetric_contraction.py:189-193``) on the HIP kernels."""
from __future__ import annotations

import torch

from .runtime import require_gpu_fp32


def factorized_contractions(owner, x: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """owner: ICTDBridgeUSymmetricContractionSO3; x [N, C, (L+1)^2] (the MACE feature layout,
    ``_so3_flat_to_mace_features``); index: species [N] -> [N, C * sum_l (2 l + 1)] (per target
    degree a [C, 2l+1] block).  The module's U buffers are projected onto the kernels' coupling
    chains behind the reconstruction gate (ValueError when they do not reconstruct, as in the
    reference); the module weights stay live through the projection."""
    from ictc_o3.ops.symmetric_contraction import _mace_features_to_flat, _species
    from .symmetric_contraction import symmetric_contraction
    require_gpu_fp32(x)
    if x.ndim != 3 or x.shape[1:] != (owner.channels, (owner.lmax + 1) ** 2):
        raise ValueError("features must have shape [N, C, (lmax+1)^2]")
    species = _species(None, index, x.shape[0], owner.num_elements)
    flat = _mace_features_to_flat(x, owner.lmax)
    return symmetric_contraction(owner.plan, flat, species, owner.weight_table(flat))
