"""Dense layers of the model: ``mm`` / ``linear`` of ``ictc_o3.backends.hip.linear`` (rocBLAS
called explicitly for plain products, split-K batched products for the weight gradients that
reduce over edge rows; differentiable to any order) and a bias-free ``nn.Linear`` on top."""
from __future__ import annotations

import torch.nn as nn

from ictc_o3.backends.hip.linear import (SPLIT_ROWS, SPLIT_ROWS_LARGE, _product, linear,  # noqa: F401
                                         mm)


class Linear(nn.Linear):
    """Bias-free nn.Linear (same parameter name and shape) computed through ``linear``; inputs
    of any leading shape."""

    def __init__(self, fan_in: int, fan_out: int):
        super().__init__(fan_in, fan_out, bias=False)

    def forward(self, x):
        lead = x.shape[:-1]
        return linear(x.reshape(-1, x.shape[-1]), self.weight).reshape(*lead, self.out_features)
