"""Operand guards of the HIP backend (counterpart of reference
``ictc_o3/backends/ascend/runtime.py:94-110``): FP32 only, one GPU device, eager
autograd, no autocast.  Precision is never changed automatically."""
from __future__ import annotations

import torch


def is_gpu(value: torch.Tensor) -> bool:
    return value.device.type == "cuda"


def require_gpu_fp32(*values: torch.Tensor) -> None:
    if not values or any(not is_gpu(v) or v.dtype != torch.float32 for v in values):
        raise ValueError("ictc_o3 HIP operators require FP32 tensors on a ROCm GPU; "
                         "precision is never changed automatically")
    if any(v.device != values[0].device for v in values):
        raise ValueError("All operands must be on the same GPU")
    if torch.is_autocast_enabled("cuda"):
        raise ValueError("ictc_o3 HIP operators require autocast to be disabled")
    if torch.compiler.is_compiling() or torch._C._are_functorch_transforms_active():
        raise ValueError("ictc_o3 HIP operators require ordinary eager autograd")


def strict_fp32() -> None:
    """Disable TF32-style reduced-precision matmuls for the surrounding torch ops
    (counterpart of reference backends/ascend/runtime.py:105-110)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
