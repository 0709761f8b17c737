"""Caller-side runtime of the MACE model (reference ``mace_ictc/hp/runtime.py:84-145``):
``check_model`` / ``configure_model`` argument handling and coverage report, and the batch
index check of ``energy_and_forces``.  CPU only: a CPU model is reported unsupported (the
operators need a ROCm GPU) and nothing launches."""
import pytest
import torch

from mace_hip import MaceICTC, check_model, configure_model
from mace_hip.runtime import _validate_batch


def _cpu_model():
    return MaceICTC(channels=8, lmax=1, num_interactions=1, correlation=2, atomic_numbers=(1, 8))


def test_check_model_reports_instead_of_raising():
    report = check_model(torch.nn.Linear(2, 2))
    assert report == {"supported": False, "backend": "hip",
                      "reasons": ["Expected the MACE-ICTC model (mace_hip.MaceICTC)"]}
    report = check_model(_cpu_model(), training=True, capture=True)
    assert not report["supported"] and report["backend"] == "hip"
    assert "All model parameters must already be ROCm GPU FP32" in report["reasons"]


def test_configure_model_validates_its_arguments():
    model = _cpu_model()
    with pytest.raises(ValueError, match="layout must be packed or fused_pack"):
        configure_model(model, layout="dense")
    with pytest.raises(ValueError, match="policy must be auto, generated or reference"):
        configure_model(model, policy="fast")
    with pytest.raises(ValueError, match="positive integer"):
        configure_model(model, message_chunk_edges=0)
    with pytest.raises(ValueError, match="electrostatics"):
        configure_model(model, electrostatics_backend="mesh_fft")
    with pytest.raises(ValueError, match="no reference"):
        configure_model(model, policy="reference")
    with pytest.raises(ValueError, match="HIP HP unavailable"):
        configure_model(model)                       # CPU parameters: unsupported, no fallback
    assert all(i.edge_chunk_size is None for i in model.interactions)


def test_batch_indices_are_range_checked():
    _validate_batch(torch.tensor([0, 0, 1, 1]), 2)
    with pytest.raises(ValueError, match=r"batch indices must lie in \[0, 2\)"):
        _validate_batch(torch.tensor([0, 2, 1]), 2)
    with pytest.raises(ValueError):
        _validate_batch(torch.tensor([-1, 0]), 2)
    b = torch.tensor([0, 1])
    _validate_batch(b, 2)
    b[1] = 5                                          # in-place change: version bump, checked again
    with pytest.raises(ValueError):
        _validate_batch(b, 2)
