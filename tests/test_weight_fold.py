"""The frozen path weight of the TP owner is folded into the gates unless it is all ones
(EdgeWeightedPathPreservingTensorProduct.effective_gates; the reference always multiplies,
backends/ascend/packed_tensor_product.py:163-164).  The all-ones shortcut must notice every
way the weight can change.  CPU only (no kernel runs)."""
import torch

from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct


def _owner():
    tp = EdgeWeightedPathPreservingTensorProduct(4, 1, internal_compute_dtype=torch.float32)
    with torch.no_grad():
        tp.weight.fill_(1.0)
    tp.weight.requires_grad_(False)
    return tp


def _expected(tp, gates):
    return (gates.reshape(3, tp.num_paths, tp.channels) * tp.weight[None]).reshape(3, -1)


def test_unit_weight_skips_the_fold_and_notices_changes():
    tp = _owner()
    gates = torch.randn(3, tp.num_paths * tp.channels)
    assert torch.equal(tp.effective_gates(gates, 3), gates)
    with torch.no_grad():
        tp.weight.mul_(2.0)                                  # in-place: version bump
    assert torch.equal(tp.effective_gates(gates, 3), _expected(tp, gates))
    state = {k: v.clone() for k, v in tp.state_dict().items()}
    tp2 = _owner()
    tp2.effective_gates(gates, 3)                            # caches "all ones"
    tp2.load_state_dict(state)                               # copy_ into the same storage
    assert torch.equal(tp2.effective_gates(gates, 3), _expected(tp2, gates))


def test_write_through_data_after_invalidation():
    tp = _owner()
    gates = torch.randn(3, tp.num_paths * tp.channels)
    tp.effective_gates(gates, 3)
    tp.weight.data.mul_(3.0)                                 # invisible to the version counter
    tp.invalidate_weight_cache()
    assert torch.equal(tp.effective_gates(gates, 3), _expected(tp, gates))
    tp.weight.data = torch.ones_like(tp.weight) * 0.5        # new storage: detected by address
    assert torch.equal(tp.effective_gates(gates, 3), _expected(tp, gates))


def test_live_weight_fold_of_an_empty_edge_set():
    tp = _owner()
    tp.weight.requires_grad_(True)
    assert tp.effective_gates(torch.randn(0, tp.num_paths * tp.channels), 0).shape == (0, tp.num_paths * tp.channels)
