"""The TP owner's per-(path, channel) weight is applied on every call, as the reference does
(``backends/ascend/packed_tensor_product.py:163-164``: gates * weight), so no change of the
weight can be missed: in-place updates, ``load_state_dict``, new storage and writes through
``weight.data`` (which bypass the version counter).  The message applies it to the receiver
rows (``output_weight_rows``) instead of the gates; its layout is checked here against the
oracle's gate-weighted message.  CPU only (no kernel runs)."""
import torch

from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
from oracle.tensor_product import TensorProductOracle, enumerate_paths


def _owner(channels=4, lmax=1, paths=None):
    tp = EdgeWeightedPathPreservingTensorProduct(channels, lmax, allowed_paths=paths,
                                                 internal_compute_dtype=torch.float32)
    with torch.no_grad():
        tp.weight.fill_(1.0)
    tp.weight.requires_grad_(False)
    return tp


def _expected(tp, gates):
    return (gates.reshape(3, tp.num_paths, tp.channels) * tp.weight[None]).reshape(3, -1)


def test_every_weight_change_is_seen():
    tp = _owner()
    gates = torch.randn(3, tp.num_paths * tp.channels)
    assert torch.equal(tp.effective_gates(gates, 3), gates)          # unit weight: exact
    with torch.no_grad():
        tp.weight.mul_(2.0)                                           # in-place update
    assert torch.equal(tp.effective_gates(gates, 3), _expected(tp, gates))
    tp.weight.data.mul_(3.0)                                          # invisible to the version counter
    assert torch.equal(tp.effective_gates(gates, 3), _expected(tp, gates))
    tp.weight.data = torch.ones_like(tp.weight) * 0.5                 # new storage
    assert torch.equal(tp.effective_gates(gates, 3), _expected(tp, gates))
    state = {k: v.clone() * 1.5 for k, v in tp.state_dict().items()}
    tp.load_state_dict(state)
    assert torch.equal(tp.effective_gates(gates, 3), _expected(tp, gates))
    rows = tp.output_weight_rows()
    tp.weight.data.fill_(-1.0)
    assert torch.equal(tp.output_weight_rows(), -torch.ones_like(rows))


def test_live_weight_fold_of_an_empty_edge_set():
    tp = _owner()
    tp.weight.requires_grad_(True)
    assert tp.effective_gates(torch.randn(0, tp.num_paths * tp.channels), 0).shape == (0, tp.num_paths * tp.channels)


def test_receiver_row_weight_equals_the_gate_fold():
    """message(gates * weight) == output_weight_rows * message(gates) on the oracle, for a full
    path set and a subset (the rows follow the owner's path_offset order per output degree)."""
    full = enumerate_paths(2, 2, 2)
    for paths in (full, [p for i, p in enumerate(full) if i % 2 == 0]):
        c = 3
        tp = _owner(c, 2, paths)
        gen = torch.Generator().manual_seed(7)
        with torch.no_grad():
            tp.weight.copy_(torch.randn(tp.num_paths, c, generator=gen))
        weighted = TensorProductOracle(c, 2, 2, 2, paths=paths, weight=tp.weight.detach().double())
        plain = TensorProductOracle(c, 2, 2, 2, paths=paths)
        nodes, edges = 5, 12
        x = torch.randn(nodes, plain.input_width, generator=gen, dtype=torch.float64)
        y = torch.randn(edges, 9, generator=gen, dtype=torch.float64)
        g = torch.randn(edges, plain.gate_width, generator=gen, dtype=torch.float64)
        src = torch.randint(0, nodes, (edges,), generator=gen)
        dst = torch.randint(0, nodes, (edges,), generator=gen)
        want = weighted.graph_message(x, y, g, src, dst)
        rows = tp.output_weight_rows().double()
        assert rows.shape == (plain.output_width // c * c,)
        got = plain.graph_message(x, y, g, src, dst) * rows
        assert torch.allclose(got, want, atol=1e-12)


def test_receiver_row_weight_is_differentiable():
    tp = _owner(2, 2)
    tp.weight.requires_grad_(True)
    rows = tp.output_weight_rows()
    (rows * torch.arange(rows.numel(), dtype=rows.dtype)).sum().backward()
    assert tp.weight.grad is not None and tp.weight.grad.abs().sum() > 0
