"""GPU parity of the fused energy readouts (``ictc_hip_readout``: one inner layer's Linear(C, 1)
plus the last layer's Linear(C, H) -> normalised SiLU -> Linear(H, 1)) through the C ABI, against
the composed formula in float64 on the CPU: the value, both input adjoints, a graph recorded through
the adjoint (second derivatives through the composed route), and the MACE model's energies and
forces with the fused readout against its composed layers."""
import pytest
import torch

from conftest import assert_rel

pytestmark = pytest.mark.gpu

SCALE = 1.6791767923989418


def _case(n, c, h, seed, with_y=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, c, generator=g)
    y = torch.randn(n, c, generator=g) if with_y else None
    w_lin = torch.randn(c, generator=g) / c ** 0.5 if with_y else None
    w1 = torch.randn(h, c, generator=g) / c ** 0.5
    w2 = torch.randn(h, generator=g) / h ** 0.5
    return y, x, w_lin, w1, w2


def _dev(ts, gpu):
    return [None if t is None else t.to(gpu) for t in ts]


@pytest.mark.parametrize("n,c,h,with_y", [(2048, 128, 16, True), (37, 70, 5, True), (5, 8, 1, False),
                                          (64, 1024, 256, True)])
def test_value_and_adjoints(gpu, n, c, h, with_y):
    from mace_hip.readout import readout, readout_formula
    y, x, w_lin, w1, w2 = _case(n, c, h, n + c, with_y)
    g = torch.randn(n, generator=torch.Generator().manual_seed(3))
    ref_in = [None if t is None else t.double().requires_grad_(i < 2) for i, t in enumerate((y, x, w_lin, w1, w2))]
    ref = readout_formula(*ref_in, SCALE)
    dy, dx, dwl, dw1, dw2 = _dev((y, x, w_lin, w1, w2), gpu)
    leaves = [t.requires_grad_() for t in (dy, dx) if t is not None]
    got = readout(dy, dx, dwl, dw1, dw2, SCALE)
    assert_rel(got, ref, what="readout value")
    targets = [t for t in ref_in[:2] if t is not None]
    want = torch.autograd.grad(ref, targets, g.double())
    have = torch.autograd.grad(got, leaves, g.to(gpu))
    for a, b in zip(have, want):
        assert_rel(a, b, what="readout adjoint")


def test_second_derivative_through_composed_route(gpu):
    from mace_hip.readout import readout, readout_formula
    y, x, w_lin, w1, w2 = _case(50, 32, 16, 9)
    gen = torch.Generator().manual_seed(10)
    g, hx = torch.randn(50, generator=gen), torch.randn(50, 32, generator=gen)

    def second(fn, ins, dev):
        yy, xx = [t.to(dev).requires_grad_() for t in ins[:2]]
        e = fn(yy, xx, *[t.to(dev) for t in ins[2:]], SCALE)
        (gx,) = torch.autograd.grad(e, xx, g.to(dev).to(e.dtype), create_graph=True)
        return torch.autograd.grad((gx * hx.to(dev).to(gx.dtype)).sum(), [xx, yy], allow_unused=True)

    got = second(readout, [y, x, w_lin, w1, w2], gpu)
    want = second(readout_formula, [t.double() for t in (y, x, w_lin, w1, w2)], "cpu")
    assert_rel(got[0], want[0], what="d2 readout / dx2")
    assert got[1] is None or float(got[1].abs().max()) == 0.0


def test_model_energy_and_forces_match_composed_readouts(gpu):
    import mace_hip.model as M
    from mace_hip import create_model, energy_and_forces, radius_graph, sequential_insertion
    zs, atoms = (1, 6, 8), 96
    model = create_model(channels=32, lmax=2, num_interactions=2, correlation=3, atomic_numbers=zs, cutoff=4.0,
                         avg_num_neighbors=12.0, device=gpu, seed=1)
    model.eval().requires_grad_(False)
    st = sequential_insertion(atoms, 0.05, min_separation=1.2, num_species=len(zs), seed=2)
    src, dst, shifts = radius_graph(st.positions, st.cell, 4.0)
    graph = dict(positions=st.positions.to(gpu), atomic_numbers=torch.tensor(zs)[st.species].to(gpu),
                 batch=torch.zeros(atoms, dtype=torch.int64, device=gpu), edge_src=src.to(gpu),
                 edge_dst=dst.to(gpu), edge_shifts=shifts.to(gpu), cell=st.cell[None].to(gpu))
    fused = energy_and_forces(model, **graph)
    orig = M.readout_supported
    try:
        M.readout_supported = lambda *a: False
        composed = energy_and_forces(model, **graph)
    finally:
        M.readout_supported = orig
    assert_rel(fused["energy"], composed["energy"], what="energy")
    assert_rel(fused["atomic_energy"], composed["atomic_energy"], what="atomic energies")
    assert_rel(fused["forces"], composed["forces"], what="forces")
