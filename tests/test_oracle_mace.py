"""Pin the MACE oracle restatement and the host-side structure/radial code (CPU).

* radius graph: equals a brute-force search over all 27 periodic images, ordered by
  (dst, src), no self pairs, every pair in both directions with opposite vectors;
* radial envelope: 1 at r = 0; value, first and second derivatives vanish at r_max and
  the third equals its closed form; product and oracle embeddings agree;
* oracle model (float64, parameters of a randomly initialised model): energy invariant
  under rotation + translation of the whole periodic structure, forces rotate with it,
  net force zero, and forces equal central finite differences of the energy.
"""
import math

import numpy as np
import pytest
import torch

from oracle.mace import MaceOracle, bessel_features, polynomial_cutoff


def _brute_force(pos, cell, cutoff):
    pairs = {}
    n = pos.shape[0]
    for i in range(n):          # dst
        for j in range(n):      # src
            for sx in (-1, 0, 1):
                for sy in (-1, 0, 1):
                    for sz in (-1, 0, 1):
                        s = np.array([sx, sy, sz], dtype=float)
                        v = pos[i] - pos[j] + s @ cell
                        if (i != j or s.any()) and v @ v < cutoff ** 2:
                            pairs[(i, j)] = pairs.get((i, j), []) + [tuple(s)]
    return pairs


@pytest.mark.parametrize("seed", [0, 1])
def test_radius_graph_matches_brute_force(seed):
    from mace_hip.structures import radius_graph, uniform_box
    st = uniform_box(60, 0.06, num_species=3, seed=seed, dtype=torch.float64)
    cutoff = 3.7
    src, dst, shifts = radius_graph(st.positions, st.cell, cutoff, rows_per_chunk=17)
    pairs = _brute_force(st.positions.numpy(), st.cell.numpy(), cutoff)
    assert all(len(v) == 1 for v in pairs.values())        # minimum image is unique here
    got = {(int(d), int(s)): tuple(sh.tolist()) for s, d, sh in zip(src, dst, shifts)}
    assert got == {k: v[0] for k, v in pairs.items()}
    key = dst * 1000 + src
    assert bool((key[1:] > key[:-1]).all())                 # strictly (dst, src) ordered
    assert bool((src != dst).all())
    vec = st.positions[dst] - st.positions[src] + shifts @ st.cell
    rev = {(int(s), int(d)): i for i, (s, d) in enumerate(zip(src, dst))}
    for i, (s, d) in enumerate(zip(src.tolist(), dst.tolist())):
        assert torch.allclose(vec[rev[(d, s)]], -vec[i])


def test_radius_graph_rejects_small_cells():
    from mace_hip.structures import radius_graph
    with pytest.raises(ValueError):
        radius_graph(torch.zeros(2, 3), torch.eye(3) * 7.0, 4.0)


def test_polynomial_cutoff_smoothness():
    """u(r_max) = u'(r_max) = u''(r_max) = 0 and u'''(r_max) = -p(p+1)(p+2)/r_max^3: the
    polynomial is C^2 at the cutoff, whatever p."""
    p, r_max = 5, 5.0
    r = torch.tensor([r_max], dtype=torch.float64, requires_grad=True)
    x = r / r_max      # the polynomial itself (the step factor is exactly 0 at r_max)
    u = (1.0 - (p + 1.0) * (p + 2.0) / 2.0 * x ** p + p * (p + 2.0) * x ** (p + 1)
         - p * (p + 1.0) / 2.0 * x ** (p + 2))
    inside = polynomial_cutoff(torch.tensor([r_max - 1e-12], dtype=torch.float64), r_max, p)
    assert torch.allclose(inside, u.detach(), atol=1e-9)
    derivs = [u]
    for _ in range(3):
        derivs.append(torch.autograd.grad(derivs[-1].sum(), r, create_graph=True)[0])
    assert all(abs(float(d.detach())) < 1e-12 for d in derivs[:3])
    assert abs(float(derivs[3].detach()) + p * (p + 1) * (p + 2) / r_max ** 3) < 1e-9
    assert float(polynomial_cutoff(torch.zeros(1, dtype=torch.float64), r_max, p)) == 1.0
    from mace_hip.radial import bessel_embedding
    rr = torch.linspace(0.3, 6.0, 40, dtype=torch.float64)
    assert torch.allclose(bessel_embedding(rr, r_max=r_max, num_basis=8, cutoff_p=p),
                          bessel_features(rr, r_max, 8, p), atol=1e-14)
    # closed form of the first basis function inside the cutoff
    expect = math.sqrt(2 / r_max) * math.sin(math.pi * 1.0 / r_max) / 1.0 * float(
        polynomial_cutoff(torch.tensor([1.0], dtype=torch.float64), r_max, p))
    assert abs(float(bessel_features(torch.tensor([1.0], dtype=torch.float64), r_max, 8, p)[0, 0]) - expect) < 1e-15


def _oracle(channels=8, seed=0):
    from mace_hip.model import MaceICTC
    torch.manual_seed(seed)
    model = MaceICTC(channels=channels, lmax=2, num_interactions=2, correlation=3, atomic_numbers=(1, 6, 8),
                     cutoff=3.5, avg_num_neighbors=8.0)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "linear_up" in name or "self_connection" in name:
                p.add_(torch.randn_like(p) * 0.2)
    params = {k: v.detach().double() for k, v in [*model.named_parameters(), *model.named_buffers()]}
    return MaceOracle(params, channels=channels, lmax=2, num_interactions=2, correlation=3, num_elements=3,
                      cutoff=3.5, avg_num_neighbors=8.0)


def _structure(seed=2):
    from mace_hip.structures import radius_graph, sequential_insertion
    st = sequential_insertion(24, 0.05, min_separation=1.0, num_species=3, seed=seed, dtype=torch.float64)
    src, dst, shifts = radius_graph(st.positions, st.cell, 3.5)
    return dict(pos=st.positions, species=st.species, src=src, dst=dst, shifts=shifts, cell=st.cell[None],
                batch=torch.zeros(24, dtype=torch.int64))


def test_oracle_symmetries_and_finite_differences():
    oracle, g = _oracle(), _structure()
    e, f, _ = oracle.energy_and_forces(**g)
    om = torch.tensor([0.4, -0.8, 1.1], dtype=torch.float64)
    k = torch.zeros(3, 3, dtype=torch.float64)
    k[0, 1], k[0, 2], k[1, 2] = -om[2], om[1], -om[0]
    rot = torch.linalg.matrix_exp(k - k.T)
    g2 = dict(g, pos=g["pos"] @ rot.T + torch.tensor([0.3, 1.2, -0.7], dtype=torch.float64),
              cell=g["cell"] @ rot.T)
    e2, f2, _ = oracle.energy_and_forces(**g2)
    assert abs(float((e2 - e).detach())) < 1e-10 * max(1.0, abs(float(e)))
    assert (f2 - f @ rot.T).abs().max() < 1e-9 * max(1.0, float(f.abs().max()))
    assert f.sum(0).abs().max() < 1e-10 * max(1.0, float(f.abs().max()))
    assert float(f.abs().max()) > 1e-6
    h = 1e-5
    for atom, axis in ((0, 0), (5, 2), (17, 1)):
        pp, pm = g["pos"].clone(), g["pos"].clone()
        pp[atom, axis] += h
        pm[atom, axis] -= h
        ep = oracle.energy_and_forces(**dict(g, pos=pp))[0]
        em = oracle.energy_and_forces(**dict(g, pos=pm))[0]
        fd = -(ep - em) / (2 * h)
        assert abs(float(fd) - float(f[atom, axis])) < 1e-6 * max(1.0, float(f.abs().max()))
