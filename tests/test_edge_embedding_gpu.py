"""GPU parity of the fused edge embedding (directions and Bessel x cutoff radial embedding,
``ictc_hip_edge_embedding``) against float64 autograd of the oracle's restatement
(``oracle/mace.py`` ``bessel_features``; directions v / max(|v|, 1e-8) as reference
``pure_cartesian_ictd_fix.py:2935-2936``): every kernel mode (value, VJP with either cotangent
absent, JVP, HVP), the force-training chain through the autograd Functions (forces with
create_graph, then the gradient of a force loss), edges past the cutoff, and bit-identical
repeat runs."""
import pytest
import torch

from conftest import RTOL, assert_rel
from oracle.mace import bessel_features

pytestmark = pytest.mark.gpu

R_MAX, B, P = 5.0, 8, 5


def _vectors(rows, seed):
    g = torch.Generator().manual_seed(seed)
    d = torch.nn.functional.normalize(torch.randn(rows, 3, generator=g, dtype=torch.float64), dim=-1)
    r = 0.4 + 5.2 * torch.rand(rows, generator=g, dtype=torch.float64)      # ~10 % past r_max
    return (d * r[:, None]).float()


def _ref(v):
    r = v.norm(dim=1)
    return v / r.clamp(min=1e-8)[:, None], bessel_features(r, R_MAX, B, P)


def _raw(mode, v, gn=None, ge=None, t=None, want_n=True, want_e=True):
    from mace_hip.embedding import EmbeddingSpec, _raw as raw
    return raw(mode, v, EmbeddingSpec(R_MAX, B, P), gn=gn, ge=ge, t=t, want_n=want_n, want_e=want_e)


def test_modes_match_float64_autograd(gpu):
    from mace_hip.embedding import HVP, JVP, VALUE, VJP
    rows = 4099
    v = _vectors(rows, 1)
    g0 = torch.Generator().manual_seed(2)
    gn, ge, t = (torch.randn(rows, w, generator=g0) for w in (3, B, 3))
    vd = v.double().requires_grad_()
    n_ref, e_ref = _ref(vd)
    n, e = _raw(VALUE, v.to(gpu))
    assert_rel(n, n_ref, what="directions")
    assert_rel(e, e_ref, what="embedding")
    assert float(e_ref.detach()[v.double().norm(dim=1) >= R_MAX].abs().max()) == 0.0
    assert float(e.cpu()[v.double().norm(dim=1) >= R_MAX].abs().max()) == 0.0
    # VJP, with both cotangents and with either one absent
    for a, b in ((gn, ge), (gn, None), (None, ge)):
        total = sum((x.double() * y).sum() for x, y in ((a, n_ref), (b, e_ref)) if x is not None)
        want, = torch.autograd.grad(total, vd, retain_graph=True)
        got = _raw(VJP, v.to(gpu), gn=None if a is None else a.to(gpu), ge=None if b is None else b.to(gpu),
                   want_e=False)[0]
        assert_rel(got, want, what=f"VJP (gn {a is not None}, ge {b is not None})")
    # JVP via forward-mode autograd
    _, (jn, je) = torch.func.jvp(_ref, (v.double(),), (t.double(),))
    got_n, got_e = _raw(JVP, v.to(gpu), t=t.to(gpu))
    assert_rel(got_n, jn, what="JVP directions")
    assert_rel(got_e, je, what="JVP embedding")
    # HVP: d/dv <(gn, ge), df[t]>
    gv, = torch.autograd.grad((gn.double() * n_ref).sum() + (ge.double() * e_ref).sum(), vd, create_graph=True)
    want, = torch.autograd.grad((gv * t.double()).sum(), vd)
    got = _raw(HVP, v.to(gpu), gn=gn.to(gpu), ge=ge.to(gpu), t=t.to(gpu), want_e=False)[0]
    assert_rel(got, want, what="HVP")


def test_force_training_chain(gpu):
    """E = sum w_n . n + sum w_e . emb^2; forces = -dE/dv (create_graph); the gradient of
    sum forces^2 with respect to v and to the weights, through the autograd Functions."""
    from mace_hip.embedding import edge_embedding
    rows = 1031
    v = _vectors(rows, 3)
    g0 = torch.Generator().manual_seed(4)
    wn, we = torch.randn(rows, 3, generator=g0), torch.randn(rows, B, generator=g0)

    def chain(f, vv, a, b):
        vv, a, b = (x.clone().requires_grad_() for x in (vv, a, b))
        n, e = f(vv)
        energy = (a * n).sum() + (b * e * e).sum()
        forces, = torch.autograd.grad(-energy, vv, create_graph=True)
        loss = (forces * forces).sum()
        return (forces,) + torch.autograd.grad(loss, (vv, a, b))

    got = chain(lambda x: edge_embedding(x, r_max=R_MAX, num_basis=B, cutoff_p=P), v.to(gpu), wn.to(gpu), we.to(gpu))
    want = chain(_ref, v.double(), wn.double(), we.double())
    for name, a, b in zip(("forces", "d loss/dv", "d loss/dw_n", "d loss/dw_e"), got, want):
        assert_rel(a, b, rtol=10 * RTOL, what=name)


def test_repeat_runs_bit_identical(gpu):
    from mace_hip.embedding import VALUE, VJP
    v = _vectors(20000, 5).to(gpu)
    ge = torch.randn(20000, B, device=gpu)
    a = _raw(VALUE, v)
    b = _raw(VALUE, v)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    assert torch.equal(_raw(VJP, v, ge=ge, want_e=False)[0], _raw(VJP, v, ge=ge, want_e=False)[0])


def test_rejects_bad_arguments(gpu):
    from ictc_o3 import _lib
    from mace_hip.embedding import edge_embedding
    with pytest.raises(ValueError):
        edge_embedding(torch.zeros(4, 3, device=gpu, dtype=torch.float64), r_max=R_MAX)
    lib = _lib.lib()
    x = torch.zeros(4, 3, device=gpu)
    for basis, p, rmax in ((0, 5, 5.0), (65, 5, 5.0), (8, 0, 5.0), (8, 17, 5.0), (8, 5, 0.0)):
        assert lib.ictc_hip_edge_embedding(0, x.data_ptr(), None, None, None, x.data_ptr(), x.data_ptr(), basis,
                                           p, rmax, 4, None) == 1
    assert lib.ictc_hip_edge_embedding(7, x.data_ptr(), None, None, None, x.data_ptr(), x.data_ptr(), 8, 5, 5.0,
                                       4, None) == 1
