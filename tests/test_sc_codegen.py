"""The generated symmetric-contraction code, evaluated on the CPU (no GPU, no compiler).

csrc/gen_sc.py emits straight-line C++ (one Plan<L, T, K> per configuration) that the HIP
kernels instantiate.  Here that exact text is translated statement by statement into
numpy (float64, vectorised over channels) and run:

* forward(x, w)        == sum_p W_p U_p[x, x, x]           (dense U per (l_out, order); both the
                                                            straight-line float branch and the step loop)
* vjp(x, w, u)         == d/dx <u, forward(x)>             (autograd through the dense form)
* weight_features(x,u) == <u, U_p[x, x, x]> per column p

The dense U is the chain-assembled U of ictc_o3/basis/symmetric_u.py, which
tests/test_oracle_sc.py pins (to 1e-12, every lmax <= 3, l_out and order) to the oracle's
restatement of the reference's coupled basis (ictc_o3/basis/ictd_irreps.py:1387-1517).  A wrong coupling entry, a chain routed to the wrong accumulator
slot, a missed batch reset or a dropped sign in the emitted schedule fails here before any
GPU run.
"""
import os
import re
import sys

import numpy as np
import pytest
import torch

from ictc_o3.basis import symmetric_u as S

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "ictc-o3-hp-ascend_amd", "csrc")
if CSRC not in sys.path:
    sys.path.insert(0, CSRC)
import gen_sc  # noqa: E402

# the emitted CG constants are float32-rounded; a wrong entry, slot or sign errs by O(1)
TOL = 1e-6
_SKIP = ("//", "#pragma", "asm ", "switch", "case ", "default:", "for (int step", "int Cs = C;")


def _translate(lines):
    """Emitted C++ statements -> Python statements over lists of numpy arrays."""
    out = []
    for raw in lines:
        line = raw.split("//")[0].strip() if not raw.strip().startswith("//") else ""
        if line.startswith("{ "):          # block scopes of the emitted steps
            line = line[2:]
        if line.endswith("; }"):
            line = line[:-2]
        if not line or line in ("{", "}", "} break;") or line.startswith(_SKIP) or "launder(" in line:
            continue
        m = re.match(r"for \(int i = 0; i < (\d+); \+\+i\) (\w+)\[i\] = (.+);$", line)
        if m:
            n, arr, val = m.groups()
            out.append(f"{arr}[:] = [{val.replace('[i]', '[_i]').replace('0.0f', '0.0')} for _i in range({n})]")
            continue
        m = re.match(r"(?:V|float) (\w+\[\d+\](?:, \w+\[\d+\])*);$", line)
        if m:
            for decl in m.group(1).split(","):
                name, n = re.match(r"\s*(\w+)\[(\d+)\]", decl).groups()
                out.append(f"{name} = [0.0] * {n}")
            continue
        line = re.sub(r"^const (float|V) ", "", line)
        line = re.sub(r"\b(w|phi)\[(\d+) \* Cs?\]", r"\1[\2]", line)
        line = re.sub(r"(-?0x[0-9a-fA-F.]+p[+-]?\d+)f", lambda mm: repr(float.fromhex(mm.group(1))), line)
        line = re.sub(r"\b(\d+\.\d+)f\b", r"\1", line)
        assert line.endswith(";"), raw
        out.append(line[:-1])
    return out


def _branch(body, which):
    """Keep one branch of an emitted ``if constexpr (__is_same(V, float)) { ... } else { ... }``:
    "float" (the straight-line code) or "generic" (the step loop)."""
    out, mode = [], None
    for line in body:
        st = line.strip()
        if st == "if constexpr (__is_same(V, float)) {":
            mode = "float"
            continue
        if mode == "float" and line == "  } else {":
            mode = "generic"
            continue
        if mode == "generic" and line == "  }":
            mode = None
            continue
        if mode is None or mode == which:
            out.append(line)
    return out


def _functions(text, which="float"):
    """{name: python source} for forward / vjp / weight_features of one emitted plan."""
    segs = text.split("  template <typename V>\n")[1:]
    funcs = {}
    for seg in segs:
        name = re.search(r"void (\w+)\(", seg).group(1)
        body = seg[seg.index("{\n") + 2:].split("\n")
        while body and body[-1].strip() in ("", "};", "}}  // namespace ictc::sc") or body[-1].startswith("}"):
            body.pop()
        body = [b for b in _branch(body, which) if not b.startswith("  // ")]
        funcs[name] = "\n".join(_translate(body))
    return funcs


def _run(src, **env):
    ns = dict(env, sfma=lambda a, b, c: a * b + c, part=lambda a: a)
    exec(src, ns)  # noqa: S102 - the statements come from this repository's own generator
    return ns


def _dense(lmax, target, corr, x, w):
    """out[l_out] [C, 2l+1] = sum_order sum_p W_p U_p[x,...] (float64 torch, differentiable in x)."""
    _, offsets, _ = gen_sc._columns(lmax, target, corr)
    outs = []
    for lo in range(target + 1):
        acc = torch.zeros(x.shape[0], 2 * lo + 1, dtype=torch.float64)
        for order in range(corr, 0, -1):
            u = torch.from_numpy(S.u_matrix(lmax, lo, order))
            if lo == 0:
                u = u.unsqueeze(0)
            k = u.shape[-1]
            if k == 0:
                continue
            wp = w[:, offsets[(lo, order)]:offsets[(lo, order)] + k]          # [C, K]
            if order == 1:
                acc = acc + torch.einsum("mip,ci,cp->cm", u, x, wp)
            elif order == 2:
                acc = acc + torch.einsum("mijp,ci,cj,cp->cm", u, x, x, wp)
            else:
                acc = acc + torch.einsum("mijkp,ci,cj,ck,cp->cm", u, x, x, x, wp)
        outs.append(acc)
    return torch.cat(outs, 1)                                             # [C, (T+1)^2]


@pytest.mark.parametrize("lmax,target,corr", [(3, 1, 3), (3, 3, 3), (3, 0, 3), (2, 2, 3), (3, 2, 2),
                                              (1, 1, 3), (2, 0, 2), (0, 0, 3)])
def test_generated_plan_matches_dense_u(lmax, target, corr):
    text = gen_sc.emit(lmax, target, corr)
    funcs = _functions(text)
    d, no = (lmax + 1) ** 2, (target + 1) ** 2
    ktot = gen_sc.weight_columns(lmax, target, corr)
    chans = 5
    g = torch.Generator().manual_seed(lmax * 100 + target * 10 + corr)
    x = torch.randn(chans, d, generator=g, dtype=torch.float64)
    w = torch.randn(chans, ktot, generator=g, dtype=torch.float64)
    u = torch.randn(chans, no, generator=g, dtype=torch.float64)
    xs, ws, us = list(x.T.numpy()), list(w.T.numpy()), list(u.T.numpy())

    xt = x.clone().requires_grad_()
    dense = _dense(lmax, target, corr, xt, w)
    dxe = torch.autograd.grad((dense * u).sum(), xt)[0]
    scale_f, scale_b = dense.abs().max().item(), dxe.abs().max().item()

    for which, fn in (("float", funcs["forward"]), ("generic", _functions(text, "generic")["forward"])):
        o = [np.zeros(chans) for _ in range(no)]
        _run(fn, x=xs, w=ws, C=chans, o=o)
        err = np.abs(np.stack(o, 1) - dense.detach().numpy()).max() / scale_f
        assert err < TOL, f"forward ({which} branch) relative error {err:.3e}"

    dx = [np.zeros(chans) for _ in range(d)]
    _run(funcs["vjp"], x=xs, w=ws, C=chans, u=us, dx=dx)
    err = np.abs(np.stack(dx, 1) - dxe.numpy()).max() / scale_b
    assert err < TOL, f"vjp relative error {err:.3e}"

    phi = [np.zeros(chans) for _ in range(ktot)]
    _run(funcs["weight_features"], x=xs, C=chans, u=us, phi=phi)
    # <u, forward(x; w)> is linear in w with gradient phi
    wt = w.clone().requires_grad_()
    phie = torch.autograd.grad((_dense(lmax, target, corr, x, wt) * u).sum(), wt)[0]
    phi = [np.broadcast_to(v, (chans,)) for v in phi]
    err = np.abs(np.stack(phi, 1) - phie.numpy()).max() / phie.abs().max().item()
    assert err < TOL, f"weight features relative error {err:.3e}"


def test_accumulator_batches_stay_within_bound():
    """Every batch of coupling accumulators fits QMAX floats (or holds a single triple wider
    than that), one mid per batch, and every
    order-2/3 chain of a non-vanishing prefix is evaluated exactly once."""
    for lmax, target, corr in gen_sc.configs():
        order1, vanishing, groups, batches, o2_only = gen_sc._schedule(lmax, target, corr)
        seen = [p for p in (q for _, q in order1)] + list(vanishing)
        for b in batches:
            mids = {t[0] for t, _ in b["triples"]}
            assert len(mids) <= 1
            if b["triples"]:
                t, off = b["triples"][-1]
                assert off + 2 * t[0] + 1 <= max(gen_sc.QMAX, 2 * t[0] + 1)
            ts = {t for t, _ in b["triples"]}
            for key in b["groups"]:
                seen += [p for t, p, _ in groups[key]["o3"] if t in ts]
            for members in b["o2"].values():
                seen += [p for _, p, _ in members]
        for key in o2_only:
            seen += [p for _, p, _ in groups[key]["o2"]]
        assert sorted(seen) == list(range(gen_sc.weight_columns(lmax, target, corr)))
