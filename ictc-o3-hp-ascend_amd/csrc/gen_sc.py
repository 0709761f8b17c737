"""Emit generated/sc_<lmax><target><corr>.hpp: straight-line device code of the
symmetric contraction for one (lmax, target_lmax, correlation) configuration.

For every U column (a coupling chain, see ictc_o3/basis/symmetric_u.py) of every
target degree and order, the emitted code adds  w_p * chain_p(x)  to the output,
where w_p = W[species, p, channel] is read at ``w[p*C]`` (W columns concatenated per
target degree as [order corr, corr-1, ..., 1], the reference's weights_max,
weights[0], ... order).  Chains share their pair prefixes
P_{la,lb,L1}[q] = sum_ij CG(la,lb,L1)[i,j,q] x_la,i x_lb,j, evaluated once per
(la <= lb, L1) group; the swapped pair uses the exchange sign of the intertwiner and
symmetric groups (la == lb) whose prefix vanishes identically are skipped.

Emitted per configuration (struct ``ictc::sc::Plan<L, T, K>``), each a template over
the scalar V of x (float, or the dual number ictc::sc::Dual of sc_plan.hpp, whose
tangent part turns forward into a JVP, vjp into a Hessian-vector product and
weight_features into its directional derivative):
  forward(x, w, C, o)     o[T-packed] += sum_p w_p chain_p(x)
  vjp(x, w, C, u, dx)     dx = d/dx <u, forward(x)>
  weight_features(x, C, u, phi)   phi[p*C] = <u, chain_p(x)> (the weight adjoint per node)
plus constants D (input components), NO (output components), KTOT (weight columns)
and the per-(degree, order) column offsets.

Usage: python gen_sc.py <out_dir> [configs...]   (config = "LTK", e.g. "313")
"""
from __future__ import annotations

import os
import sys
from typing import Dict, List, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from ictc_o3.basis.symmetric_u import chains, coupling  # noqa: E402

EPS = 1e-12


def _f(v: float) -> str:
    return float(np.float32(v)).hex() + "f"


def _columns(lmax: int, target: int, corr: int):
    """[(l_out, order, chain, column)] in W column order, and per-(l_out, order) offsets."""
    cols, offsets, p = [], {}, 0
    for lo in range(target + 1):
        for order in range(corr, 0, -1):
            offsets[(lo, order)] = p
            for ch in chains(lmax, lo, order):
                cols.append((lo, order, ch, p))
                p += 1
    return cols, offsets, p


def _pair_group(la: int, lb: int, mid: int):
    """(key, sign) such that P_{la,lb,mid} = sign * P_key, key = (min, max, mid); sign 0 when
    the prefix vanishes identically (antisymmetric coupling of equal degrees)."""
    c = coupling(la, lb, mid)
    if la == lb:
        if np.abs(c + c.transpose(1, 0, 2)).max() < EPS:
            return (la, lb, mid), 0
        if np.abs(c - c.transpose(1, 0, 2)).max() > 1e-10:
            raise RuntimeError(f"coupling ({la},{lb},{mid}) is neither symmetric nor antisymmetric")
        return (la, lb, mid), 1
    if la < lb:
        return (la, lb, mid), 1
    swapped = coupling(lb, la, mid).transpose(1, 0, 2)
    if np.abs(c - swapped).max() < 1e-10:
        return (lb, la, mid), 1
    if np.abs(c + swapped).max() < 1e-10:
        return (lb, la, mid), -1
    raise RuntimeError(f"no exchange symmetry for ({la},{lb},{mid})")


def _pair_terms(a: int, b: int, mid: int) -> List[Tuple[int, int, int, float]]:
    """Nonzero (i, j, q, v) of P_q = sum v x_{a,i} x_{b,j}; for a == b the (i,j)/(j,i) terms
    are merged onto i <= j."""
    c = coupling(a, b, mid)
    terms = []
    for i in range(2 * a + 1):
        for j in range(2 * b + 1):
            if a == b and j < i:
                continue
            for q in range(2 * mid + 1):
                v = c[i, j, q] + (c[j, i, q] if a == b and i != j else 0.0)
                if abs(v) > EPS:
                    terms.append((i, j, q, v))
    return terms


def emit(lmax: int, target: int, corr: int) -> str:
    D, NO = (lmax + 1) ** 2, (target + 1) ** 2
    cols, offsets, ktot = _columns(lmax, target, corr)
    # group the chains of order >= 2 by their pair prefix
    groups: Dict[Tuple[int, int, int], List] = {}
    order1, vanishing = [], []
    for lo, order, ch, p in cols:
        if order == 1:
            order1.append((lo, p))
            continue
        key, sign = _pair_group(ch.la, ch.lb, ch.mid)
        if sign == 0:
            vanishing.append(p)
            continue
        groups.setdefault(key, []).append((lo, order, ch, p, sign))
    X = lambda l, m: f"xl[{l * l + m}]"           # noqa: E731
    fw, bw, aw = [], [], []
    # ---- order 1
    for lo, p in order1:
        terms = []
        for m in range(2 * lo + 1):
            fw.append(f"  o[{lo * lo + m}] = sfma(w[{p} * C], x[{lo * lo + m}], o[{lo * lo + m}]);")
            bw.append(f"  dx[{lo * lo + m}] = sfma(w[{p} * C], u[{lo * lo + m}], dx[{lo * lo + m}]);")
            terms.append(f"u[{lo * lo + m}] * x[{lo * lo + m}]")
        aw.append(f"  phi[{p} * C] = part({' + '.join(terms)});")
    for p in vanishing:
        aw.append(f"  phi[{p} * C] = 0.0f;   // chain with an identically vanishing prefix")
    # ---- pair groups as a sequence of small steps (switch cases of a loop that is not
    # unrolled: every step is its own basic block, so register pressure and scheduling
    # regions stay bounded).  P (prefix) and G (its adjoint) are loop-carried arrays.
    fsteps, bsteps, asteps = [], [], []
    maxq = 1
    for (a, b, mid), members in sorted(groups.items()):
        terms = _pair_terms(a, b, mid)
        nq = 2 * mid + 1
        maxq = max(maxq, nq)
        pre = [f"    // pair group ({a},{b})->{mid}"]
        for q in range(nq):
            expr = "0.0f"
            for i, j, qq, v in terms:
                if qq == q:
                    expr = f"sfma({_f(v)}, {X(a, i)} * {X(b, j)}, {expr})"
            pre.append(f"    P[{q}] = {expr};")
        fsteps.append(pre)
        asteps.append(pre)
        bsteps.append(pre + [f"    G[{q}] = 0.0f;" for q in range(nq)])
        for lo, order, ch, p, sign in members:
            f, b_, ad = [], [], []
            f.append(f"    const float wv = {sign}.0f * w[{p} * Cs];")
            b_.append(f"    const float wv = {sign}.0f * w[{p} * Cs];")
            if order == 2:
                for m in range(2 * lo + 1):
                    f.append(f"    o[{lo * lo + m}] = sfma(wv, P[{m}], o[{lo * lo + m}]);")
                    b_.append(f"    G[{m}] = sfma(wv, u[{lo * lo + m}], G[{m}]);")
                ad.append(f"    phi[{p} * Cs] = {sign}.0f * part(" +
                          " + ".join(f"u[{lo * lo + m}] * P[{m}]" for m in range(2 * lo + 1)) + ");")
            else:
                lc = ch.lc
                c2 = coupling(mid, lc, lo)
                ent = [(aa, k, m, c2[aa, k, m]) for aa in range(nq) for k in range(2 * lc + 1)
                       for m in range(2 * lo + 1) if abs(c2[aa, k, m]) > EPS]
                for m in range(2 * lo + 1):
                    expr = "0.0f"
                    for aa, k, mm, v in ent:
                        if mm == m:
                            expr = f"sfma({_f(v)}, P[{aa}] * {X(lc, k)}, {expr})"
                    f.append(f"    o[{lo * lo + m}] = sfma(wv, {expr}, o[{lo * lo + m}]);")
                    b_.append(f"    const float um{m} = wv * u[{lo * lo + m}];")
                    ad.append(f"    const V t{m} = {expr};")
                ad.append(f"    phi[{p} * Cs] = {sign}.0f * part(" +
                          " + ".join(f"u[{lo * lo + m}] * t{m}" for m in range(2 * lo + 1)) + ");")
                for aa, k, m, v in ent:
                    b_.append(f"    G[{aa}] = sfma({_f(v)} * um{m}, {X(lc, k)}, G[{aa}]);")
                    b_.append(f"    dx[{lc * lc + k}] = sfma({_f(v)} * um{m}, P[{aa}], dx[{lc * lc + k}]);")
            fsteps.append(f)
            bsteps.append(b_)
            asteps.append(ad)
        adj = []
        for i, j, q, v in terms:
            if a == b and i == j:
                adj.append(f"    dx[{a * a + i}] = sfma({_f(2 * v)} * G[{q}], {X(a, i)}, dx[{a * a + i}]);")
            else:
                adj.append(f"    dx[{a * a + i}] = sfma({_f(v)} * G[{q}], {X(b, j)}, dx[{a * a + i}]);")
                adj.append(f"    dx[{b * b + j}] = sfma({_f(v)} * G[{q}], {X(a, i)}, dx[{b * b + j}]);")
        bsteps.append(adj)

    def loop(steps, decl):
        # C is re-laundered every iteration so that weight addresses are formed inside their
        # step instead of being hoisted (all at once) out of the loop
        out = [f"  {decl}", "  #pragma clang loop unroll(disable)",
               f"  for (int step = 0; step < {len(steps)}; ++step) {{",
               '    int Cs = C;', '    asm volatile("" : "+s"(Cs));',
               f"    #pragma unroll\n    for (int i = 0; i < {D}; ++i) launder(xl[i]);",
               "    switch (step) {"]
        for k, body in enumerate(steps):
            out.append(f"    case {k}: {{")
            out.extend("  " + line for line in body)
            out.append("    } break;")
        out += ["    default: break;", "    }", "  }"]
        return out
    if fsteps:
        copy = f"V xl[{D}];\n  for (int i = 0; i < {D}; ++i) xl[i] = x[i];\n  "
        fw += loop(fsteps, copy + f"V P[{maxq}];")
        bw += loop(bsteps, copy + f"V P[{maxq}], G[{maxq}];")
        aw += loop(asteps, copy + f"V P[{maxq}];")
    off_lines = ", ".join(str(offsets[(lo, o)]) for lo in range(target + 1) for o in range(corr, 0, -1))
    return "\n".join([
        f"// Generated by csrc/gen_sc.py for lmax={lmax}, target_lmax={target}, correlation={corr}.",
        "#pragma once",
        '#include "sc_plan.hpp"',
        "namespace ictc { namespace sc {",
        f"template <> struct Plan<{lmax}, {target}, {corr}> {{",
        f"  static constexpr int D = {D};",
        f"  static constexpr int NO = {NO};",
        f"  static constexpr int KTOT = {ktot};",
        f"  // first W column of (l_out, order), l_out ascending, order descending",
        f"  static constexpr int offsets[{(target + 1) * corr}] = {{{off_lines}}};",
        "  // x: the channel's input components (float, or Dual carrying a tangent);",
        "  // w: weight row of (species, channel).",
        "  template <typename V>",
        "  __device__ static __forceinline__ void forward(const V* x, const float* __restrict__ w, int C, V* o) {",
        *fw,
        "  }",
        "  template <typename V>",
        "  __device__ static __forceinline__ void vjp(const V* x, const float* __restrict__ w, int C,",
        "                                             const float* u, V* dx) {",
        f"    for (int i = 0; i < {D}; ++i) dx[i] = 0.0f;",
        *bw,
        "  }",
        "  // phi[p*C] = part(sum_m u_m chain_p(x)_m) for every weight column p (weight adjoint;",
        "  // part() is the value for float and the tangent for Dual)",
        "  template <typename V>",
        "  __device__ static __forceinline__ void weight_features(const V* x, int C, const float* u,",
        "                                                         float* __restrict__ phi) {",
        *aw,
        "  }",
        "};",
        "}}  // namespace ictc::sc",
        "",
    ])


def weight_columns(lmax: int, target: int, corr: int) -> int:
    return _columns(lmax, target, corr)[2]


def flop_counts(lmax: int, target: int, corr: int) -> Dict[str, int]:
    """Floating-point operations per (node, channel) of the emitted forward and VJP, counted
    on the emitted code: an fma counts 2, a multiply or an add 1."""
    import re
    text = emit(lmax, target, corr)
    bodies = {"forward": text[text.index("void forward"):text.index("void vjp")],
              "vjp": text[text.index("void vjp"):text.index("void weight_features")]}
    return {k: 2 * b.count("sfma(") + len(re.findall(r" [*+] ", b)) for k, b in bodies.items()}


def configs():
    return [(l, t, k) for l in range(4) for t in range(l + 1) for k in (1, 2, 3)]


def main(out_dir: str, which=None) -> List[Tuple[int, int, int]]:
    os.makedirs(out_dir, exist_ok=True)
    done = []
    for l, t, k in (which or configs()):
        path = os.path.join(out_dir, f"sc_{l}{t}{k}.hpp")
        text = emit(l, t, k)
        if not os.path.exists(path) or open(path).read() != text:
            with open(path, "w") as fh:
                fh.write(text)
        done.append((l, t, k))
    return done


if __name__ == "__main__":
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(HERE, "generated")
    sel = [tuple(int(ch) for ch in s) for s in sys.argv[2:]] or None
    print(main(out, sel))
