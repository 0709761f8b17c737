"""Emit generated/sc_<lmax><target><corr>.hpp: straight-line device code of the
symmetric contraction for one (lmax, target_lmax, correlation) configuration.

Every U column (a coupling chain, see ictc_o3/basis/symmetric_u.py) of every target
degree and order contributes  w_p * chain_p(x)  to the output, where
w_p = W[species, p, channel] is read at ``w[p*C]`` (W columns concatenated per target
degree as [order corr, corr-1, ..., 1], the reference's weights_max, weights[0], ...
order).  The chains are evaluated in two shared stages:

* pair prefixes P_{la,lb,mid}[q] = sum_ij CG(la,lb,mid)[i,j,q] x_la,i x_lb,j, once per
  (la <= lb, mid) group; the swapped pair uses the exchange sign of the intertwiner and
  symmetric groups (la == lb) whose prefix vanishes identically are skipped;
* the final coupling of an order-3 chain, CG(mid,lc,l_out)[P, x_lc], is linear in P, so
  the chains that share (mid, lc, l_out) first accumulate  Q = sum_p w_p sign_p P_p  and
  are then coupled once:  o_l_out += CG(mid,lc,l_out)[Q, x_lc].  At lmax 3 -> 0e+1o this
  is 13 couplings instead of 69.  The accumulators of one mid are live together, split
  into batches of at most QMAX floats (register bound).

The float forward is emitted as straight-line code (fewest instructions: no loop-carried copies,
every CG literal folded into its FMA); the dual-number forward, the VJP and the weight features run
one switch case per accumulator batch inside a non-unrolled loop (straight-line within a batch,
registers bounded by the batch; their fully straight-line forms spill).

The VJP runs the same schedule backwards per batch: accumulate Q, couple's adjoint to x_lc
(reading Q), Q := the coupling's adjoint to the prefix, then per group the prefix adjoint
G = sum_p w_p sign_p Q_p (plus order-2 members) and its adjoint to x.  The weight
features are <P_p, adjoint of p's coupling>, one dot per chain.

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
import re
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


# accumulator floats live per batch (the Q array below); bounds register pressure
QMAX = 21


def _schedule(lmax: int, target: int, corr: int):
    """Chains grouped for evaluation.

    Returns (order1, vanishing, groups, batches, o2_only):
      groups[key] = {"o2": [(l_out, p, sign)], "o3": [(triple, p, sign)]} per pair prefix
        key = (la <= lb, mid); triple = (mid, lc, l_out);
      batches = [{"triples": [(triple, q_offset)], "groups": [key], "o2": {key: [...]}}]
        per mid (ascending), triples packed greedily so that sum(2 mid + 1) <= QMAX; a group's
        order-2 members ride with the first batch that evaluates the group's prefix;
      o2_only = groups without order-3 members (evaluated on their own).
    """
    cols, _, _ = _columns(lmax, target, corr)
    order1, vanishing, groups, triples = [], [], {}, set()
    for lo, order, ch, p in cols:
        if order == 1:
            order1.append((lo, p))
            continue
        key, sign = _pair_group(ch.la, ch.lb, ch.mid)
        if sign == 0:
            vanishing.append(p)
            continue
        g = groups.setdefault(key, {"o2": [], "o3": []})
        if order == 2:
            g["o2"].append((lo, p, sign))
        else:
            t = (ch.mid, ch.lc, lo)
            g["o3"].append((t, p, sign))
            triples.add(t)
    batches = []
    for mid in sorted({t[0] for t in triples}):
        cur, size = [], 0
        for t in sorted(t for t in triples if t[0] == mid):
            n = 2 * mid + 1
            if cur and size + n > QMAX:
                batches.append(cur)
                cur, size = [], 0
            cur.append((t, size))
            size += n
        batches.append(cur)
    placed, out = set(), []
    for trip in batches:
        ts = {t for t, _ in trip}
        keys = sorted(k for k, g in groups.items() if any(t in ts for t, _, _ in g["o3"]))
        o2 = {k: groups[k]["o2"] for k in keys if k not in placed and groups[k]["o2"]}
        placed.update(keys)
        out.append({"triples": trip, "groups": keys, "o2": o2})
    o2_only = sorted(k for k, g in groups.items() if not g["o3"])
    return order1, vanishing, groups, out, o2_only


def _split_args(text: str) -> List[str]:
    """Top-level comma-separated arguments of a call's argument text."""
    args, depth, cur = [], 0, ""
    for ch in text:
        if ch == "," and depth == 0:
            args.append(cur.strip())
            cur = ""
            continue
        depth += (ch == "(") - (ch == ")")
        cur += ch
    args.append(cur.strip())
    return args


_ASSIGN = re.compile(r"^(\s*)(?:\{ )?(\w+\[\d+\]) = (.*);( \})?$")
_ZERO_LOOP = re.compile(r"for \(int i = 0; i < (\d+); \+\+i\) (\w+)\[i\] = 0\.0f;")


def _fold_zero_starts(lines: List[str]) -> List[str]:
    """Rewrite the first accumulation into an accumulator known to hold exactly 0,
    ``X = sfma(a, b, X)``, as the product ``X = a * b``.  fma(a, b, +0) needs a VOP3 encoding
    that cannot hold a literal operand, so the compiler moves the constant into an SGPR, and on
    gfx950 a VALU instruction with an SGPR operand issues at half the rate of one whose operands
    are VGPRs or a literal (4.1 against 2.1 cycles per wave64 instruction, measured); the product
    has a VOP2 form with the literal.  The value only differs in the sign of an exact zero
    product, which no later sum can tell.  Straight-line statements only: the known zeros are
    those assigned 0.0f earlier in the same list of lines."""
    zero, out = set(), []
    for raw in lines:
        for line in raw.split("\n"):
            m = _ZERO_LOOP.search(line)
            if m:
                zero.update(f"{m.group(2)}[{i}]" for i in range(int(m.group(1))))
                out.append(line)
                continue
            m = _ASSIGN.match(line)
            if m:
                indent, target, rhs, close = m.groups()
                if rhs == "0.0f":
                    zero.add(target)
                else:
                    if rhs.startswith("sfma(") and rhs.endswith(")") and target in zero:
                        args = _split_args(rhs[5:-1])
                        if len(args) == 3 and args[2] == target:
                            opened = "{ " if line.strip().startswith("{ ") else ""
                            line = f"{indent}{opened}{target} = {args[0]} * ({args[1]});{close or ''}"
                    zero.discard(target)
            out.append(line)
    return out


def emit(lmax: int, target: int, corr: int) -> str:
    D, NO = (lmax + 1) ** 2, (target + 1) ** 2
    _, offsets, ktot = _columns(lmax, target, corr)
    order1, vanishing, groups, batches, o2_only = _schedule(lmax, target, corr)
    X = lambda l, m: f"xl[{l * l + m}]"           # noqa: E731
    U = lambda l, m: f"ul[{l * l + m}]"           # noqa: E731
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

    maxq = max([1] + [2 * k[2] + 1 for k in groups])
    qn = max([1] + [off + 2 * t[0] + 1 for b in batches for t, off in b["triples"]])

    def nested(pairs):
        """sum of coef * operand as one nested sfma chain ([(coef, operand)], coef a literal),
        started by a plain product (see _fold_zero_starts)."""
        (v0, op0), rest = pairs[0], pairs[1:]
        expr = f"{_f(v0)} * {op0}"
        for v, operand in rest:
            expr = f"sfma({_f(v)}, {operand}, {expr})"
        return expr

    def by_pair(terms):
        pairs = {}
        for i, j, q, v in terms:
            pairs.setdefault((i, j), []).append((q, v))
        return pairs

    def prefix(key):
        """P[q] = sum v x_a,i x_b,j, pair-major: one product live at a time."""
        a, b, mid = key
        lines = [f"    // pair prefix ({a},{b})->{mid}"] + [f"    P[{q}] = 0.0f;" for q in range(2 * mid + 1)]
        for (i, j), qs in by_pair(_pair_terms(a, b, mid)).items():
            lines.append(f"    {{ const V pr = {X(a, i)} * {X(b, j)};")
            lines += [f"      P[{q}] = sfma({_f(v)}, pr, P[{q}]);" for q, v in qs]
            lines.append("    }")
        return lines

    def prefix_adjoint(key):
        """dx from the prefix adjoint G: h_ij = sum_q v G[q] per pair, then two FMAs."""
        a, b, _ = key
        lines = []
        for (i, j), qs in by_pair(_pair_terms(*key)).items():
            h = nested([(v, f"G[{q}]") for q, v in qs])
            lines.append(f"    {{ const V h = {h};")
            if a == b and i == j:
                lines.append(f"      dx[{a * a + i}] = sfma(h + h, {X(a, i)}, dx[{a * a + i}]); }}")
            else:
                lines.append(f"      dx[{a * a + i}] = sfma(h, {X(b, j)}, dx[{a * a + i}]);")
                lines.append(f"      dx[{b * b + j}] = sfma(h, {X(a, i)}, dx[{b * b + j}]); }}")
        return lines

    def weight(p, sign, name):
        return f"    const float {name} = {sign}.0f * w[{p} * Cs];"

    def entries(t):
        mid, lc, lo = t
        c2 = coupling(mid, lc, lo)
        return [(q, k, m, c2[q, k, m]) for q in range(2 * mid + 1) for k in range(2 * lc + 1)
                for m in range(2 * lo + 1) if abs(c2[q, k, m]) > EPS]

    def coupling_lines(t, off):
        """o_m += sum_k x_k (sum_q c[q,k,m] Q[q])."""
        mid, lc, lo = t
        km = {}
        for q, k, m, v in entries(t):
            km.setdefault((k, m), []).append((v, f"Q[{off + q}]"))
        return [f"    o[{lo * lo + m}] = sfma({X(lc, k)}, {nested(terms)}, o[{lo * lo + m}]);"
                for (k, m), terms in sorted(km.items(), key=lambda kv: (kv[0][1], kv[0][0]))]

    def coupling_adjoint_x(t, off):
        """dx_k += sum_m u_m (sum_q c[q,k,m] Q[q])  (reads the accumulated prefix)."""
        mid, lc, lo = t
        km = {}
        for q, k, m, v in entries(t):
            km.setdefault((k, m), []).append((v, f"Q[{off + q}]"))
        return [f"    dx[{lc * lc + k}] = sfma({U(lo, m)}, {nested(terms)}, dx[{lc * lc + k}]);"
                for (k, m), terms in sorted(km.items())]

    def dual_coupling(t, off):
        """Q[off + q] = sum_m u_m (sum_k c[q,k,m] x_k): the adjoint of the triple's coupling
        with respect to its accumulated prefix."""
        mid, lc, lo = t
        qm = {}
        for q, k, m, v in entries(t):
            qm.setdefault(q, {}).setdefault(m, []).append((v, X(lc, k)))
        lines = []
        for q in range(2 * mid + 1):
            expr = None
            for m, terms in sorted(qm.get(q, {}).items()):
                expr = (f"{U(lo, m)} * ({nested(terms)})" if expr is None
                        else f"sfma({U(lo, m)}, {nested(terms)}, {expr})")
            lines.append(f"    Q[{off + q}] = {expr or '0.0f'};")
        return lines

    fsteps, bsteps, asteps = [], [], []
    fgroups, bgroups, agroups = [], [], []     # steps per batch: one loop case per batch
    for batch in batches:
        nf0, nb0, na0 = len(fsteps), len(bsteps), len(asteps)
        offs = dict(batch["triples"])
        # forward / VJP phase A: accumulate the weighted prefixes of each triple
        for key in batch["groups"]:
            g = groups[key]
            nq = 2 * key[2] + 1
            f = prefix(key)
            acc = []
            for r, (t, p, sign) in enumerate(m for m in g["o3"] if m[0] in offs):
                acc.append(weight(p, sign, f"wq{r}"))
                acc += [f"    Q[{offs[t] + q}] = sfma(wq{r}, P[{q}], Q[{offs[t] + q}]);" for q in range(nq)]
            f += acc
            for r, (lo, p, sign) in enumerate(batch["o2"].get(key, [])):
                f.append(weight(p, sign, f"wo{r}"))
                f += [f"    o[{lo * lo + m}] = sfma(wo{r}, P[{m}], o[{lo * lo + m}]);" for m in range(2 * lo + 1)]
            fsteps.append(f)
            bsteps.append(prefix(key) + acc)
        # forward: one coupling per triple on the accumulated prefix (then clear its slots)
        for t, off in batch["triples"]:
            mid, lc, lo = t
            f = [f"    // coupling ({mid},{lc})->{lo}"] + coupling_lines(t, off)
            f += [f"    Q[{off + q}] = 0.0f;" for q in range(2 * mid + 1)]
            fsteps.append(f)
        # VJP phase B: coupling adjoint to x_lc (reads Q), then Q := adjoint to the prefix
        for t, off in batch["triples"]:
            mid, lc, lo = t
            b_ = [f"    // coupling adjoint ({mid},{lc})->{lo}"] + coupling_adjoint_x(t, off)
            b_ += dual_coupling(t, off)
            bsteps.append(b_)
        # VJP phase C: prefix adjoint G = sum_p w_p (adjoint of p's triple) per group
        for n, key in enumerate(batch["groups"]):
            g = groups[key]
            nq = 2 * key[2] + 1
            b_ = [f"    // prefix adjoint ({key[0]},{key[1]})->{key[2]}"] + [f"    G[{q}] = 0.0f;" for q in range(nq)]
            for r, (t, p, sign) in enumerate(m for m in g["o3"] if m[0] in offs):
                b_.append(weight(p, sign, f"wq{r}"))
                b_ += [f"    G[{q}] = sfma(wq{r}, Q[{offs[t] + q}], G[{q}]);" for q in range(nq)]
            for r, (lo, p, sign) in enumerate(batch["o2"].get(key, [])):
                b_.append(weight(p, sign, f"wo{r}"))
                b_ += [f"    G[{q}] = sfma(wo{r}, {U(lo, q)}, G[{q}]);" for q in range(nq)]
            b_ += prefix_adjoint(key)
            if n == len(batch["groups"]) - 1:
                b_ += [f"    Q[{i}] = 0.0f;" for i in range(qn)]
            bsteps.append(b_)
        fgroups.append(len(fsteps) - nf0)
        bgroups.append(len(bsteps) - nb0)
        # weight features: Q := prefix adjoints of the triples, then one dot per chain
        for t, off in batch["triples"]:
            asteps.append([f"    // coupling adjoint ({t[0]},{t[1]})->{t[2]}"] + dual_coupling(t, off))
        for key in batch["groups"]:
            g = groups[key]
            nq = 2 * key[2] + 1
            ad = prefix(key)
            for t, p, sign in g["o3"]:
                if t in offs:
                    dot = " + ".join(f"P[{q}] * Q[{offs[t] + q}]" for q in range(nq))
                    ad.append(f"    phi[{p} * Cs] = {sign}.0f * part({dot});")
            for lo, p, sign in batch["o2"].get(key, []):
                dot = " + ".join(f"{U(lo, m)} * P[{m}]" for m in range(2 * lo + 1))
                ad.append(f"    phi[{p} * Cs] = {sign}.0f * part({dot});")
            asteps.append(ad)
        agroups.append(len(asteps) - na0)
    for key in o2_only:
        fgroups.append(1)
        bgroups.append(1)
        agroups.append(1)
        g = groups[key]
        nq = 2 * key[2] + 1
        f, ad = prefix(key), prefix(key)
        b_ = [f"    // order-2 prefix adjoint ({key[0]},{key[1]})->{key[2]}"] + [f"    G[{q}] = 0.0f;" for q in range(nq)]
        for r, (lo, p, sign) in enumerate(g["o2"]):
            f.append(weight(p, sign, f"wo{r}"))
            f += [f"    o[{lo * lo + m}] = sfma(wo{r}, P[{m}], o[{lo * lo + m}]);" for m in range(2 * lo + 1)]
            b_.append(weight(p, sign, f"wo{r}"))
            b_ += [f"    G[{q}] = sfma(wo{r}, {U(lo, q)}, G[{q}]);" for q in range(nq)]
            dot = " + ".join(f"{U(lo, m)} * P[{m}]" for m in range(2 * lo + 1))
            ad.append(f"    phi[{p} * Cs] = {sign}.0f * part({dot});")
        fsteps.append(f)
        bsteps.append(b_ + prefix_adjoint(key))
        asteps.append(ad)

    def straight(steps, decl):
        # the steps one after another in their own scopes (no loop, nothing laundered)
        out = [f"  {decl}"]
        for k, body in enumerate(steps):
            out.append(f"  {{  // step {k}")
            out.extend(body)
            out.append("  }")
        return _fold_zero_starts([ln.replace("* Cs]", "* C]") for ln in out])

    def merged(steps, sizes):
        """Concatenate consecutive steps into one step per group (sizes sum to len(steps))."""
        out, k = [], 0
        for n in sizes:
            body = []
            for st in steps[k:k + n]:
                body += ["    {"] + st + ["    }"]
            out.append(body)
            k += n
        assert k == len(steps)
        return out

    def loop(steps, decl, with_u=False):
        # C, the input copy and (when used) the cotangent copy are re-laundered every
        # iteration, so that weight addresses and products of x or u with constants are
        # formed inside their step instead of being hoisted (all at once) out of the loop
        out = [f"  {decl}"]
        if with_u:
            out.append(f"float ul[{NO}];\n  for (int i = 0; i < {NO}; ++i) ul[i] = u[i];")
        out += ["  #pragma clang loop unroll(disable)",
                f"  for (int step = 0; step < {len(steps)}; ++step) {{",
                '    int Cs = C;', '    asm volatile("" : "+s"(Cs));',
                f"    #pragma unroll\n    for (int i = 0; i < {D}; ++i) launder(xl[i]);"]
        if with_u:
            out.append(f"    #pragma unroll\n    for (int i = 0; i < {NO}; ++i) launder(ul[i]);")
        out.append("    switch (step) {")
        for k, body in enumerate(steps):
            out.append(f"    case {k}: {{")
            out.extend("  " + line for line in _fold_zero_starts(body))
            out.append("    } break;")
        out += ["    default: break;", "    }", "  }"]
        return out
    if fsteps:
        copy = f"V xl[{D}];\n  for (int i = 0; i < {D}; ++i) xl[i] = x[i];\n  "
        zq = f"V Q[{qn}];\n  for (int i = 0; i < {qn}; ++i) Q[i] = 0.0f;\n  "
        # float forward: straight-line (no loop-carried copies, constants folded into the FMAs;
        # more registers, fewer instructions); dual-number forward (the JVP): the step loop
        fw += ["  if constexpr (__is_same(V, float)) {"] + straight(fsteps, copy + zq + f"V P[{maxq}];")
        fw += ["  } else {"] + loop(merged(fsteps, fgroups), copy + zq + f"V P[{maxq}];") + ["  }"]
        bw += loop(merged(bsteps, bgroups), copy + zq + f"V P[{maxq}], G[{maxq}];", with_u=True)
        aw += loop(merged(asteps, agroups), copy + f"V Q[{qn}];\n  V P[{maxq}];", with_u=True)
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
