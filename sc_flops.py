"""Useful floating-point operations of the generated symmetric-contraction code.

The emitted Plan<L, T, K> (gen_sc.py) is straight-line C++ per (node, channel) lane.  Its
statements are translated into Python and executed once over a scalar type that only tracks
whether a value is exactly zero, exactly +-1 (a literal) or anything else, and counts the
arithmetic that does work:

* a product with an exact zero or +-1 operand costs nothing (it is a copy or a sign);
* a sum with an exact zero operand costs nothing;
* ``sfma(a, b, c)`` costs its product and its sum by the two rules above (2, 1 or 0).

So an accumulator set to 0 and then fed one fma counts one multiply, and a product by the
literal 1.0 counts nothing.  These are useful FLOPs (the arithmetic the contraction needs),
not executed instructions; the hardware's executed counts come from the VALU counters
(``SQ_INSTS_VALU_FMA_F32`` / ``_MUL_F32`` / ``_ADD_F32``).
"""
from __future__ import annotations

import os
import re
import sys
from typing import Dict, List

_SKIP = ("//", "#pragma", "asm ", "switch", "case ", "default:", "for (int step", "int Cs = C;")


class _Tally:
    def __init__(self):
        self.flops = 0


class _Val:
    """'z' (exact zero), 'o' (exact +-1) or 'g' (general)."""
    __slots__ = ("kind", "tally")

    def __init__(self, kind: str, tally: _Tally):
        self.kind, self.tally = kind, tally

    @staticmethod
    def of(value, tally: _Tally) -> "_Val":
        if isinstance(value, _Val):
            return value
        value = float(value)
        return _Val("z" if value == 0.0 else "o" if abs(value) == 1.0 else "g", tally)

    def _mul(self, other, count=True):
        o = _Val.of(other, self.tally)
        if "z" in (self.kind, o.kind):
            return _Val("z", self.tally), 0
        if self.kind == "o":
            return _Val(o.kind, self.tally), 0
        if o.kind == "o":
            return _Val(self.kind, self.tally), 0
        return _Val("g", self.tally), 1

    def _add(self, other):
        o = _Val.of(other, self.tally)
        if self.kind == "z":
            return o, 0
        if o.kind == "z":
            return self, 0
        return _Val("g", self.tally), 1

    def __mul__(self, other):
        value, flops = self._mul(other)
        self.tally.flops += flops
        return value

    __rmul__ = __mul__

    def __add__(self, other):
        value, flops = self._add(other)
        self.tally.flops += flops
        return value

    __radd__ = __add__

    def __sub__(self, other):
        return self + (-_Val.of(other, self.tally))

    def __rsub__(self, other):
        return _Val.of(other, self.tally) + (-self)

    def __neg__(self):
        return _Val(self.kind, self.tally)


def _sfma(a, b, c, tally: _Tally):
    a = _Val.of(a, tally)
    prod, mul_flops = a._mul(b)
    value, add_flops = prod._add(c)
    tally.flops += mul_flops + add_flops
    return value


def translate(lines: List[str]) -> List[str]:
    """Emitted C++ statements -> Python statements over lists of scalars."""
    out = []
    for raw in lines:
        line = raw.split("//")[0].strip() if not raw.strip().startswith("//") else ""
        if line.startswith("{ "):
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
        if not line.endswith(";"):
            raise ValueError(f"unexpected emitted statement: {raw!r}")
        out.append(line[:-1])
    return out


def _float_branch(body: List[str]) -> List[str]:
    """Keep the straight-line float branch of an ``if constexpr (__is_same(V, float))``."""
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
        if mode in (None, "float"):
            out.append(line)
    return out


def functions(text: str) -> Dict[str, str]:
    """{forward, vjp, weight_features: Python source} of one emitted plan (float branch)."""
    funcs = {}
    for seg in text.split("  template <typename V>\n")[1:]:
        name = re.search(r"void (\w+)\(", seg).group(1)
        body = seg[seg.index("{\n") + 2:].split("\n")
        while body and (body[-1].strip() in ("", "};", "}}  // namespace ictc::sc") or body[-1].startswith("}")):
            body.pop()
        body = [b for b in _float_branch(body) if not b.startswith("  // ")]
        funcs[name] = "\n".join(translate(body))
    return funcs


def useful_flops(text: str, D: int, NO: int, KTOT: int) -> Dict[str, int]:
    """Useful FLOPs per (node, channel) lane of forward and vjp of one emitted plan."""
    out = {}
    for name, src in functions(text).items():
        if name not in ("forward", "vjp"):
            continue
        tally = _Tally()
        g = lambda: _Val("g", tally)                                   # noqa: E731
        env = {"x": [g() for _ in range(D)], "w": [g() for _ in range(KTOT)],
               "o": [_Val("z", tally) for _ in range(NO)], "u": [g() for _ in range(NO)],
               "dx": [_Val("z", tally) for _ in range(D)], "C": 1, "Cs": 1,
               "sfma": lambda a, b, c: _sfma(a, b, c, tally), "part": lambda a: a}
        exec(src, env)  # noqa: S102 - statements emitted by this repository's own generator
        out[name] = tally.flops
    return out


def flop_counts(lmax: int, target: int, corr: int) -> Dict[str, int]:
    """Useful floating-point operations per (node, channel) of the emitted float forward and VJP
    of one (lmax, target, correlation) configuration (products with an exact zero or +-1 and
    sums with an exact zero are free; an fma is its product plus its sum)."""
    csrc = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ictc-o3-hp-ascend_amd", "csrc")
    if csrc not in sys.path:
        sys.path.insert(0, csrc)
    import gen_sc
    D, NO, ktot = (lmax + 1) ** 2, (target + 1) ** 2, gen_sc.weight_columns(lmax, target, corr)
    return useful_flops(gen_sc.emit(lmax, target, corr), D, NO, ktot)
