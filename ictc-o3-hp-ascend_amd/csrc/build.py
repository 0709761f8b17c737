"""Build libictc_hip.so for gfx950 with hipcc (no cmake/ninja).

Steps:
  1. generate ``generated/ictc_cg_table.hpp`` (CG constants from the frozen basis);
  2. write one translation unit per (input_lmax, edge_lmax, output_lmax, kernel
     kind) with the explicit template instantiation, plus ``tp_instances.def``
     listing the compiled combinations for the dispatch tables (every degree <= 3),
     and the tensor-product units of the wide sets in ``WIDE_COMBOS`` (listed in
     ``tp_wide_instances.def``; other sets with a degree of 4 to 6 run the
     degree-generic kernels);
  3. compile every TU to an object in parallel, largest first;
  4. link the objects and the API TUs into ``ictc_o3/lib/libictc_hip.so``;
  5. build ``libictc_stream_probe.so`` beside bench.py from the repository root's
     ``stream_probe.hip`` (bench.py's streaming-bandwidth and FMA-rate reference; not part of
     the operator library).

Every HIP TU is compiled with ``-Xclang -target-feature -Xclang -packed-fp32-ops``
(no packed FP32 VALU instructions are generated).

``ICTC_HIP_COMBOS`` (e.g. ``"333,222,033"``) restricts the degree combinations for
quick development builds; entries left out report ICTC_ERR_UNSUPPORTED at run time.

Usage: python build.py [-j JOBS] [--incremental]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)                         # ictc-o3-hp-ascend_amd/
REPO = os.path.dirname(PKG)
INCLUDE = os.path.join(REPO, "include")
GEN = os.path.join(HERE, "generated")
OBJ = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(PKG, "ictc_o3", "lib")
LIB = os.path.join(LIB_DIR, "libictc_hip.so")
PROBE_SRC = os.path.join(REPO, "stream_probe.hip")
PROBE_LIB = os.path.join(REPO, "libictc_stream_probe.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++20", "-fPIC", "-Wno-c99-designator",
         "-mcode-object-version=5",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I", INCLUDE, "-I", HERE]

API_SOURCES = ["tp_api.hip", "harmonics_api.hip", "message_api.hip", "sc_api.hip", "graph_api.hip",
               "elementwise_api.hip", "blas_api.hip", "linear_api.hip", "generic_kernels.hip",
               "edge_embedding_api.hip", "radial_mlp_api.hip", "species_linear_api.hip",
               "readout_api.hip"]
# rocBLAS (the channel-linear products): the same SONAME as the copy torch loads, which the
# dynamic linker then binds to
LINK_LIBS = ["-L/opt/rocm/lib", "-lrocblas"]
HARM_LMAX = 6
# degree sets above 3 with compiled tensor-product kernels (the symmetric lmax-4 set)
WIDE_COMBOS = [(4, 4, 4)]
INSTANCE_KINDS = {
    "fwd": ("tp_kernels.hpp", "template int launch_forward<{a}, {b}, {c}>(const ictc_tp_desc&, "
            "const float*, const float*, const float*, float*, int64_t, hipStream_t);"),
    "bwd": ("tp_kernels.hpp", "template int launch_backward<{a}, {b}, {c}>(const ictc_tp_desc&, "
            "const float*, const float*, const float*, const float*, float*, float*, float*, "
            "int64_t, hipStream_t);"),
    "msg": ("message_kernels.hpp",
            "template int launch_msg_bonds<{a}, {b}, {c}>(const ictc_tp_desc&, const float*, float*, "
            "int64_t, hipStream_t);\n"
            "template int launch_msg_forward<{a}, {b}, {c}>(const ictc_tp_desc&, const float*, "
            "const float*, const float*, const int64_t*, const int64_t*, const int64_t*, float*, "
            "int64_t, int64_t, hipStream_t);\n"
            "template int launch_msg_edge_grad<{a}, {b}, {c}>(const ictc_tp_desc&, const float*, "
            "const float*, const float*, const float*, const int64_t*, const int64_t*, const int64_t*, "
            "float*, float*, float*, int64_t, int64_t, hipStream_t, int);\n"
            "template int launch_msg_forward_tangent<{a}, {b}, {c}>(const ictc_tp_desc&, const float*, "
            "const float*, const float*, const MsgTangent&, const int64_t*, const int64_t*, const int64_t*, "
            "float*, int64_t, int64_t, hipStream_t);\n"
            "template int launch_msg_edge_grad_tangent<{a}, {b}, {c}>(const ictc_tp_desc&, const float*, "
            "const float*, const float*, const MsgTangent&, const float*, const int64_t*, const int64_t*, "
            "const int64_t*, float*, float*, float*, int64_t, int64_t, hipStream_t);"),
}


def _combos():
    spec = os.environ.get("ICTC_HIP_COMBOS", "").strip()
    if spec:
        out = []
        for tok in spec.split(","):
            tok = tok.strip()
            if len(tok) != 3 or not tok.isdigit() or any(int(ch) > 3 for ch in tok):
                raise SystemExit(f"bad ICTC_HIP_COMBOS entry {tok!r}")
            out.append(tuple(int(ch) for ch in tok))
        return sorted(set(out))
    return [(a, b, c) for a in range(4) for b in range(4) for c in range(4)]


def _sc_configs():
    """(lmax, target_lmax, correlation) of the symmetric-contraction plans to compile."""
    spec = os.environ.get("ICTC_HIP_SC", "").strip()
    if spec:
        return sorted({tuple(int(ch) for ch in tok.strip()) for tok in spec.split(",")})
    return [(l, t, k) for l in range(4) for t in range(l + 1) for k in (1, 2, 3)]


def _cost(a: int, b: int, c: int, kind: str) -> int:
    """Rough compile cost (path-set size) to start the biggest TUs first."""
    n = sum((2 * i + 1) * (2 * j + 1) * (2 * k + 1) for i in range(a + 1) for j in range(b + 1)
            for k in range(c + 1) if abs(i - j) <= k <= i + j and (i + j + k) % 2 == 0)
    return n * {"fwd": 1, "bwd": 4, "msg": 6}[kind]


def _write_if_changed(path: str, text: str) -> None:
    if not os.path.exists(path) or open(path).read() != text:
        with open(path, "w") as fh:
            fh.write(text)


def _generate(combos) -> list:
    os.makedirs(GEN, exist_ok=True)
    subprocess.run([sys.executable, os.path.join(HERE, "gen_cg_table.py"),
                    os.path.join(GEN, "ictc_cg_table.hpp")], check=True)
    _write_if_changed(os.path.join(GEN, "tp_instances.def"),
                      "".join(f"ICTC_DECLARE({a}, {b}, {c})\n" for a, b, c in combos))
    _write_if_changed(os.path.join(GEN, "tp_wide_instances.def"),
                      "".join(f"ICTC_DECLARE({a}, {b}, {c})\n" for a, b, c in WIDE_COMBOS))
    units = []
    for a, b, c in WIDE_COMBOS:
        for kind in ("fwd", "bwd"):
            header, line = INSTANCE_KINDS[kind]
            path = os.path.join(GEN, f"tp_inst_{a}{b}{c}_{kind}.hip")
            _write_if_changed(path, f'#define ICTC_CG_WIDE 1\n#include "{header}"\nnamespace ictc {{\n'
                                    f'{line.format(a=a, b=b, c=c)}\n}}  // namespace ictc\n')
            units.append((_cost(a, b, c, kind), path))
    for a, b, c in combos:
        for kind, (header, line) in INSTANCE_KINDS.items():
            path = os.path.join(GEN, f"{'msg' if kind == 'msg' else 'tp'}_inst_{a}{b}{c}_{kind}.hip")
            _write_if_changed(path, f'#include "{header}"\nnamespace ictc {{\n'
                                    f'{line.format(a=a, b=b, c=c)}\n}}  // namespace ictc\n')
            units.append((_cost(a, b, c, kind), path))
    for l in range(HARM_LMAX + 1):
        path = os.path.join(GEN, f"harm_inst_{l}.hip")
        _write_if_changed(path, '#include "harmonics.hpp"\nnamespace ictc {\n'
                                f'template int launch_harmonics<{l}>(int, const float*, const float*, '
                                'const float*, const float*, float*, int64_t, hipStream_t);\n'
                                '}  // namespace ictc\n')
        units.append((60 * (l + 1) ** 3, path))
    # symmetric contraction: generated straight-line plans, one TU per configuration
    sys.path.insert(0, HERE)
    import gen_sc
    sc_cfgs = _sc_configs()
    gen_sc.main(GEN, sc_cfgs)
    _write_if_changed(os.path.join(GEN, "sc_instances.def"),
                      "".join(f"ICTC_SC({l}, {t}, {k}, {gen_sc.weight_columns(l, t, k)})\n"
                              for l, t, k in sc_cfgs))
    for l, t, k in sc_cfgs:
        path = os.path.join(GEN, f"sc_inst_{l}{t}{k}.hip")
        _write_if_changed(path, f'#include "sc_kernels.hpp"\n#include "generated/sc_{l}{t}{k}.hpp"\n'
                                f'namespace ictc {{\ntemplate int launch_sc<{l}, {t}, {k}>(int, const float*, '
                                'const float*, const int64_t*, const float*, const float*, float*, int, '
                                'int64_t, int, '
                                'hipStream_t);\n}  // namespace ictc\n')
        units.append((os.path.getsize(os.path.join(GEN, f"sc_{l}{t}{k}.hpp")) // 20, path))
    units.sort(reverse=True)
    return [p for _, p in units]


_INCLUDE_RE = None


def _newest_dependency(src: str, seen=None) -> float:
    """Latest modification time of src and of every file it includes with quotes
    (searched next to it, in this directory, generated/ and include/)."""
    import re
    global _INCLUDE_RE
    if _INCLUDE_RE is None:
        _INCLUDE_RE = re.compile(r'^\s*#\s*include\s+"([^"]+)"', re.M)
    seen = set() if seen is None else seen
    if src in seen:
        return 0.0
    seen.add(src)
    newest = os.path.getmtime(src)
    for name in _INCLUDE_RE.findall(open(src).read()):
        for base in (os.path.dirname(src), HERE, GEN, INCLUDE):
            path = os.path.join(base, name)
            if os.path.isfile(path):
                newest = max(newest, _newest_dependency(path, seen))
                break
    return newest


def _compile(src: str, incremental: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    obj = os.path.join(OBJ, os.path.splitext(os.path.basename(src))[0] + ".o")
    if incremental and os.path.exists(obj) and os.path.getmtime(obj) >= _newest_dependency(src):
        return obj
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = True, incremental: bool = False) -> str:
    """Compile every unit (incremental: only units whose object is older than the unit or
    anything it includes) and link the library."""
    t0 = time.time()
    combos = _combos()
    units = [os.path.join(HERE, s) for s in API_SOURCES] + _generate(combos)
    jobs = jobs or max(1, min(len(units), os.cpu_count() or 1))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda u: _compile(u, incremental), units))
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    res = subprocess.run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", *objs, *LINK_LIBS, "-o", tmp],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    res = subprocess.run([HIPCC, *FLAGS, "-shared", PROBE_SRC, "-o", PROBE_LIB + ".tmp"],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"stream probe build failed:\n{res.stderr}")
    os.replace(PROBE_LIB + ".tmp", PROBE_LIB)
    if verbose:
        print(f"built {LIB} ({len(combos)} degree combinations, {len(units)} units, "
              f"{time.time() - t0:.0f}s)", flush=True)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--incremental", action="store_true",
                    help="recompile only units whose sources or included headers changed")
    args = ap.parse_args()
    build(args.jobs, incremental=args.incremental)
