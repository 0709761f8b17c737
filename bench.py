#!/usr/bin/env python3
"""Benchmark of the ictc_o3 hot path on one MI355X.

Headline (``value``): channelwise CG tensor product forward + VJP (grads to
features, harmonics and gates), C=128, lmax=3 (23 paths), 131,072 instances,
fp32 -- BASELINE.json configs[1].  One "step" = one TP forward + one fused VJP
over the batch; inputs are resident in HBM before the timed region.

Also reported on the same JSON line:
* ``roofline`` of the dominant kernel (the fused VJP kernel): algorithmic bytes
  per launch / its mean duration from HIP events around each launch on the
  launch stream, against the 8 TB/s HBM3E peak;
* ``cpu_baseline``: the CPU oracle (a PyTorch restatement of the reference's CPU
  path, ``_forward_index_add`` + autograd) on a bounded sample on the host cores;
* ``extra``: forward-only throughput at 262,144 instances and its roofline.

``--kernels-only`` runs a 1 GiB device-to-device copy (the counter calibration
reference) and three launches of each TP kernel at the benchmark sizes, for
rocprofv3 --pmc passes.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--kernels-only]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ictc-o3-hp-ascend_amd"))

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0                       # MI355X HBM3E, GB/s
PUBLISHED_FWD_VJP_INST_S = 0.729e6          # reference HP on Ascend 910B3
C, L, ROWS_VJP, ROWS_FWD = 128, 3, 131072, 262144
P = 23
X_W, Y_W, G_W, O_W = C * (L + 1) ** 2, (L + 1) ** 2, P * C, 99 * C
BYTES_FWD = 4 * (X_W + Y_W + G_W + O_W)                   # 70,720 B/inst
BYTES_VJP = 4 * (O_W + 2 * (X_W + Y_W + G_W))             # 90,752 B/inst


def _harmonics(n: torch.Tensor) -> torch.Tensor:
    from ictc_o3.backends.hip.harmonics import direction_harmonics_packed
    return direction_harmonics_packed(n, L)


def _inputs(rows: int, device, seed: int = 0):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(rows, X_W, generator=gen)
    n = torch.nn.functional.normalize(torch.randn(rows, 3, generator=gen), dim=-1)
    g = torch.randn(rows, G_W, generator=gen) / math.sqrt(P)
    o = torch.randn(rows, O_W, generator=gen)
    x, n, g, o = (t.to(device) for t in (x, n, g, o))
    return x, _harmonics(n).contiguous(), g, o


def _time_gpu(args, plan, device):
    from ictc_o3.backends.hip.tensor_product import _backward_raw, _forward_raw
    x, y, g, o = _inputs(ROWS_VJP, device)
    need = (True, True, True)
    stream = torch.cuda.current_stream(device)

    def step(ev=None):
        out = _forward_raw(plan, x, y, g)
        if ev is not None:
            ev[0].record(stream)
        dx, dy, dg = _backward_raw(plan, need, x, y, g, o)
        if ev is not None:
            ev[1].record(stream)
        return out, dx, dy, dg

    t_end = time.time() + 2.0                 # reference protocol: >= 2 s warmup
    for _ in range(max(args.warmup, 1)):
        step()
    while time.time() < t_end:
        step()
    torch.cuda.synchronize(device)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)]
    torch.cuda.synchronize(device)
    t0 = time.perf_counter()
    for k in range(args.steps):
        step(events[k])
    torch.cuda.synchronize(device)
    elapsed = time.perf_counter() - t0
    vjp_ms = sum(a.elapsed_time(b) for a, b in events) / args.steps
    del x, y, g, o

    # forward-only at 262,144 instances
    x, y, g, _ = _inputs(ROWS_FWD, device, seed=1)
    for _ in range(3):
        _forward_raw(plan, x, y, g)
    torch.cuda.synchronize(device)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = max(args.steps, 5)
    s.record(stream)
    for _ in range(reps):
        _forward_raw(plan, x, y, g)
    e.record(stream)
    torch.cuda.synchronize(device)
    fwd_ms = s.elapsed_time(e) / reps
    return elapsed, vjp_ms, fwd_ms


def _copy_gbs(device, nbytes: int = 1 << 30, reps: int = 5) -> float:
    """Device-to-device copy bandwidth (read + write bytes / time)."""
    src = torch.empty(nbytes // 4, device=device)
    dst = torch.empty_like(src)
    src.fill_(1.0)
    dst.copy_(src)
    torch.cuda.synchronize(device)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        dst.copy_(src)
    e.record()
    torch.cuda.synchronize(device)
    return 2 * nbytes * reps / (s.elapsed_time(e) * 1e-3) / 1e9


def _kernels_only(plan, device) -> None:
    from ictc_o3.backends.hip.tensor_product import _backward_raw, _forward_raw
    src = torch.ones((1 << 30) // 4, device=device)
    torch.empty_like(src).copy_(src)          # calibration copy: 1 GiB read + 1 GiB written
    torch.cuda.synchronize(device)
    del src
    x, y, g, o = _inputs(ROWS_VJP, device)
    for _ in range(3):
        _forward_raw(plan, x, y, g)
        _backward_raw(plan, (True, True, True), x, y, g, o)
    torch.cuda.synchronize(device)
    print("kernels-only pass done", flush=True)


def _measured_traffic():
    """HBM bytes per VJP launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    (calibrated against a 1 GiB copy); None if the summary is absent."""
    path = os.path.join(ROOT, "profiles", "tp_c128_l3_hbm_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_vjp_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _cpu_baseline(budget_s: float = 12.0):
    """Oracle fwd+VJP (reference CPU path restated) on a bounded C128/L3 sample."""
    sys.path.insert(0, ROOT)
    from oracle import ictc_basis as B
    from oracle.tensor_product import TensorProductOracle
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    op = TensorProductOracle(C, L, L, L, dtype=torch.float32)
    rows = 2048
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(rows, X_W, generator=gen)
    n = torch.nn.functional.normalize(torch.randn(rows, 3, generator=gen, dtype=torch.float64), dim=-1)
    y = B.direction_harmonics_packed(n, L).float()
    g = torch.randn(rows, G_W, generator=gen) / math.sqrt(P)
    o = torch.randn(rows, O_W, generator=gen)

    def step():
        leaves = [t.clone().requires_grad_() for t in (x, y, g)]
        torch.autograd.grad(op.forward(*leaves), leaves, o)

    step()
    done, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        step()
        done += 1
    dt = time.perf_counter() - t0
    return {"value": rows * done / dt, "unit": "instances/s", "cores": threads, "kind": "port",
            "sample": f"oracle fwd+VJP (PyTorch CPU fp32, reference _forward_index_add + autograd), "
                      f"C128/lmax3, {rows} instances x {done} steps in {dt:.1f}s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kernels-only", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the hot "
              "path is embarrassingly parallel over instances and is not run multi-GPU here.",
              file=sys.stderr)
        return 2
    device = torch.device("cuda", 0)
    from ictc_o3 import EdgeTensorProduct
    op = EdgeTensorProduct.create(channels=C, input_lmax=L, edge_lmax=L, device=device)
    if args.kernels_only:
        _kernels_only(op.plan, device)
        return 0
    elapsed, vjp_ms, fwd_ms = _time_gpu(args, op.plan, device)
    copy_gbs = _copy_gbs(device)
    value = ROWS_VJP * args.steps / elapsed
    achieved = BYTES_VJP * ROWS_VJP / (vjp_ms * 1e-3) / 1e9
    fwd_achieved = BYTES_FWD * ROWS_FWD / (fwd_ms * 1e-3) / 1e9
    cpu = None if args.no_cpu else _cpu_baseline()
    line = {
        "metric": "TP instances/s fwd+VJP C128/lmax3; MACE E+F atom-steps/s; % HBM peak",
        "value": value, "unit": "instances/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": elapsed * 1e3 / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": value / PUBLISHED_FWD_VJP_INST_S, "dtype": "fp32",
        "data": "synthetic (seeded N(0,1) features, unit-sphere directions -> ICTC Y, N(0,1)/sqrt(P) gates)",
        "config": {"workload": "channelwise CG TP forward + VJP (grads x, Y, gates)", "channels": C,
                   "lmax": L, "paths": P, "instances": ROWS_VJP, "layout": "ir_mul"},
        "roofline": {"bound": "hbm", "kernel": "tp_backward_kernel<3,3,3,2>", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": _measured_traffic(), "traffic_unit": "bytes/launch",
                     "algorithmic_bytes_per_launch": BYTES_VJP * ROWS_VJP,
                     "mean_launch_ms": vjp_ms},
        "cpu_baseline": cpu,
        "extra": {"copy_gbs_measured": copy_gbs,
                  "vjp_frac_of_copy": achieved / copy_gbs,
                  "step_hbm_gbs": (BYTES_FWD + BYTES_VJP) * value / 1e9,
                  "step_hbm_frac": (BYTES_FWD + BYTES_VJP) * value / 1e9 / HBM_PEAK_GBS,
                  "forward_only": {"instances": ROWS_FWD, "instances_per_s": ROWS_FWD / (fwd_ms * 1e-3),
                                   "mean_launch_ms": fwd_ms, "achieved_gbs": fwd_achieved,
                                   "frac": fwd_achieved / HBM_PEAK_GBS,
                                   "vs_published_2.70M": ROWS_FWD / (fwd_ms * 1e-3) / 2.70e6}},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
