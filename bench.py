#!/usr/bin/env python3
"""Benchmark of the MI355X fmt=6 int4 decode hot path (libcoli_hip.so).

Workload: lm_head decode - a fmt=6 int4 GEMV with 248320
vocab rows x K=2048, gs=128, scales f16(|N(0,0.02)|) and zero points U{0..15} as f32,
x ~ N(0,1) fp32, followed by a device top-8 over the 248320 logits, fused into the same
launch.  One step = one such launch with all inputs resident in HBM; two weight copies
alternate so the 287 MB stream cannot be served from the 256 MB Infinity Cache.

Prints ONE JSON line (rank 0, N=1).  `value` is the achieved HBM bandwidth of the step
in GB/s from algorithmic bytes (nibbles + f32 [scale, zero] pairs + x + logits).
`roofline` prices the launch against the 8 TB/s HBM3E peak; `cpu_baseline` times the
reference's own CPU kernel (c/qwen.c:211-229, compiled from the reference checkout into
oracle/_ref) on this host over a bounded row sample.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "int4 GEMV/MoE achieved HBM GB/s (% of peak) and decode tok/s, 1 MI355X"
PEAK_GBS = 8000.0

O_VOCAB, K_HID, GS = 248320, 2048, 128


def alg_bytes_lmhead():
    ng = K_HID // GS
    return O_VOCAB * K_HID // 2 + O_VOCAB * ng * 8 + K_HID * 4 + O_VOCAB * 4


def load_product():
    import importlib.util
    spec = importlib.util.spec_from_file_location("qwen3_c_amd", os.path.join(ROOT, "qwen3.c_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def profile_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (committed summary), or None."""
    p = os.path.join(ROOT, "profiles", "gemv6_lmhead_traffic.json")
    try:
        with open(p) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline(budget_s=12.0):
    """Reference CPU kernel on a bounded sample of the same workload (rows of W)."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import _util

    ref_path = _util.REF_SO
    kind = "reference" if os.path.exists(ref_path) else "port"
    omp = os.environ.get("BENCH_CPU_OMP", "0") == "1"
    if kind == "reference":
        so = ref_path.replace("libqwenref.so", "libqwenref_omp.so") if omp else ref_path
        L = C.CDLL(so)
        fn = L.ref_matmul_q4g_asym
    else:
        L = C.CDLL(_util.ORACLE_OMP_SO if omp else _util.ORACLE_SO)
        fn = L.orc_matmul_q4g_asym
    fn.restype = None
    fn.argtypes = [C.c_void_p] * 4 + [C.c_int] * 3
    gen = _util.Gen(_util.load_oracle())
    rows = 16384
    q, sz = gen.fmt6(rows, K_HID, GS, 0xC1)
    x = gen.normal(K_HID, 7)
    y = np.empty(rows, np.float32)
    P = _util.P
    fn(P(y), P(x), P(q), P(sz), K_HID, rows, GS)   # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end and len(times) < 50:
        t0 = time.perf_counter()
        fn(P(y), P(x), P(q), P(sz), K_HID, rows, GS)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    sample_bytes = rows * K_HID // 2 + rows * (K_HID // GS) * 8 + K_HID * 4 + rows * 4
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)) if omp else 1
    return {"value": round(sample_bytes / med / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": kind,
            "sample": f"matmul_q4g_asym on {rows} of the 248320 lm_head rows (K=2048, gs=128), "
                      f"median of {len(times)} runs; full-op time {med * O_VOCAB / rows * 1e3:.1f} ms"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the fmt=6 GEMV/MoE path runs on a single "
              "MI355X; see DESIGN.md for how it would shard); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch  # plumbing: device buffers and event timing (imported before the library)

    mod = load_product()
    lib = mod.Lib().init()
    dev = torch.device("cuda:0")
    ext = torch.cuda.ExternalStream(lib.stream())

    seeds = [0xC1, 0xC2]
    w = [lib.tensor_synth(6, K_HID, O_VOCAB, GS, s, 0.02) for s in seeds]
    x = torch.empty(K_HID, dtype=torch.float32, device=dev)
    y = torch.empty(O_VOCAB, dtype=torch.float32, device=dev)
    idx = torch.empty(8, dtype=torch.int32, device=dev)
    val = torch.empty(8, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    lib.synth_normal_dev(x.data_ptr(), K_HID, 7, 1.0)
    lib.sync()

    def step(i):
        lib.gemv_topk_dev(w[i & 1], x.data_ptr(), y.data_ptr(), 8, idx.data_ptr(), val.data_ptr())

    for i in range(args.warmup):
        step(i)
    lib.sync()
    torch.cuda.synchronize()

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        ev[i][0].record(ext)
        step(i)
        ev[i][1].record(ext)
    lib.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = [a.elapsed_time(b) for a, b in ev]
    kern_ms.sort()
    avg_ms = sum(kern_ms) / len(kern_ms)
    bytes_per = alg_bytes_lmhead()
    achieved = bytes_per / (avg_ms * 1e-3) / 1e9
    ms_per_step = wall * 1e3 / args.steps

    out = {
        "metric": METRIC,
        "value": round(achieved, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x fp32 activations (exact int dot, fp32 scale/accumulate)",
        "data": "synthetic (device splitmix64 generator, seeded)",
        "config": {"workload": "cfg1: lm_head fmt6 GEMV 248320x2048 gs128 + fused device top-8",
                   "rows": O_VOCAB, "K": K_HID, "group_size": GS, "topk": 8, "weight_copies": 2},
        "us_per_op": round(avg_ms * 1e3, 2),
        "us_per_op_median": round(kern_ms[len(kern_ms) // 2] * 1e3, 2),
        "lmhead_tok_s": round(1e3 / avg_ms, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": profile_traffic(),
                     "alg_bytes_per_launch": bytes_per},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
