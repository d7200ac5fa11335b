#!/usr/bin/env python
"""Benchmark of the MTP speculative-decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode gemv|model]

Prints ONE JSON line.  Modes:
  gemv  : config 1 of the workload -- one batched IQ4_XS dequant-GEMV,
          17408 x 5120, B = 4 columns, seeded random super-blocks
          (d ~ fp16(|N(0,0.02)|), random 6-bit scales and nibbles), x ~ N(0,1).
          A step is one gemv_batch call (activation prep + GEMV kernel).
          Weights rotate over 12 copies (568 MB) so the 256 MB MALL cannot
          serve repeats.

Timing: HIP events recorded on the library stream around K back-to-back
steps (inputs resident in HBM).  roofline.achieved = algorithmic bytes per
launch / average GEMV kernel duration (events around K launches of the GEMV
kernel alone).  cpu_baseline: the reference engine's own AVX2 gemv_batch
(oracle/_ref, compiled from the reference sources) on the host cores, on a
bounded sample of the same workload.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
IQ4 = 23
METRIC = "accepted tok/s, 27B IQ4_XS MTP k=3 on 1 GPU; gemv_batch HBM GB/s (% peak)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_for(kernel):
    """HBM bytes per launch measured with rocprofv3 PMC counters (profiles/traffic.json)."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f).get(kernel, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline_gemv(W, x, ne0, ne1, n, seconds=10.0):
    """Reference AVX2 gemv_batch (kernels.c:640) with its own thread pool, pinned."""
    ref = os.path.join(ROOT, "oracle", "_ref", "libqwenref.so")
    if not os.path.exists(ref):
        return None
    L = ctypes.CDLL(ref)

    class TI(ctypes.Structure):
        _fields_ = [("name", ctypes.c_char * 64), ("n_dims", ctypes.c_uint32), ("ne", ctypes.c_uint64 * 4),
                    ("type", ctypes.c_int), ("offset", ctypes.c_uint64), ("data", ctypes.c_void_p)]

    F = ctypes.POINTER(ctypes.c_float)
    L.pool_create.restype = ctypes.c_void_p
    L.pool_create.argtypes = [ctypes.c_int, ctypes.c_int]
    L.pool_destroy.argtypes = [ctypes.c_void_p]
    L.gemv_batch.argtypes = [ctypes.c_void_p, ctypes.POINTER(TI), F, ctypes.c_uint64, ctypes.c_int, F,
                             ctypes.c_uint64]
    cores = len(os.sched_getaffinity(0))
    pool = L.pool_create(cores, 1)
    copies = [W.copy() for _ in range(4)]            # 190 MB: larger than the host L3
    tis = []
    for c in copies:
        t = TI(name=b"W", n_dims=2, type=IQ4, offset=0, data=c.ctypes.data_as(ctypes.c_void_p))
        t.ne[0], t.ne[1], t.ne[2], t.ne[3] = ne0, ne1, 1, 1
        tis.append(t)
    out = np.zeros((n, ne1), np.float32)
    xp, op = x.ctypes.data_as(F), out.ctypes.data_as(F)
    L.gemv_batch(pool, ctypes.byref(tis[0]), xp, ne0, n, op, ne1)   # warm-up
    calls, t0 = 0, time.perf_counter()
    while True:
        L.gemv_batch(pool, ctypes.byref(tis[calls % 4]), xp, ne0, n, op, ne1)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    L.pool_destroy(pool)
    return calls, el, cores


def bench_gemv(args):
    from qwen_pkg import host_lib, pyqwen
    host, gpu = host_lib(), pyqwen.gpu_lib()
    ne0, ne1, B = 5120, 17408, 4
    W = host.synth_matrix(IQ4, ne0, ne1, 1, 0, 0.02)
    x = host.synth_normal(B * ne0, 1, 1).reshape(B, ne0)
    R = 12
    Ts = [gpu.tensor(W, IQ4, ne0, ne1) for _ in range(R)]
    xb, ob = gpu.put(x), gpu.buf(B * ne1 * 4)
    algo = W.nbytes + B * (ne0 + ne1) * 4
    L = gpu.L

    def step(i):
        gpu.ok(L.qgpu_gemv_batch(Ts[i % R].h, xb.f32(), ne0, B, ob.f32(), ne1, 0))

    for i in range(args.warmup):
        step(i)
    gpu.sync()
    e0, e1 = gpu.event(), gpu.event()
    gpu.record(e0)
    for i in range(args.steps):
        step(i)
    gpu.record(e1)
    ms_total = gpu.elapsed_ms(e0, e1)
    ms_step = ms_total / args.steps
    # GEMV kernel alone: activations prepared once, K launches of the GEMV kernel
    gpu.ok(L.qgpu_gemv_prepare(xb.f32(), ne0, B, ne0))
    for i in range(args.warmup):
        gpu.ok(L.qgpu_gemv_prepared(Ts[i % R].h, B, ob.f32(), ne1, 0))
    gpu.record(e0)
    for i in range(args.steps):
        gpu.ok(L.qgpu_gemv_prepared(Ts[i % R].h, B, ob.f32(), ne1, 0))
    gpu.record(e1)
    ms_kernel = gpu.elapsed_ms(e0, e1) / args.steps
    gpu.sync()
    achieved = algo / (ms_kernel * 1e-3) / 1e9
    value = algo / (ms_step * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        r = cpu_baseline_gemv(W, x, ne0, ne1, B, args.cpu_seconds)
        if r:
            calls, el, cores = r
            cpu = {"value": round(algo * calls / el / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "reference",
                   "sample": f"{calls} calls of the reference gemv_batch (IQ4_XS 17408x5120, B=4) over {el:.1f} s, "
                             f"4 rotating weight copies, pool of {cores} pinned threads"}
    name, ncu, _ = gpu.device_info()
    return {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "iq4_xs x fp32 (int8 MFMA, exact int32 sub-block sums, fp32 accumulate)",
        "data": "synthetic (seeded random IQ4_XS super-blocks, x ~ N(0,1))",
        "config": {"workload": "gemv_batch IQ4_XS 17408x5120, B=4 (1 token + 3 drafts)", "rows": ne1, "cols": ne0,
                   "B": B, "weight_copies": R, "device": name, "cus": ncu},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_for("k_gemv_iq4"),
                     "kernel": "k_gemv_iq4<1,4>", "kernel_ms": round(ms_kernel, 5), "algo_bytes": algo},
        "cpu_baseline": cpu,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=["gemv"], default="gemv")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run the k_copy kernel on 256 MiB x 5 (reference point for PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.copy_calib:
        from qwen_pkg import pyqwen
        gpu = pyqwen.gpu_lib()
        nb = 256 << 20
        a, b = gpu.buf(nb), gpu.buf(nb)
        gpu.ok(gpu.L.qgpu_memset(ctypes.c_void_p(a.ptr), 1, nb))
        for _ in range(5):
            gpu.ok(gpu.L.qgpu_copy(ctypes.c_void_p(b.ptr), ctypes.c_void_p(a.ptr), nb))
        gpu.sync()
    res = bench_gemv(args)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
