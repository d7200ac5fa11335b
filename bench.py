#!/usr/bin/env python
"""Benchmark of the MTP speculative-decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--mode model|gemv|longctx|sweep|sample]

Prints ONE JSON line on stdout (progress goes to stderr).

mode model (default) -- the headline workload: the random-init 27B hybrid
    (64 layers: 48 Gated-DeltaNet + 16 gated-GQA, hidden 5120, FFN 17408,
    vocab 248320, all matrices IQ4_XS, plus the MTP draft layer), greedy MTP
    speculative decode with k = 3 drafts after a 512-token seeded random-id
    prompt.  A step is one speculative cycle (k MTP drafts, one batched verify
    of k+1 tokens, on-device argmax/acceptance, state-ring rollback, MTP
    re-anchor); K = 256 cycles are timed.  value = tokens emitted per second.
    Random-init weights make the MTP drafts disagree with the backbone, so
    about one token is accepted per cycle; the same loop with every draft
    accepted (forced_accept_tok_s) and the verify/decode/draft step times are
    reported beside it.
mode gemv -- one batched IQ4_XS dequant-GEMV, 17408 x 5120, B = 4 columns.
mode longctx -- the same model after an 8192-token prompt; verify-step
    latency and forced-acceptance throughput for k in {1, 3, 5, 7}.
mode sweep -- gemv_batch over every weight format of the path (IQ4_XS, Q4_K,
    Q5_K, Q6_K, Q8_0) x shapes 5120->17408, 17408->5120, 5120->248320 x B in
    {1, 2, 4, 8}; HBM GB/s of algorithmic bytes per call (weights rotate over
    enough copies to exceed the 256 MB MALL).  value = the IQ4_XS 17408x5120
    B=4 point.
mode sample -- the non-speculative sampled decode (main.c:232-248) on the same
    27B model after a 512-token prompt: every token drawn on the device by the
    reference sampler (temp 0.8, top-p 0.9, top-k 40, repeat penalty 1.1 over
    the last 64 tokens), then one model_forward step; K = 128 tokens timed.
    value = sampled tokens per second; the greedy decode of the same length,
    and the sampler kernels alone at the 248,320-token vocabulary (graph
    replays), are reported beside it.

roofline (every mode): the dominant kernel, k_gemv_mfma (IQ4_XS), on the gemv workload
(17408 x 5120 IQ4_XS, B = 4), run first in the process: W + K gemv_batch calls,
then the GEMV kernel alone on prepared activations.  Each timed series of K
calls is captured in a HIP graph, replayed once untimed and once bracketed by
HIP events on the library stream (the replay issues the K kernels back to back,
so the host loop's per-call cost does not enter the kernel time).  achieved =
algorithmic bytes per launch (47,349,760 weight + 4 x (5120 + 17408) x 4
activation/output = 47,710,208 B) / average launch duration.  Weights rotate over 12 copies
(568 MB) so the 256 MB MALL cannot serve repeats.  read_floor_us: the same
47,349,760 weight bytes of each copy read by a plain XOR-reduction kernel
(qgpu_tensor_checksum, 8192 blocks x 256 threads, 4 x 16 B loads in flight per
thread, one 4-byte store per block), timed the same way: the read bandwidth a
kernel of this size reaches.

cpu_baseline: the reference engine itself (oracle/_ref, compiled from the
reference sources; AVX2, its own pinned thread pool) on the host cores:
model mode runs the reference's speculative cycle on the same 27B model file
after the same 512-token prompt (its batched prefill, then a bounded sample of
cycles); gemv mode runs its gemv_batch; sample mode runs its sampled decode
loop (sampler_sample + model_forward) after the same prompt.
"""
import argparse
import ctypes
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
IQ4 = 23
METRIC = "accepted tok/s, 27B IQ4_XS MTP k=3 on 1 GPU; gemv_batch HBM GB/s (% peak)"
ROOF_TILES = 17408 // 16   # 16-row tiles of the roofline GEMV
MIX_NOTE = "the real checkpoint's format mix: token_embd Q4_K, attn_qkv Q5_K, output Q6_K, nextn.eh_proj Q8_0, the rest IQ4_XS"


def roof_kernel(ncu):
    """the kernel instance the roofline GEMV launches on a device of ncu compute units: IQ4_XS, one
    digit plane; when its tiles are a little over a multiple of the compute units (1088 = 4 x 256 + 64
    on MI355X) mode 20 (pair split 4, no prefetch rings 16) with 8 waves per tile (at most 1100 tiles),
    else mode 0 with 4"""
    r = ROOF_TILES % ncu if ncu else 0
    pair = bool(ncu) and ROOF_TILES > ncu and 0 < r <= ncu // 2 and r <= 256
    noring = pair and ROOF_TILES <= 12 * ncu
    nw = 8 if ROOF_TILES <= (1100 if noring else 512) else 4
    return f"k_gemv_mfma<23, 1, {nw}, {20 if noring else (4 if pair else 0)}>"
READ_BLOCKS = 8192      # plain-read floor launch: 8192 blocks x 256 threads (best of 1024..8192 at 47.7 MB)


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def traffic_for(kernel):
    """HBM bytes per launch measured with rocprofv3 PMC counters (profiles/traffic.json), when they were
    measured on this kernel instance"""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as f:
            d = json.load(f).get(kernel.split("<")[0], {})
    except (OSError, ValueError):
        return None
    return d.get("bytes_per_launch") if d.get("kernel") == kernel else None


def host_info():
    """The host as lscpu reports it, and the threads the CPU baselines use: the physical cores
    of one NUMA node, capped by the CPUs this process may run on."""
    info = {"affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = dict((k.strip(), v.strip()) for k, v in (ln.split(":", 1) for ln in out.splitlines() if ":" in ln))
        info.update({"model": kv.get("Model name"), "sockets": int(kv.get("Socket(s)", 1)),
                     "cores_per_socket": int(kv.get("Core(s) per socket", 0)),
                     "threads_per_core": int(kv.get("Thread(s) per core", 1)),
                     "numa_nodes": int(kv.get("NUMA node(s)", 1))})
        node_cores = info["sockets"] * info["cores_per_socket"] // max(1, info["numa_nodes"])
        info["threads_used"] = max(1, min(info["affinity_cpus"], node_cores or info["affinity_cpus"]))
    except (OSError, ValueError, subprocess.SubprocessError):
        info["threads_used"] = info["affinity_cpus"]
    return info


def host_cores():
    return host_info()["threads_used"]


# ---------------------------------------------------------------------------------- CPU baselines
def cpu_baseline_gemv(W, x, ne0, ne1, n, seconds):
    """Reference AVX2 gemv_batch (kernels.c:640) with its own pinned thread pool."""
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
    cores = host_cores()
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
    algo = W.nbytes + n * (ne0 + ne1) * 4
    return {"value": round(algo * calls / el / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "reference",
            "sample": f"{calls} calls of the reference gemv_batch (IQ4_XS 17408x5120, B=4) over {el:.1f} s, "
                      f"4 rotating weight copies, pool of {cores} pinned threads", "host": host_info()}


def cpu_baseline_spec(path, prompt, k, seconds, gpu_prompt, kv_note):
    """The reference's greedy MTP speculative cycle (main.c:158-231) on the same model file."""
    drv = os.path.join(ROOT, "oracle", "_ref", "librefbench.so")
    if not os.path.exists(drv):
        return None
    L = ctypes.CDLL(drv)
    U = ctypes.POINTER(ctypes.c_uint32)
    L.ref_spec_bench.argtypes = [ctypes.c_char_p, ctypes.c_uint32, U, ctypes.c_uint32, ctypes.c_uint32,
                                 ctypes.c_uint32, ctypes.c_uint32, ctypes.c_double, ctypes.c_int,
                                 ctypes.POINTER(ctypes.c_double)]
    p = np.ascontiguousarray(prompt, np.uint32)
    out = (ctypes.c_double * 5)()
    cores = host_cores()
    n_ctx = len(p) + 1024                   # the loop stops before a cycle would pass n_ctx
    rc = L.ref_spec_bench(path.encode(), n_ctx, p.ctypes.data_as(U), len(p), k, 1, 1000, seconds, cores, out)
    if rc == -1 or out[3] < 1:
        return None
    tps = out[2] / out[1]
    return {"value": round(tps, 4), "unit": "tok/s", "cores": cores, "kind": "reference",
            "sample": f"reference engine, same 27B model file, {len(p)}-token prompt (prefill {out[0]:.1f} s), "
                      f"then {int(out[3])} greedy speculative cycles with k={k} over {out[1]:.1f} s "
                      f"({int(out[2])} tokens, {int(out[4])} drafts accepted), pool of {cores} pinned threads"
                      + ("; stopped early: a cycle accepted 2 drafts, which the reference cannot roll back"
                         if rc == -2 else ""),
            "prompt_as_gpu_run": len(p) == gpu_prompt,
            **({} if len(p) == gpu_prompt else {
                "differs_from_gpu_run": f"prompt of {len(p)} tokens, not {gpu_prompt}: the cycles' attention spans "
                                        f"{len(p)}+ instead of {gpu_prompt}+ positions ({kv_note})"}),
            "host": host_info()}


def cpu_baseline_sample(path, prompt, cfg, seconds, gpu_prompt):
    """The reference's sampled decode (main.c:232-248) on the same model file."""
    drv = os.path.join(ROOT, "oracle", "_ref", "librefbench.so")
    if not os.path.exists(drv):
        return None
    L = ctypes.CDLL(drv)
    U = ctypes.POINTER(ctypes.c_uint32)
    f32, u32 = ctypes.c_float, ctypes.c_uint32
    L.ref_sample_bench.argtypes = [ctypes.c_char_p, u32, U, u32, f32, f32, u32, f32, ctypes.c_uint64, u32,
                                   ctypes.c_double, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    p = np.ascontiguousarray(prompt, np.uint32)
    out = (ctypes.c_double * 5)()
    cores = host_cores()
    temp, top_p, top_k, pen, seed = cfg
    if L.ref_sample_bench(path.encode(), len(p) + 1024, p.ctypes.data_as(U), len(p), temp, top_p, top_k, pen, seed,
                          1000, seconds, cores, out) or out[2] < 1:
        return None
    return {"value": round(out[2] / out[1], 4), "unit": "tok/s", "cores": cores, "kind": "reference",
            "sample": f"reference engine, same 27B model file, {len(p)}-token prompt (prefill {out[0]:.1f} s), "
                      f"then {int(out[2])} sampled tokens over {out[1]:.1f} s; sampler_sample "
                      f"{1e6 * out[3] / out[4]:.0f} us per call; pool of {cores} pinned threads",
            "prompt_as_gpu_run": len(p) == gpu_prompt,
            "host": host_info()}


# ---------------------------------------------------------------------------------- roofline microbench
ROOF_UNTIMED, ROOF_TIMED = 2, 5     # graph replays of the roofline series: untimed, then timed


def graph_ms(gpu, calls, e0, e1, timed=1, untimed=1):
    """Captures the stream work of calls() in a HIP graph, replays it `untimed` times, then
    `timed` times each between HIP events; returns the timed replays' milliseconds.  A replay
    issues the captured kernels back to back, so the host's per-call cost is not in the figure."""
    L = gpu.L
    gpu.sync()
    gpu.ok(L.qgpu_graph_begin())
    calls()
    gexec = ctypes.c_void_p()
    gpu.ok(L.qgpu_graph_end(ctypes.byref(gexec)))
    for _ in range(untimed):
        gpu.ok(L.qgpu_graph_launch(gexec))
    out = []
    for _ in range(timed):
        gpu.record(e0)
        gpu.ok(L.qgpu_graph_launch(gexec))
        gpu.record(e1)
        gpu.sync()
        out.append(gpu.elapsed_ms(e0, e1))
    gpu.ok(L.qgpu_graph_destroy(gexec))
    return out if timed > 1 else out[0]


def gemv_roofline(gpu, host, steps, warmup):
    """config-1 GEMV: gemv_batch calls, then the GEMV kernel alone (roofline)."""
    ne0, ne1, B = 5120, 17408, 4
    rk = roof_kernel(gpu.device_info()[1])
    W = host.synth_matrix(IQ4, ne0, ne1, 1, 0, 0.02)
    x = host.synth_normal(B * ne0, 1, 1).reshape(B, ne0)
    R = 12
    Ts = [gpu.tensor(W, IQ4, ne0, ne1) for _ in range(R)]
    xb, ob = gpu.put(x), gpu.buf(B * ne1 * 4)
    algo = W.nbytes + B * (ne0 + ne1) * 4
    L = gpu.L
    e0, e1 = gpu.event(), gpu.event()
    # gemv_batch calls (activation prep + GEMV kernel), the library entry point
    for i in range(warmup):
        gpu.ok(L.qgpu_gemv_batch(Ts[i % R].h, xb.f32(), ne0, B, ob.f32(), ne1, 0))

    def batch_calls():
        for i in range(steps):
            gpu.ok(L.qgpu_gemv_batch(Ts[i % R].h, xb.f32(), ne0, B, ob.f32(), ne1, 0))
    ms_call = graph_ms(gpu, batch_calls, e0, e1) / steps
    # the GEMV kernel alone: activations prepared once
    gpu.ok(L.qgpu_gemv_prepare(xb.f32(), ne0, B, ne0))

    def kernel_calls():
        for i in range(steps):
            gpu.ok(L.qgpu_gemv_prepared(Ts[i % R].h, B, ob.f32(), ne1, 0))
    # several timed replays: the launch time moves by several percent between replays (clocks), so
    # the line reports the median replay and the range
    reps = [ms / steps for ms in graph_ms(gpu, kernel_calls, e0, e1, ROOF_TIMED, ROOF_UNTIMED)]
    med = sorted(range(ROOF_TIMED), key=lambda i: reps[i])[ROOF_TIMED // 2]
    ms_kernel = reps[med]
    # plain-read floor over the same device bytes: k_checksum over each rotating copy's records
    dev_bytes = int(L.qgpu_tensor_device_bytes(Ts[0].h))
    cs = gpu.buf(READ_BLOCKS * 4)

    def read_calls():
        for i in range(steps):
            gpu.ok(L.qgpu_tensor_checksum(Ts[i % R].h, cs.u32(), READ_BLOCKS))
    ms_read = sorted(ms / steps for ms in graph_ms(gpu, read_calls, e0, e1, ROOF_TIMED, ROOF_UNTIMED))[ROOF_TIMED // 2]
    for T in Ts:
        T.close()
    achieved = algo / (ms_kernel * 1e-3) / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_for(rk),
            "kernel": rk, "workload": "IQ4_XS 17408x5120, B=4", "kernel_us": round(ms_kernel * 1e3, 3),
            "kernel_us_range": [round(min(reps) * 1e3, 3), round(max(reps) * 1e3, 3)],
            "algo_bytes": algo,
            # the same weight bytes read by a plain XOR-reduction kernel (k_checksum), same rotation
            "read_floor_us": round(ms_read * 1e3, 3), "read_floor_gbs": round(dev_bytes / (ms_read * 1e-3) / 1e9, 1),
            "kernel_over_read_floor": round(ms_kernel / ms_read, 3),
            # dispatch ordinals of this kernel (0-based, in launch order) that the events of the
            # median replay bracket: warm-up calls, the gemv_batch series (2 replays), the untimed
            # replays, then the timed ones
            "dispatches": {"first": warmup + (2 + ROOF_UNTIMED + med) * steps, "count": steps}}
    gemv_call_gbs = algo / (ms_call * 1e-3) / 1e9
    return roof, gemv_call_gbs, ms_call, (W, x, ne0, ne1, B)


SWEEP_FORMATS = [("IQ4_XS", 23), ("Q4_K", 12), ("Q5_K", 13), ("Q6_K", 14), ("Q8_0", 8)]
SWEEP_SHAPES = [(5120, 17408), (17408, 5120), (5120, 248320)]     # (columns ne0, rows ne1)


def bench_sweep(gpu, host, steps, warmup):
    """gemv_batch GB/s over formats x shapes x B (algorithmic bytes: weights + B x (in + out) x 4)."""
    L = gpu.L
    e0, e1 = gpu.event(), gpu.event()
    rows = []
    for fname, t in SWEEP_FORMATS:
        for ne0, ne1 in SWEEP_SHAPES:
            W = host.synth_matrix(t, ne0, ne1, 7, t, 0.02)
            R = max(2, -(-(600 << 20) // W.nbytes))
            Ts = [gpu.tensor(W, t, ne0, ne1) for _ in range(R)]
            x = host.synth_normal(8 * ne0, 1, 3).reshape(8, ne0)
            xb, ob = gpu.put(x), gpu.buf(8 * ne1 * 4)

            def first_calls():
                for i in range(steps):
                    gpu.ok(L.qgpu_gemv_batch(Ts[i % R].h, xb.f32(), ne0, 1, ob.f32(), ne1, 0))
            # one discarded graph replay per shape: the first one after the copies are made ran
            # 10-15% slow (lm_head B = 1: 139 against 122 us measured again)
            graph_ms(gpu, first_calls, e0, e1)
            for B in (1, 2, 4, 8):
                for i in range(warmup):
                    gpu.ok(L.qgpu_gemv_batch(Ts[i % R].h, xb.f32(), ne0, B, ob.f32(), ne1, 0))

                def calls():
                    for i in range(steps):
                        gpu.ok(L.qgpu_gemv_batch(Ts[i % R].h, xb.f32(), ne0, B, ob.f32(), ne1, 0))
                us = graph_ms(gpu, calls, e0, e1) / steps * 1e3
                algo = W.nbytes + B * (ne0 + ne1) * 4
                rows.append({"format": fname, "rows": ne1, "cols": ne0, "B": B, "us": round(us, 2),
                             "gbs": round(algo / us / 1e3, 1), "frac": round(algo / us / 1e3 / HBM_PEAK_GBS, 4),
                             "weight_bytes": W.nbytes})
                log(f"sweep {fname:6s} {ne1:6d}x{ne0:<5d} B={B}: {us:8.2f} us {algo / us / 1e3:7.1f} GB/s")
            gpu.sync()
            for T in Ts:
                T.close()
            xb.close()
            ob.close()
            del W
    return rows


# ---------------------------------------------------------------------------------- model workloads
def spec_27b(host, seed, weights="iq4"):
    """the seeded 27B hybrid: every 2-D weight IQ4_XS, or (weights "mix") the real checkpoint's
    format mix: token_embd Q4_K, attn_qkv Q5_K, output Q6_K, nextn.eh_proj Q8_0, the rest IQ4_XS"""
    return host.spec_27b_mix(seed) if weights == "mix" else host.spec_27b(seed)


def model_file(host, seed, keep_dir=None, weights="iq4"):
    """Writes the seeded random-init 27B model as a GGUF file (tmpfs when it fits)."""
    spec = spec_27b(host, seed, weights)
    need = sum(t.nbytes for t in host.tensors(spec)) + (64 << 20)
    for d in ([keep_dir] if keep_dir else []) + ["/dev/shm", tempfile.gettempdir()]:
        try:
            if shutil.disk_usage(d).free > need + (2 << 30):
                path = os.path.join(d, f"qwen27b_synth_{seed}_{os.getpid()}.gguf")
                t = time.time()
                host.write_gguf(spec, path)
                log(f"model file {path}: {os.path.getsize(path) / 1e9:.2f} GB written in {time.time() - t:.1f} s")
                return path, spec
        except OSError:
            continue
    return None, spec


def step_bytes(host, spec, B, pos):
    """Algorithmic HBM bytes of one verify (B tokens) step and of one MTP draft."""
    ts = host.tensors(spec)
    mtp_layer = f"blk.{spec.n_layer}."
    w_backbone = sum(t.nbytes for t in ts if t.n_dims == 2 and not t.name.startswith(b"token_embd")
                     and not t.name.decode().startswith(mtp_layer))
    out_w = next(t.nbytes for t in ts if t.name == b"output.weight")
    w_mtp = sum(t.nbytes for t in ts if t.n_dims == 2 and t.name.decode().startswith(mtp_layer)) + out_w
    n_attn = spec.n_layer // spec.full_attn_interval
    n_gdn = spec.n_layer - n_attn
    state = spec.n_v_heads * spec.state * spec.state * 4
    gdn = n_gdn * (state * (1 + B))                       # read current state, write B snapshots
    kv = n_attn * (pos + B) * 2 * spec.n_kv_head * spec.head_dim * 4
    return w_backbone + gdn + kv, w_mtp + (pos + 1) * 2 * spec.n_kv_head * spec.head_dim * 4


def bench_model(args, gpu, host, roof, gemv_call_gbs):
    from qwen_pkg import pyqwen
    k, n_prompt = args.k, args.prompt
    K, W, F = args.steps, args.warmup, args.forced_cycles
    path = None
    if not args.no_cpu:
        path, spec = model_file(host, args.seed, weights=args.weights)
    else:
        spec = spec_27b(host, args.seed, args.weights)
    n_ctx = ((n_prompt + (k + 1) * (W + K + F) + 64 + 255) // 256) * 256
    t = time.time()
    m = pyqwen.Model(path, n_ctx) if path else pyqwen.Model(spec=spec, n_ctx=n_ctx)
    log(f"model on the GPU in {time.time() - t:.1f} s (n_ctx {n_ctx})")
    V = m.V
    prompt = np.random.default_rng(args.seed + 512).integers(0, V, n_prompt).astype(np.uint32)
    t = time.time()
    m.spec_begin(prompt, k)
    t_prefill = time.time() - t
    log(f"prefill {n_prompt} tokens: {t_prefill:.2f} s")
    m.spec_run(k, W)                                         # warm-up cycles
    gpu.sync()
    toks, js, st = m.spec_run(k, K)                          # timed: exactly K cycles
    gpu.sync()
    t_dec = st.t_decode_s
    log(f"{K} cycles: {len(toks)} tokens in {t_dec:.3f} s, {st.n_accepted}/{st.n_drafts} drafts accepted")
    ftoks, fjs, fst = m.spec_run(k, F, force_accept=1)       # every draft accepted
    log(f"forced acceptance: {F} cycles, {len(ftoks)} tokens in {fst.t_decode_s:.3f} s")
    ms_verify, ms_decode, ms_draft = m.time_steps(k + 1, 20)
    pos = m.pos
    vbytes, dbytes = step_bytes(host, spec, k + 1, pos)
    dec_bytes, _ = step_bytes(host, spec, 1, pos)
    m.close()
    cpu = None
    if path:
        try:
            log("CPU baseline: reference speculative loop on the host cores")
            kv = 2 * spec.n_kv_head * spec.head_dim * 4 * (spec.n_layer // spec.full_attn_interval)
            kv_note = (f"the KV bytes a cycle reads at {n_prompt} positions are {kv * n_prompt / 1e6:.0f} MB, "
                       f"{100 * kv * n_prompt / vbytes:.2f}% of the verify step's {vbytes / 1e9:.2f} GB")
            cpu = cpu_baseline_spec(path, prompt, k, args.cpu_seconds, n_prompt, kv_note)
        finally:
            os.remove(path)
    value = len(toks) / t_dec
    return {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(t_dec / K * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32 (IQ4_XS weights; int8-MFMA digit GEMV, fp32 accumulate)",
        "data": "synthetic: seeded random-init 27B hybrid (" + (MIX_NOTE if args.weights == "mix" else "IQ4_XS")
                + "), seeded random-id prompt",
        "config": {"workload": f"27B hybrid greedy MTP speculative decode, k={k}, {n_prompt}-token prompt, "
                               f"{K} cycles", "k": k, "prompt_tokens": n_prompt, "n_ctx": n_ctx,
                   "weights": MIX_NOTE if args.weights == "mix" else "every 2-D weight IQ4_XS",
                   "layers": "48 GDN + 16 GQA + MTP", "device": gpu.device_info()[0]},
        "tokens": int(len(toks)), "drafts_accepted": int(st.n_accepted), "drafts": int(st.n_drafts),
        # accepted drafts per timed cycle: j_hist[j] = cycles that accepted j of the k drafts
        "j_hist": [int(c) for c in np.bincount(np.asarray(js, np.int64), minlength=k + 1)[:k + 1]],
        "forced_accept_tok_s": round(len(ftoks) / fst.t_decode_s, 2),
        "verify_ms": round(ms_verify, 4), "decode_ms": round(ms_decode, 4), "draft_ms": round(ms_draft, 4),
        "verify_over_decode": round(ms_verify / ms_decode, 4),
        "verify_hbm_gbs": round(vbytes / (ms_verify * 1e-3) / 1e9, 1),
        "decode_hbm_gbs": round(dec_bytes / (ms_decode * 1e-3) / 1e9, 1),
        "draft_hbm_gbs": round(dbytes / (ms_draft * 1e-3) / 1e9, 1),
        "prefill_s": round(t_prefill, 3),
        "gemv_batch_gbs": round(gemv_call_gbs, 1), "gemv_batch_frac": round(gemv_call_gbs / HBM_PEAK_GBS, 4),
        "roofline": roof, "cpu_baseline": cpu,
    }


def bench_longctx(args, gpu, host, roof, gemv_call_gbs):
    from qwen_pkg import pyqwen
    spec = host.spec_27b(args.seed)
    n_prompt, F = args.prompt, args.forced_cycles
    ks = [1, 3, 5, 7]
    n_ctx = ((n_prompt + sum((kk + 1) * (F + 1) for kk in ks) + 64 + 255) // 256) * 256
    m = pyqwen.Model(spec=spec, n_ctx=n_ctx)
    prompt = np.random.default_rng(args.seed + 8192).integers(0, m.V, n_prompt).astype(np.uint32)
    t = time.time()
    m.spec_begin(prompt, 7)
    t_prefill = time.time() - t
    log(f"prefill {n_prompt} tokens: {t_prefill:.2f} s")
    rows, tot_t = {}, 0.0
    for kk in ks:
        ms_verify, ms_decode, ms_draft = m.time_steps(kk + 1, 10)
        m.spec_run(kk, 1, force_accept=1)
        toks, js, st = m.spec_run(kk, F, force_accept=1)
        rows[f"k{kk}"] = {"verify_ms": round(ms_verify, 4), "decode_ms": round(ms_decode, 4),
                          "draft_ms": round(ms_draft, 4), "verify_over_decode": round(ms_verify / ms_decode, 4),
                          "forced_accept_tok_s": round(len(toks) / st.t_decode_s, 2), "pos": m.pos}
        tot_t += st.t_decode_s
        log(f"k={kk}: {rows[f'k{kk}']}")
    m.close()
    K = F * len(ks)
    return {
        "metric": METRIC, "value": rows["k3"]["forced_accept_tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": len(ks), "ms_per_step": round(tot_t / K * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32 (IQ4_XS weights; int8-MFMA digit GEMV, fp32 accumulate)",
        "data": "synthetic: seeded random-init 27B hybrid (IQ4_XS), seeded random-id prompt",
        "config": {"workload": f"27B hybrid, {n_prompt}-token prompt, forced-acceptance k sweep {ks}",
                   "prompt_tokens": n_prompt, "n_ctx": n_ctx, "cycles_per_k": F},
        "per_k": rows, "prefill_s": round(t_prefill, 3),
        "gemv_batch_gbs": round(gemv_call_gbs, 1), "roofline": roof, "cpu_baseline": None,
    }


SAMPLE_CFG = (0.8, 0.9, 40, 1.1, 7)        # temp, top_p, top_k, repeat penalty, seed


ATTN_CASES = [(800, 1), (800, 4), (800, 8), (8392, 4), (8392, 6), (8392, 8)]     # (KV positions before the call, B)


def bench_attn(args, gpu):
    """The model's attention call alone at the 27B shapes (24 query / 4 KV heads, head_dim 256, RoPE on 64
    dims): qgpu_attn_fused_act (span kernel + combine with the o-projection digits) at several context
    lengths and batch sizes, random caches, with the live-context bound the model passes
    (qgpu_attn_fused_act_live); per case K calls captured in a HIP graph, the median of five
    timed replays (--eager: K calls launched from the host, five timed series).  Bytes per call: the K and
    V rows of every position plus q, k, v in and out."""
    L = gpu.L
    nh, nkv, hd, rope_dim, eps, n_ctx = 24, 4, 256, 64, 1e-6, 8448
    rng = np.random.default_rng(args.seed)
    kc = gpu.put(rng.standard_normal((n_ctx, nkv, hd)).astype(np.float32))
    vc = gpu.put(rng.standard_normal((n_ctx, nkv, hd)).astype(np.float32))
    half = rope_dim // 2
    ang = np.arange(n_ctx, dtype=np.float32)[:, None] * \
        np.power(np.float32(1e7), (-2.0 * np.arange(half) / rope_dim).astype(np.float32))[None]
    rc, rs = gpu.put(np.cos(ang).astype(np.float32)), gpu.put(np.sin(ang).astype(np.float32))
    qw = gpu.put((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    kw = gpu.put((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    e0, e1 = gpu.event(), gpu.event()
    rows = []
    for pos, B in ATTN_CASES:
        q = gpu.put(rng.standard_normal((B, nh * 2 * hd)).astype(np.float32))
        k = gpu.put(rng.standard_normal((B, nkv * hd)).astype(np.float32))
        v = gpu.put(rng.standard_normal((B, nkv * hd)).astype(np.float32))
        out, posb = gpu.buf(B * nh * hd * 4), gpu.put(np.array([pos], np.int32))
        # the live-context bound the model gives this call (the head split while the context allows)
        bound = L.qgpu_attn_split_bound(n_ctx, B, nh, nkv)
        live = bound if pos + B <= bound else 0

        def calls():
            for _ in range(args.steps):
                gpu.ok(L.qgpu_attn_fused_act_live(q.f32(), nh * 2 * hd, k.f32(), v.f32(), nkv * hd, qw.f32(),
                                                  kw.f32(), kc.f32(), vc.f32(), rc.f32(), rs.f32(), rope_dim,
                                                  posb.i32(), n_ctx, B, nh, nkv, hd, eps, out.f32(), nh * hd, live))
        for _ in range(args.warmup):
            calls()
        if args.eager:                  # no graph: K calls launched from the host between two events
            reps = []
            for _ in range(ROOF_TIMED):
                gpu.record(e0)
                calls()
                gpu.record(e1)
                gpu.sync()
                reps.append(gpu.elapsed_ms(e0, e1) / args.steps * 1e3)
            reps.sort()
        else:
            reps = sorted(ms / args.steps * 1e3 for ms in graph_ms(gpu, calls, e0, e1, ROOF_TIMED, ROOF_UNTIMED))
        by = (pos + B) * 2 * nkv * hd * 4 + B * (nh * 2 * hd + 2 * nkv * hd + nh * hd) * 4
        rows.append({"pos": pos, "B": B, "head_split": live > 0, "us": round(reps[ROOF_TIMED // 2], 3),
                     "us_range": [round(reps[0], 3),
                     round(reps[-1], 3)], "bytes": by, "gbs": round(by / (reps[ROOF_TIMED // 2] * 1e-6) / 1e9, 1)})
        log(f"attention pos {pos} B {B}: {rows[-1]['us']} us per call, {rows[-1]['gbs']} GB/s")
    return rows


def bench_sample(args, gpu, host, roof, gemv_call_gbs):
    from qwen_pkg import pyqwen
    K, W, n_prompt = args.steps, args.warmup, args.prompt
    path = None
    if not args.no_cpu:
        path, spec = model_file(host, args.seed, weights=args.weights)
    else:
        spec = spec_27b(host, args.seed, args.weights)
    n_ctx = ((n_prompt + max(K, W) + 64 + 255) // 256) * 256
    m = pyqwen.Model(path, n_ctx) if path else pyqwen.Model(spec=spec, n_ctx=n_ctx)
    V = m.V
    prompt = np.random.default_rng(args.seed + 512).integers(0, V, n_prompt).astype(np.uint32)
    m.reset()
    m.generate_sample(prompt, W, *SAMPLE_CFG)                # warm-up (first call allocates the candidates)
    m.reset()
    toks, st = m.generate_sample(prompt, K, *SAMPLE_CFG)
    log(f"sampled decode: {len(toks)} tokens in {st.t_decode_s:.3f} s (prefill {st.t_prefill_s:.2f} s)")
    m.reset()
    gtoks, gst = m.generate_greedy(prompt, K)
    log(f"greedy decode: {len(gtoks)} tokens in {gst.t_decode_s:.3f} s")
    m.close()
    # the sampler kernels alone on 27B-vocabulary logits, graph replays of 200 calls
    L, reps = gpu.L, 200
    lg = gpu.put((np.random.default_rng(1).standard_normal(V) * 4).astype(np.float32))
    tk, rng, out = gpu.put(prompt[-64:]), gpu.put(np.array([7], np.uint64)), gpu.buf(4)
    e0, e1 = gpu.event(), gpu.event()
    kern = {}
    for name, (temp, top_p, top_k, pen) in {"sample_us": SAMPLE_CFG[:4], "sample_top256_us": (1.0, 1.0, 256, 1.1),
                                            "sample_greedy_us": (0.0, 1.0, 40, 1.1)}.items():
        def call():
            gpu.ok(L.qgpu_sample(lg.f32(), V, tk.u32(), 64, temp, top_p, top_k, pen, 64, rng.u64(), out.u32()))
        call()
        kern[name] = round(graph_ms(gpu, lambda: [call() for _ in range(reps)], e0, e1) * 1e3 / reps, 2)
    kern["argmax_us"] = round(graph_ms(gpu, lambda: [gpu.ok(L.qgpu_argmax(lg.f32(), V, V, 1, out.u32()))
                                                     for _ in range(reps)], e0, e1) * 1e3 / reps, 2)
    log(f"sampler kernels: {kern}")
    cpu = None
    if path:
        try:
            log("CPU baseline: reference sampled decode on the host cores")
            cpu = cpu_baseline_sample(path, prompt, SAMPLE_CFG, args.cpu_seconds, n_prompt)
        finally:
            os.remove(path)
    temp, top_p, top_k, pen, seed = SAMPLE_CFG
    return {
        "metric": f"sampled decode tok/s, 27B IQ4_XS (temp {temp}, top-p {top_p}, top-k {top_k}, repeat penalty "
                  f"{pen}) on 1 GPU", "value": round(len(toks) / st.t_decode_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": K, "warmup": W, "ms_per_step": round(st.t_decode_s / len(toks) * 1e3, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32 (IQ4_XS weights; int8-MFMA digit GEMV, fp32 accumulate; sampler fp32 / fp64 sum)",
        "data": "synthetic: seeded random-init 27B hybrid (IQ4_XS), seeded random-id prompt",
        "config": {"workload": f"27B hybrid sampled decode, {n_prompt}-token prompt, {K} tokens",
                   "prompt_tokens": n_prompt, "n_ctx": n_ctx, "sampler": {"temp": temp, "top_p": top_p,
                   "top_k": top_k, "repeat_penalty": pen, "repeat_last_n": 64, "seed": seed}},
        "greedy_tok_s": round(len(gtoks) / gst.t_decode_s, 2), **kern,
        "prefill_s": round(st.t_prefill_s, 3), "gemv_batch_gbs": round(gemv_call_gbs, 1), "roofline": roof,
        "cpu_baseline": cpu,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (model: cycles; gemv: calls)")
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--mode", choices=["model", "gemv", "longctx", "sweep", "sample", "attn"], default="model")
    ap.add_argument("--k", type=int, default=3, help="drafts per speculative cycle (model mode)")
    ap.add_argument("--prompt", type=int, default=None, help="prompt tokens (model 512, longctx 8192)")
    ap.add_argument("--forced-cycles", type=int, default=None)
    ap.add_argument("--seed", type=int, default=27)
    ap.add_argument("--gemv-steps", type=int, default=200)
    ap.add_argument("--gemv-warmup", type=int, default=20)
    ap.add_argument("--weights", choices=["iq4", "mix"], default="iq4",
                    help="model mode: every 2-D weight IQ4_XS (the headline workload) or the real checkpoint's "
                         "format mix (Q4_K embedding, Q5_K attn_qkv, Q6_K output, Q8_0 eh_proj)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=None)
    ap.add_argument("--eager", action="store_true",
                    help="attn mode: launch the timed calls from the host instead of replaying a HIP graph")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run the k_copy kernel on 256 MiB x 5 (reference point for PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    dflt = {"model": (256, 8, 512, 64, 15.0), "gemv": (200, 20, 0, 0, 5.0), "longctx": (0, 0, 8192, 16, 0.0),
            "sweep": (40, 5, 0, 0, 0.0), "sample": (128, 8, 512, 0, 15.0), "attn": (100, 5, 0, 0, 0.0)}
    s, w, p, f, c = dflt[args.mode]
    args.steps = s if args.steps is None else args.steps
    args.warmup = w if args.warmup is None else args.warmup
    args.prompt = p if args.prompt is None else args.prompt
    args.forced_cycles = f if args.forced_cycles is None else args.forced_cycles
    args.cpu_seconds = c if args.cpu_seconds is None else args.cpu_seconds

    from qwen_pkg import host_lib, pyqwen
    host, gpu = host_lib(), pyqwen.gpu_lib()
    name, ncu, _ = gpu.device_info()
    log(f"device {name}, {ncu} CUs; mode {args.mode}")
    gs, gw = (args.steps, args.warmup) if args.mode == "gemv" else (args.gemv_steps, args.gemv_warmup)
    roof, gemv_gbs, ms_call, wx = gemv_roofline(gpu, host, gs, gw)
    log(f"roofline {roof['kernel']}: {roof['kernel_us']} us/launch, {roof['achieved']} GB/s "
        f"({100 * roof['frac']:.1f}% of peak); gemv_batch call {gemv_gbs:.1f} GB/s")
    if args.copy_calib:
        nb = 256 << 20
        a, b = gpu.buf(nb), gpu.buf(nb)
        gpu.ok(gpu.L.qgpu_memset(ctypes.c_void_p(a.ptr), 1, nb))
        for _ in range(5):
            gpu.ok(gpu.L.qgpu_copy(ctypes.c_void_p(b.ptr), ctypes.c_void_p(a.ptr), nb))
        gpu.sync()
        a.close()
        b.close()
    if args.mode == "gemv":
        W, x, ne0, ne1, B = wx
        res = {
            "metric": METRIC, "value": round(gemv_gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_call, 5), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "fp32 (IQ4_XS weights; int8-MFMA digit GEMV, fp32 accumulate)",
            "data": "synthetic (seeded random IQ4_XS super-blocks, x ~ N(0,1))",
            "config": {"workload": "gemv_batch IQ4_XS 17408x5120, B=4 (1 token + 3 drafts)", "rows": ne1,
                       "cols": ne0, "B": B, "weight_copies": 12, "device": name, "cus": ncu},
            "roofline": roof,
            "cpu_baseline": None if args.no_cpu else cpu_baseline_gemv(W, x, ne0, ne1, B, args.cpu_seconds),
        }
    elif args.mode == "sweep":
        sweep = bench_sweep(gpu, host, args.steps, args.warmup)
        pick = next(r for r in sweep if r["format"] == "IQ4_XS" and r["rows"] == 17408 and r["B"] == 4)
        res = {
            "metric": METRIC, "value": pick["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(pick["us"] / 1e3, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None,
            "dtype": "fp32 (IQ4_XS, Q4_K, Q5_K, Q6_K, Q8_0 weights; int8-MFMA digit GEMV, fp32 accumulate)",
            "data": "synthetic (seeded random super-blocks per format, x ~ N(0,1))",
            "config": {"workload": "gemv_batch sweep: 5 formats x 3 shapes x B in {1,2,4,8}", "device": name,
                       "cus": ncu},
            "sweep": sweep, "roofline": roof, "cpu_baseline": None,
        }
    elif args.mode == "attn":
        att = bench_attn(args, gpu)
        pick = next(r for r in att if r["pos"] == 8392 and r["B"] == 8)
        res = {
            "metric": "attention call latency, 27B shapes (span kernel + combine), 8392 KV positions, B=8",
            "value": pick["us"], "unit": "us per attention call", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(pick["us"] / 1e3, 5), "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None,
            "dtype": "fp32 (q.k as fp16 hi/lo and p.v as bf16 hi/lo split products, fp32 accumulate)",
            "data": "synthetic (random caches, q, k, v ~ N(0,1))",
            "config": {"workload": "27B attention call (24 / 4 heads, head_dim 256): span kernel + combine, "
                                   "8392 KV positions, B = 8", "device": name, "cus": ncu},
            "attn": att, "roofline": roof, "cpu_baseline": None,
        }
    elif args.mode == "model":
        res = bench_model(args, gpu, host, roof, gemv_gbs)
    elif args.mode == "sample":
        res = bench_sample(args, gpu, host, roof, gemv_gbs)
    else:
        res = bench_longctx(args, gpu, host, roof, gemv_gbs)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
