"""Regenerates the golden fixtures in this directory from the compiled
reference engine (oracle/_ref/libqwenref.so, built by `make -C oracle` from
the reference sources).  Run here, where the reference checkout exists:

    python tests/golden/make_golden.py

Inputs are produced with the package's deterministic generator (same seed ->
same bytes on any host), so the fixtures store the generator seeds/ids next
to the inputs and the reference outputs:

  gemv_<FMT>_<ne0>x<ne1>.npz : W bytes, x [8][ne0], out_batch [8][ne1]
                               (gemv_batch n=8), out_single [8][ne1] (8 x gemv),
                               deq [ne1][ne0] (dequant_row of every row)
  ops.npz                    : test_ops.c:171-240 random-dimension cases
  model_<variant>.npz        : tiny hybrid model scenarios (ref_harness.c)
  model_tiny_accept.npz      : speculative scenarios (ref_harness.c spec mode) on the tiny model whose
                               drafts are mostly accepted (synth variant 2): natural streams and j for
                               k = 1..7, forced-acceptance streams, final logits / MTP state; keys
                               prefixed end_ come from a run that stops at the end of a short context
  model_tiny_accept_long.npz : the same model at n_ctx 8192 after an 8176-token prompt (ref_harness.c long
                               mode): prefill logits, natural and all-accepted streams for k = 1, 3, 5, 7
                               (`python tests/golden/make_golden.py long`, ~5 min)
  sampler.npz                : sampler_sample on seeded logits (3 calls per case): tokens, generator
                               state after each call, penalised logits
  model_27b.npz              : full-size 27B greedy stream of 256 tokens + top-2 gaps
                               (`python tests/golden/make_golden.py 27b`, ~10 min)
  model_27b_mix.npz          : the same for the 27B model with the real checkpoint's format mix
                               (token_embd Q4_K, attn_qkv Q5_K, output Q6_K, eh_proj Q8_0; `... 27bmix`)
  dropin_27b.npz             : what two of the reference's own programs print on the reference engine
                               (oracle/_ref/test_forward_cpu, debug_spec2_cpu, test_quant_cpu) for that format-mix 27B
                               file with the generator's byte-level vocabulary (`... dropin27b`, ~2 min)
"""
import ctypes
import hashlib
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_INC = "/root/reference/include"
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libqwenref.so")
sys.path.insert(0, os.path.join(ROOT, "tests"))
import qwen_pkg  # noqa: E402  (loads the package's ctypes bindings)

FMT = {"F32": 0, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_XS": 23}


class TensorInfo(ctypes.Structure):
    """Layout of gguf_tensor_info_t (GGUF descriptor)."""
    _fields_ = [("name", ctypes.c_char * 64), ("n_dims", ctypes.c_uint32),
                ("ne", ctypes.c_uint64 * 4), ("type", ctypes.c_int),
                ("offset", ctypes.c_uint64), ("data", ctypes.c_void_p)]


def fptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def gemv_fixtures(ref, host):
    ref.gemv_batch.argtypes = [ctypes.c_void_p, ctypes.POINTER(TensorInfo), ctypes.POINTER(ctypes.c_float),
                               ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(ctypes.c_float), ctypes.c_uint64]
    ref.gemv.argtypes = [ctypes.c_void_p, ctypes.POINTER(TensorInfo), ctypes.POINTER(ctypes.c_float),
                         ctypes.POINTER(ctypes.c_float)]
    ref.dequant_row.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_float)]
    ref.quant_row_bytes.restype = ctypes.c_size_t
    ref.quant_row_bytes.argtypes = [ctypes.c_int, ctypes.c_uint64]
    for fmt, t in FMT.items():
        for ne0, ne1, seed in ((512, 64, 11), (5120, 32, 12)):
            rb = ref.quant_row_bytes(t, ne0)
            sigma = 0.02 if t != 0 else 1.0
            W = host.synth_matrix(t, ne0, ne1, seed, 100 + t, sigma)
            assert W.nbytes == rb * ne1
            x = host.synth_normal(8 * ne0, seed, 7, 0.0, 1.0).reshape(8, ne0)
            ti = TensorInfo(name=b"W", n_dims=2, type=t, offset=0,
                            data=W.ctypes.data_as(ctypes.c_void_p))
            ti.ne[0], ti.ne[1], ti.ne[2], ti.ne[3] = ne0, ne1, 1, 1
            ob = np.zeros((8, ne1), np.float32)
            ref.gemv_batch(None, ctypes.byref(ti), fptr(x), ne0, 8, fptr(ob), ne1)
            os_ = np.zeros((8, ne1), np.float32)
            for k in range(8):
                row = np.ascontiguousarray(x[k])
                o = np.zeros(ne1, np.float32)
                ref.gemv(None, ctypes.byref(ti), fptr(row), fptr(o))
                os_[k] = o
            deq = np.zeros((ne1, ne0), np.float32)
            for r in range(ne1 if ne0 * ne1 <= 512 * 64 else 0):
                ref.dequant_row(t, ctypes.c_void_p(W.ctypes.data + r * rb), ne0, fptr(deq[r]))
            extra = {"deq": deq} if ne0 * ne1 <= 512 * 64 else {}
            np.savez(os.path.join(HERE, f"gemv_{fmt}_{ne0}x{ne1}.npz"), W=W, x=x, out_batch=ob,
                     out_single=os_, seed=np.uint64(seed), type=np.int32(t), sigma=np.float32(sigma), **extra)
            print(fmt, ne0, ne1, "batch==single:", np.array_equal(ob, os_))


def lcg_inputs(n, seed):
    """test_ops.c:184-189 input generator (LCG, returns new seed)."""
    x = np.zeros(n, np.float32)
    w = np.zeros(n, np.float32)
    for i in range(n):
        seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
        x[i] = np.float32(((seed >> 16) - 32768)) / np.float32(3276.8)
        seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
        w[i] = np.float32(0.5) + np.float32((seed >> 16) & 0xFFF) / np.float32(4096.0)
    return x, w, seed


def ops_fixtures(ref):
    P = ctypes.POINTER(ctypes.c_float)
    ref.rmsnorm.argtypes = [P, P, P, ctypes.c_uint64, ctypes.c_float]
    ref.l2norm.argtypes = [P, P, ctypes.c_uint64, ctypes.c_float]
    for f in ("silu_inplace", "sigmoid_inplace", "softplus_inplace", "softmax_inplace"):
        getattr(ref, f).argtypes = [P, ctypes.c_uint64]
    dims = [1, 3, 7, 8, 15, 16, 32, 64, 128, 256, 512, 5120]
    seed = 12345
    out = {}
    for n in dims:
        x, w, seed = lcg_inputs(n, seed)
        out[f"x_{n}"] = x
        out[f"w_{n}"] = w
        o = np.zeros(n, np.float32)
        ref.rmsnorm(fptr(o), fptr(x), fptr(w), n, 1e-6)
        out[f"rmsnorm_{n}"] = o.copy()
        ref.l2norm(fptr(o), fptr(x), n, 1e-6)
        out[f"l2norm_{n}"] = o.copy()
        for f in ("softmax", "silu", "sigmoid", "softplus"):
            y = x.copy()
            getattr(ref, f + "_inplace")(fptr(y), n)
            out[f"{f}_{n}"] = y
    # wide-range activations: exercise the +-88 clamp, the +-20 tails and the exp bit trick
    xr = np.linspace(-100, 100, 4099).astype(np.float32)
    out["x_range"] = xr
    for f in ("silu", "sigmoid", "softplus", "softmax"):
        y = xr.copy()
        getattr(ref, f + "_inplace")(fptr(y), xr.size)
        out[f"{f}_range"] = y
    np.savez(os.path.join(HERE, "ops.npz"), dims=np.array(dims, np.int64), **out)
    print("ops fixtures", len(out))


class Sampler(ctypes.Structure):
    """Layout of sampler_t (sampler.h:7-14)."""
    _fields_ = [("temp", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("repeat_penalty", ctypes.c_float), ("repeat_last_n", ctypes.c_uint32), ("rng_state", ctypes.c_uint64)]


# (vocab, temp, top_p, top_k, repeat_penalty, seed, window tokens): greedy, top-k / top-p edges, K > 256,
# K > vocab, penalties with repeated tokens
SAMPLER_CASES = [
    (1000, 0.0, 1.0, 40, 1.1, 5, 80), (1000, 0.8, 0.9, 40, 1.1, 7, 80), (1000, 1.0, 1.0, 1, 1.0, 9, 0),
    (17, 1.0, 1.0, 40, 1.0, 11, 30), (4103, 0.5, 0.5, 5, 1.3, 12345, 120), (4103, 1.5, 0.05, 256, 1.0, 3, 0),
    (40000, 1.2, 0.95, 300, 1.05, 42, 64), (40000, 0.7, 1.0, 2, 0.9, 0, 200), (9000, 1.0, 0.99, 128, 2.0, 77, 65),
]


def sampler_fixtures(ref):
    ref.sampler_init.restype = ctypes.POINTER(Sampler)
    ref.sampler_init.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_uint32, ctypes.c_float, ctypes.c_uint64]
    ref.sampler_sample.restype = ctypes.c_uint32
    ref.sampler_sample.argtypes = [ctypes.POINTER(Sampler), ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p,
                                   ctypes.c_size_t]
    ref.sampler_free.argtypes = [ctypes.POINTER(Sampler)]
    out = {}
    for c, (V, temp, top_p, top_k, pen, seed, W) in enumerate(SAMPLER_CASES):
        rng = np.random.default_rng(1000 + c)
        logits = (rng.standard_normal(V) * 3).astype(np.float32)
        toks = rng.integers(0, min(V, 50), W).astype(np.uint32)        # repeats inside the window
        s = ref.sampler_init(temp, top_p, top_k, pen, seed)
        tok, st, lg = [], [], []
        for step in range(3):
            l = logits.copy()
            tok.append(ref.sampler_sample(s, l.ctypes.data, V, toks.ctypes.data, len(toks)))
            st.append(s.contents.rng_state)
            lg.append(l)
        ref.sampler_free(s)
        out[f"logits_{c}"] = logits
        out[f"tokens_{c}"] = toks
        out[f"sampled_{c}"] = np.array(tok, np.uint32)
        out[f"state_{c}"] = np.array(st, np.uint64)
        out[f"penalised_{c}"] = lg[0]
    np.savez(os.path.join(HERE, "sampler.npz"), cases=np.array(SAMPLER_CASES, np.float64), **out)
    print("sampler", {c: out[f"sampled_{c}"].tolist() for c in range(len(SAMPLER_CASES))})


def model_fixtures(host):
    with tempfile.TemporaryDirectory() as td:
        exe = os.path.join(td, "ref_harness")
        subprocess.check_call(["gcc", "-O2", "-std=c11", f"-I{REF_INC}", os.path.join(HERE, "ref_harness.c"),
                               REF_LIB, f"-Wl,-rpath,{os.path.dirname(REF_LIB)}", "-lm", "-lpthread", "-o", exe])
        for variant, mixed, seed in (("tiny", 0, 1234), ("tiny_mixed", 1, 4321)):
            path = os.path.join(td, variant + ".gguf")
            host.write_tiny_gguf(path, seed, mixed)
            sha = hashlib.sha256(open(path, "rb").read()).hexdigest()
            outd = os.path.join(td, variant)
            os.makedirs(outd)
            subprocess.check_call([exe, path, outd, "256"])
            arrs = {}
            for fn in sorted(os.listdir(outd)):
                base, ext = fn.rsplit(".", 1)
                arrs[base] = np.fromfile(os.path.join(outd, fn), {"f32": np.float32, "f64": np.float64}.get(ext, np.uint32))
            np.savez(os.path.join(HERE, f"model_{variant}.npz"), gguf_sha256=np.array(sha), seed=np.uint64(seed),
                     mixed=np.int32(mixed), n_ctx=np.int32(256), **arrs)
            print(variant, sha[:16], {k: v.shape for k, v in arrs.items()})


ACCEPT_SEED = 1234
ACCEPT_RUNS = (("", 256, 20, 160), ("end_", 57, 20, 200))   # key prefix, n_ctx, n_prompt, n_predict


def accept_fixtures(host):
    """Speculative decode with drafts the backbone accepts (j over 0..k)."""
    with tempfile.TemporaryDirectory() as td:
        exe = os.path.join(td, "ref_harness")
        subprocess.check_call(["gcc", "-O2", "-std=c11", f"-I{REF_INC}", os.path.join(HERE, "ref_harness.c"),
                               REF_LIB, f"-Wl,-rpath,{os.path.dirname(REF_LIB)}", "-lm", "-lpthread", "-o", exe])
        path = os.path.join(td, "accept.gguf")
        host.write_tiny_gguf(path, ACCEPT_SEED, 2)
        sha = hashlib.sha256(open(path, "rb").read()).hexdigest()
        arrs = {}
        for pre, n_ctx, n_prompt, n_predict in ACCEPT_RUNS:
            outd = os.path.join(td, "out" + pre)
            os.makedirs(outd)
            subprocess.check_call([exe, path, outd, str(n_ctx), "spec", str(n_prompt), str(n_predict)])
            for fn in sorted(os.listdir(outd)):
                base, ext = fn.rsplit(".", 1)
                arrs[pre + base] = np.fromfile(os.path.join(outd, fn), {"f32": np.float32}.get(ext, np.uint32))
            arrs[pre + "n_ctx"] = np.int32(n_ctx)
            arrs[pre + "n_predict"] = np.int32(n_predict)
        np.savez(os.path.join(HERE, "model_tiny_accept.npz"), gguf_sha256=np.array(sha), seed=np.uint64(ACCEPT_SEED),
                 variant=np.int32(2), **arrs)
        for k in range(1, 8):
            print("k", k, "j histogram", np.bincount(arrs[f"spec_seq_k{k}_j"], minlength=k + 1).tolist(),
                  "| end", np.bincount(arrs[f"end_spec_seq_k{k}_j"], minlength=k + 1).tolist())


LONG_RUN = (8192, 8176, 12)      # n_ctx, n_prompt, n_predict


def long_fixtures(host):
    """Long context (8192 positions) on the draft-accepting tiny model."""
    with tempfile.TemporaryDirectory() as td:
        exe = os.path.join(td, "ref_harness")
        subprocess.check_call(["gcc", "-O2", "-std=c11", f"-I{REF_INC}", os.path.join(HERE, "ref_harness.c"),
                               REF_LIB, f"-Wl,-rpath,{os.path.dirname(REF_LIB)}", "-lm", "-lpthread", "-o", exe])
        path = os.path.join(td, "accept.gguf")
        host.write_tiny_gguf(path, ACCEPT_SEED, 2)
        sha = hashlib.sha256(open(path, "rb").read()).hexdigest()
        n_ctx, n_prompt, n_predict = LONG_RUN
        outd = os.path.join(td, "out")
        os.makedirs(outd)
        subprocess.check_call([exe, path, outd, str(n_ctx), "long", str(n_prompt), str(n_predict)])
        arrs = {}
        for fn in sorted(os.listdir(outd)):
            base, ext = fn.rsplit(".", 1)
            if base == "prompt":
                continue                                  # prompt_tok(i): regenerated by the tests
            arrs[base] = np.fromfile(os.path.join(outd, fn), {"f32": np.float32}.get(ext, np.uint32))
        np.savez(os.path.join(HERE, "model_tiny_accept_long.npz"), gguf_sha256=np.array(sha),
                 seed=np.uint64(ACCEPT_SEED), variant=np.int32(2), n_ctx=np.int32(n_ctx), n_prompt=np.int32(n_prompt),
                 n_predict=np.int32(n_predict), **arrs)
        print("long", {k: v.tolist() for k, v in arrs.items() if k.endswith("_j")})


SEED_27B = 27            # the benchmark's model seed
PROMPT_SEED_27B = 20251201


def model27b_fixture(host, n_prompt=512, n_gen=256, n_ctx=1024, mix=False):
    """Full-size random-init 27B: reference greedy stream after a seeded
    random-id prompt, with the top-2 gap of every step (the streams must agree
    wherever the gap exceeds 1e-2), plus the prefill logits.  mix: the real
    checkpoint's format mix (model_27b_mix.npz)."""
    with tempfile.TemporaryDirectory(dir=os.environ.get("GOLDEN_TMP", None)) as td:
        exe = os.path.join(td, "ref_harness")
        subprocess.check_call(["gcc", "-O2", "-std=c11", f"-I{REF_INC}", os.path.join(HERE, "ref_harness.c"),
                               REF_LIB, f"-Wl,-rpath,{os.path.dirname(REF_LIB)}", "-lm", "-lpthread", "-o", exe])
        spec = host.spec_27b_mix(SEED_27B) if mix else host.spec_27b(SEED_27B)
        path = os.path.join(td, "m27.gguf")
        host.write_gguf(spec, path)
        V = spec.vocab
        prompt = np.random.default_rng(PROMPT_SEED_27B).integers(0, V, n_prompt).astype(np.uint32)
        pf = os.path.join(td, "prompt.u32")
        prompt.tofile(pf)
        outd = os.path.join(td, "out")
        os.makedirs(outd)
        subprocess.check_call([exe, path, outd, str(n_ctx), "greedy", pf, str(n_gen)])
        # fingerprint of the generated weights: sha256 of a few tensors' bytes
        names = [b"blk.0.attn_qkv.weight", b"blk.3.attn_q.weight", b"blk.63.ffn_down.weight", b"output.weight",
                 b"token_embd.weight", b"blk.64.nextn.eh_proj.weight"] if mix else \
            [b"blk.0.attn_qkv.weight", b"blk.3.attn_q.weight", b"blk.63.ffn_down.weight", b"output.weight"]
        ts = host.tensors(spec)
        fp = {}
        for i, t in enumerate(ts):
            if t.name in names:
                fp[t.name.decode()] = hashlib.sha256(host.fill(spec, i, t.nbytes).tobytes()).hexdigest()
        np.savez(os.path.join(HERE, "model_27b_mix.npz" if mix else "model_27b.npz"), seed=np.uint64(SEED_27B),
                 prompt=prompt,
                 n_ctx=np.int32(n_ctx), stream=np.fromfile(os.path.join(outd, "stream.u32"), np.uint32),
                 gap=np.fromfile(os.path.join(outd, "gap.f32"), np.float32),
                 prefill_logits=np.fromfile(os.path.join(outd, "prefill_logits.f32"), np.float32),
                 fingerprint=np.array(json.dumps(fp)))
        print("27b fixture", fp)


def file_digest(path, span=32 << 20):
    """sha256 of a file's first and last `span` bytes (the GGUF header, metadata and vocabulary
    lie at the start; a full hash of 14.5 GB would take longer than the programs it checks)"""
    h = hashlib.sha256()
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        h.update(f.read(span))
        f.seek(max(0, size - span))
        h.update(f.read(span))
    h.update(str(size).encode())
    return h.hexdigest()


def dropin27b_fixture(host):
    """The reference's test_forward.c and debug_spec2.c, compiled on the reference engine, on the
    seeded 27B file carrying the generator's byte-level vocabulary: their printed output is what
    the same programs linked with libqwen.so must print on the GPU."""
    with tempfile.TemporaryDirectory(dir=os.environ.get("GOLDEN_TMP", None)) as td:
        spec = host.spec_27b_mix(SEED_27B)
        spec.tokenizer = 1
        path = os.path.join(td, "m27_mix_tok.gguf")
        host.write_gguf(spec, path)
        out = {}
        for prog in ("test_forward", "debug_spec2", "test_quant"):
            exe = os.path.join(ROOT, "oracle", "_ref", f"{prog}_cpu")
            # (test_quant exits 1 on this file: its plausibility rule |mean| < 0.5 does not hold for the
            # generator's ssm_a; the output is what is compared)
            out[prog] = subprocess.run([exe, path], capture_output=True, text=True, check=prog != "test_quant",
                                       cwd=td).stdout
        np.savez(os.path.join(HERE, "dropin_27b.npz"), seed=np.uint64(SEED_27B), digest=np.array(file_digest(path)),
                 test_forward=np.array(out["test_forward"]), debug_spec2=np.array(out["debug_spec2"]),
                 test_quant=np.array(out["test_quant"]))
        print(out["test_forward"])
        print(out["debug_spec2"])


def main():
    if not os.path.exists(REF_LIB):
        sys.exit("build the reference first: make -C oracle")
    ref = ctypes.CDLL(REF_LIB)
    host = qwen_pkg.host_lib()
    which = sys.argv[1:] or ["gemv", "ops", "model", "sampler", "accept"]
    if "gemv" in which:
        gemv_fixtures(ref, host)
    if "ops" in which:
        ops_fixtures(ref)
    if "model" in which:
        model_fixtures(host)
    if "sampler" in which:
        sampler_fixtures(ref)
    if "accept" in which:
        accept_fixtures(host)
    if "long" in which:
        long_fixtures(host)
    if "27b" in which:
        model27b_fixture(host)
    if "27bmix" in which:
        model27b_fixture(host, mix=True)
    if "dropin27b" in which:
        dropin27b_fixture(host)


if __name__ == "__main__":
    main()
