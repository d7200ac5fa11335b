"""GPU parity of the device sampler (qgpu_sample: the reference's sampler_sample,
sampler.c:62-162) and of the sampled decode loop built on it (model_generate_sample:
main.c:232-248), through the C-ABI.

Checkers: the golden vectors of the compiled reference's sampler (tests/golden/sampler.npz),
the oracle's restatement (bit-exact with those vectors) and the reference's sampled streams on
the tiny models.
Bars: the sampled token and the generator state after every call identical, the penalised
logits bit-identical.  The device exponential is exp in double rounded to float, the correctly
rounded expf; the C library's expf returns the same float except within about 2^-34 of a
rounding midpoint, and a token can only differ if such a case moves a cumulative sum across the
draw, which none of these seeded cases does.
"""
import ctypes
import hashlib
import os
import tempfile

import numpy as np
import pytest

import oracle_lib as O
from gpu_util import gpu  # noqa: F401
from qwen_pkg import host_lib, pyqwen

pytestmark = pytest.mark.gpu
VOCAB_27B = 248320


def load(name):
    return np.load(os.path.join(O.GOLDEN, name), allow_pickle=False)


def device_sample(gpu, logits, tokens, s, calls, repeat_last_n=64):
    """`calls` qgpu_sample calls, each on a fresh copy of `logits`, with the generator state of the
    initialised oracle sampler `s` kept in device memory.  Returns tokens, states, penalised logits."""
    lg = gpu.put(logits)
    tk = gpu.put(np.ascontiguousarray(tokens, np.uint32)) if len(tokens) else None
    rng = gpu.put(np.array([s.rng_state], np.uint64))
    out = gpu.buf(4)
    toks, states, pen = [], [], []
    for _ in range(calls):
        lg.upload(logits)
        gpu.ok(gpu.L.qgpu_sample(lg.f32(), len(logits), tk.u32() if tk else None, len(tokens), s.temp, s.top_p,
                                 s.top_k, s.repeat_penalty, repeat_last_n, rng.u64(), out.u32()))
        toks.append(int(out.download(np.uint32)[0]))
        states.append(int(rng.download(np.uint64)[0]))
        pen.append(lg.download(np.float32))
    return toks, states, pen


def oracle_sample(logits, tokens, s, calls):
    toks, states, pen = [], [], []
    for _ in range(calls):
        lg = logits.copy()
        toks.append(O.sample(s, lg, tokens))
        states.append(int(s.rng_state))
        pen.append(lg)
    return toks, states, pen


def test_sample_vs_reference_fixtures(gpu):
    """Every case of the compiled reference's vectors: greedy, top-k 1/2/5/40/128/256/300, K > vocab,
    nucleus 0.05..0.99, penalties 0.9..2.0 over windows with repeated tokens, seed 0."""
    z = load("sampler.npz")
    for c, (V, temp, top_p, top_k, pen, seed, W) in enumerate(z["cases"]):
        print(f"\n[sample] fixture {c}: V={int(V)} temp={temp} top_p={top_p} top_k={int(top_k)} pen={pen}",
              flush=True)
        s = O.sampler(temp, top_p, int(top_k), pen, int(seed))
        toks, states, pens = device_sample(gpu, z[f"logits_{c}"], z[f"tokens_{c}"], s, 3)
        assert toks == list(z[f"sampled_{c}"]), c
        assert states == list(z[f"state_{c}"]), c
        assert np.array_equal(pens[0].view(np.uint32), z[f"penalised_{c}"].view(np.uint32)), c


CASES = [  # vocab, temp, top_p, top_k, penalty, n window tokens (of which the last 64 count), seed
    (VOCAB_27B, 0.8, 0.9, 40, 1.1, 500, 7),
    (VOCAB_27B, 0.0, 1.0, 40, 1.3, 64, 1),
    (VOCAB_27B, 1.0, 1.0, 256, 1.0, 0, 2),
    (VOCAB_27B, 1.3, 0.97, 1000, 1.05, 70, 3),
    (VOCAB_27B, 0.6, 0.3, 2, 1.0, 0, 4),
    (4096, 1.0, 0.95, 100, 1.2, 64, 5),
    (4097, 0.9, 1.0, 64, 1.2, 80, 6),
    (131077, 1.1, 0.8, 200, 0.8, 64, 8),
    (1, 1.0, 1.0, 40, 1.0, 0, 9),
    (3, 2.0, 1.0, 40, 1.5, 9, 10),
    (1_000_003, 0.9, 0.95, 300, 1.1, 64, 11),             # one further selection pass over the block lists
    (1 << 24, 1.0, 1.0, 256, 1.0, 0, 12),                 # the largest vocabulary: two further passes
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_sample_vs_oracle(gpu, case):
    """Vocabularies from 1 to 2^24 (one selection block; 61 blocks for the 27B's 248,320; one and two
    further passes over the block lists), K > 256 clamped, K > vocabulary, window tokens outside the
    vocabulary ignored, 5 calls on one device generator."""
    V, temp, top_p, top_k, pen, W, seed = CASES[case]
    print(f"\n[sample] V={V} temp={temp} top_p={top_p} top_k={top_k} pen={pen} W={W}", flush=True)
    rng = np.random.default_rng(100 + case)
    logits = (rng.standard_normal(V) * 4).astype(np.float32)
    tokens = rng.integers(0, min(V, 60), W).astype(np.uint32)
    if W > 3:
        tokens[1] = V + 5                                   # outside the vocabulary: no penalty
    s = O.sampler(temp, top_p, top_k, pen, seed)
    want = oracle_sample(logits, tokens, s, 5)
    s = O.sampler(temp, top_p, top_k, pen, seed)
    got = device_sample(gpu, logits, tokens, s, 5)
    assert got[0] == want[0] and got[1] == want[1]
    for a, b in zip(got[2], want[2]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_sample_greedy_ties_and_signed_zero(gpu):
    """Greedy is the first maximum under strict > (-0.0 == +0.0), over a 27B-sized vocabulary."""
    V = VOCAB_27B
    base = -np.abs(np.random.default_rng(3).standard_normal(V)).astype(np.float32) - 1.0
    for pos, neg in (((100, 200000), None), ((200000,), 70000), ((5,), 240000)):
        lg = base.copy()
        lg[list(pos)] = 0.0
        if neg is not None:
            lg[neg] = -0.0
        s = O.sampler(0.0, 1.0, 40, 1.0, 1)
        want = oracle_sample(lg, [], s, 1)[0]
        got = device_sample(gpu, lg, [], O.sampler(0.0, 1.0, 40, 1.0, 1), 1)[0]
        assert got == want == [min(pos + ((neg,) if neg is not None else ()))]


def test_sample_ties_at_the_cut(gpu):
    """Integer logits (thousands of equal values): the candidates are K of the largest value, so every
    draw must be one of those tokens and the generator must advance as the oracle's does.  (Which K of
    the equal logits the reference keeps follows its heap; here the smallest indices.)"""
    V = 50000
    lg = np.random.default_rng(9).integers(-3, 4, V).astype(np.float32)
    top = np.flatnonzero(lg == 3)
    for K in (40, 256):
        s = O.sampler(1.0, 1.0, K, 1.0, 21)
        want = oracle_sample(lg, [], s, 4)
        got = device_sample(gpu, lg, [], O.sampler(1.0, 1.0, K, 1.0, 21), 4)
        assert got[1] == want[1]
        assert all(t in set(top[:K].tolist()) for t in got[0]), (K, got[0])


def test_sample_graph_replays_match_eager(gpu):
    """Three sampler calls captured in a HIP graph (the sampler issues kernels only, no memset): every
    replay, with eager sampler calls and host copies between replays, gives the eager tokens, generator
    state and penalised logits (after the first call, which allocated the candidate buffers)."""
    V = VOCAB_27B
    rng0 = np.random.default_rng(41)
    logits = (rng0.standard_normal(V) * 4).astype(np.float32)
    toks = rng0.integers(0, 200, 100).astype(np.uint32)
    L = gpu.L
    lg, tk = gpu.put(logits), gpu.put(toks)
    st, out = gpu.put(np.array([99], np.uint64)), gpu.buf(3 * 4)
    cfgs = [(0.8, 0.9, 40, 1.1), (1.0, 1.0, 256, 1.0), (0.0, 1.0, 40, 1.3)]

    def calls():
        for i, (temp, top_p, top_k, pen) in enumerate(cfgs):
            gpu.ok(L.qgpu_sample(lg.f32(), V, tk.u32(), len(toks), temp, top_p, top_k, pen, 64, st.u64(),
                                 out.u32(i)))

    def reset():
        lg.upload(logits)
        st.upload(np.array([99], np.uint64))

    reset()
    calls()
    want = (out.download(np.uint32).tolist(), int(st.download(np.uint64)[0]), lg.download(np.float32))
    gpu.sync()
    gpu.ok(L.qgpu_graph_begin())
    calls()
    g = ctypes.c_void_p()
    gpu.ok(L.qgpu_graph_end(ctypes.byref(g)))
    try:
        for rep in range(4):
            reset()
            out.upload(np.zeros(3, np.uint32))
            gpu.ok(L.qgpu_graph_launch(g))
            gpu.sync()
            got = (out.download(np.uint32).tolist(), int(st.download(np.uint64)[0]), lg.download(np.float32))
            assert got[0] == want[0] and got[1] == want[1], rep
            assert np.array_equal(got[2].view(np.uint32), want[2].view(np.uint32)), rep
            reset()
            calls()                                     # eager work between replays
            gpu.sync()
            assert out.download(np.uint32).tolist() == want[0], rep
    finally:
        gpu.ok(L.qgpu_graph_destroy(g))


def test_sample_rejects_bad_arguments(gpu):
    lg = gpu.put(np.zeros(8, np.float32))
    out = gpu.buf(4)
    rng = gpu.put(np.array([1], np.uint64))
    tk = gpu.put(np.zeros(5000, np.uint32))
    L = gpu.L
    assert L.qgpu_sample(lg.f32(), 8, None, 0, 1.0, 1.0, 0, 1.0, 64, rng.u64(), out.u32()) < 0    # top_k 0
    assert L.qgpu_sample(lg.f32(), 0, None, 0, 1.0, 1.0, 40, 1.0, 64, rng.u64(), out.u32()) < 0   # empty vocab
    assert L.qgpu_sample(lg.f32(), 8, None, 0, 1.0, 1.0, 40, 1.0, 64, None, out.u32()) < 0        # no generator
    assert L.qgpu_sample(lg.f32(), 8, tk.u32(), 5000, 1.0, 1.0, 40, 1.1, 5000, rng.u64(),
                         out.u32()) < 0                                                          # window > 4096
    gpu.ok(L.qgpu_sample(lg.f32(), 8, None, 0, 0.0, 1.0, 40, 1.0, 64, None, out.u32()))          # greedy: no rng


# ---------------------------------------------------------------- sampled decode on the tiny models
@pytest.fixture(scope="module", params=["tiny", "tiny_mixed"])
def tiny(request):
    z = load(f"model_{request.param}.npz")
    td = tempfile.mkdtemp()
    path = os.path.join(td, "m.gguf")
    host_lib().write_tiny_gguf(path, int(z["seed"]), int(z["mixed"]))
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(z["gguf_sha256"])
    yield path, z
    os.remove(path)


def test_model_sample_stream(gpu, tiny):
    """model_generate_sample against (1) the oracle sampler replayed on the GPU model's own logits
    (the same forward calls through the host API: 8-token prefill chunks, then single tokens), token
    for token, and (2) the reference's sampled streams."""
    path, z = tiny
    n_ctx = int(z["n_ctx"])
    prompt = z["prompt"][:20]
    for c, (temp, top_p, top_k, pen, seed) in enumerate(z["sample_cfg"].reshape(4, 5)):
        print(f"\n[sample] {os.path.basename(path)} stream {c}", flush=True)
        m = pyqwen.Model(path, n_ctx)
        toks, st = m.generate_sample(prompt, 40, temp, top_p, int(top_k), pen, int(seed))
        m.close()
        assert len(toks) == 40
        m = pyqwen.Model(path, n_ctx)
        s = O.sampler(temp, top_p, int(top_k), pen, int(seed))
        for p0 in range(0, 20, 8):
            lg = m.forward_batch(prompt[p0:p0 + 8], p0)[-1]
        seen = list(prompt)
        for i in range(40):
            want = O.sample(s, lg.copy(), np.array(seen, np.uint32))
            assert toks[i] == want, (c, i)
            seen.append(int(toks[i]))
            if i + 1 < 40:
                lg = m.forward(int(toks[i]), 20 + i)
        m.close()
        assert np.array_equal(toks, z[f"sample_c{c}"]), c
