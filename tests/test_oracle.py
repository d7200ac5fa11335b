"""Pins the oracle (CPU restatement) against the reference's golden vectors and
against mathematics (closed forms, known answers, FP64 brute force).  CPU only.

Golden vectors: tests/golden/*.npz, produced from the compiled reference by
tests/golden/make_golden.py.  Known answers: reference src/test_ops.c:98-169.
"""
import ctypes
import hashlib
import os
import tempfile

import numpy as np
import pytest

import oracle_lib as O
from qwen_pkg import host_lib

FORMATS = ["F32", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "IQ4_XS"]


def load(name):
    return np.load(os.path.join(O.GOLDEN, name), allow_pickle=False)


# ---------------------------------------------------------------- GEMV / dequant
@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("shape", ["512x64", "5120x32"])
def test_oracle_gemv_bitexact_vs_reference(fmt, shape):
    """oracle gemv_batch == reference gemv_batch and == n single gemv (kernels.c:570-648,
    test_batch.c:38-58 property), bit for bit."""
    z = load(f"gemv_{fmt}_{shape}.npz")
    ne0, ne1 = map(int, shape.split("x"))
    t = int(z["type"])
    for n in (1, 3, 8):
        out = O.gemv(t, z["W"], ne0, ne1, z["x"][:n], n)
        assert np.array_equal(out, z["out_batch"][:n]), f"{fmt} n={n}"
    assert np.array_equal(z["out_batch"], z["out_single"])


@pytest.mark.parametrize("fmt", FORMATS)
def test_oracle_dequant_bitexact_vs_reference(fmt):
    z = load(f"gemv_{fmt}_512x64.npz")
    deq = O.dequant_rows(int(z["type"]), z["W"], 512, 64)
    assert np.array_equal(deq, z["deq"])


@pytest.mark.parametrize("fmt", FORMATS)
def test_oracle_gemv_vs_fp64(fmt):
    """FP64 dot of dequantised rows (test_kernels.c:35-49): max rel < 1e-4."""
    z = load(f"gemv_{fmt}_512x64.npz")
    ref = z["x"].astype(np.float64) @ z["deq"].astype(np.float64).T
    out = O.gemv(int(z["type"]), z["W"], 512, 64, z["x"], 8)
    err = np.abs(out - ref).max() / np.abs(ref).max()
    assert err < 1e-5


@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_K", "Q5_K", "Q6_K", "IQ4_XS"])
def test_oracle_unit_vector_probe(fmt):
    """debug_kernels.c:22-28: gemv with x = e_i returns dequantised element i exactly."""
    z = load(f"gemv_{fmt}_512x64.npz")
    t = int(z["type"])
    idx = [0, 1, 7, 8, 15, 16, 31, 32, 100, 255, 256, 300, 511]
    x = np.zeros((len(idx), 512), np.float32)
    for k, i in enumerate(idx):
        x[k, i] = 1.0
    outs = [O.gemv(t, z["W"], 512, 64, x[k:k + 1], 1)[0] for k in range(len(idx))]
    for k, i in enumerate(idx):
        if t in (12, 13):   # K-quants: d*sc*q - dmin*m*1 evaluated as two terms
            assert np.allclose(outs[k], z["deq"][:, i], rtol=0, atol=1e-6 * np.abs(z["deq"]).max())
        else:
            assert np.array_equal(outs[k], z["deq"][:, i])


def test_fp16_closed_form():
    """fp16 -> fp32 against numpy's IEEE half for every bit pattern (quant.c:6-28)."""
    L = O.lib()
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([L.or_fp16_to_f32(int(v)) for v in h[::7]], np.float32)
    sel = ref[::7]
    fin = np.isfinite(sel)
    assert np.array_equal(got[fin].view(np.uint32), sel[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(sel)]))


# ---------------------------------------------------------------- ops
def test_oracle_ops_bitexact_vs_reference():
    z = load("ops.npz")
    L = O.lib()
    for n in z["dims"]:
        n = int(n)
        x, w = z[f"x_{n}"], z[f"w_{n}"]
        o = np.zeros(n, np.float32)
        L.or_rmsnorm(O.fptr(o), O.fptr(x), O.fptr(w), n, 1e-6)
        assert np.array_equal(o, z[f"rmsnorm_{n}"]), n
        L.or_l2norm(O.fptr(o), O.fptr(x), n, 1e-6)
        assert np.array_equal(o, z[f"l2norm_{n}"]), n
        for f in ("softmax", "silu", "sigmoid", "softplus"):
            y = x.copy()
            getattr(L, f"or_{f}_inplace")(O.fptr(y), n)
            assert np.array_equal(y, z[f"{f}_{n}"]), (f, n)
    xr = z["x_range"]
    for f in ("silu", "sigmoid", "softplus", "softmax"):
        y = xr.copy()
        getattr(L, f"or_{f}_inplace")(O.fptr(y), xr.size)
        assert np.array_equal(y, z[f"{f}_range"]), f


def test_oracle_ops_known_answers():
    """test_ops.c:98-169 known answers."""
    L = O.lib()
    o = np.zeros(4, np.float32)
    L.or_rmsnorm(O.fptr(o), O.fptr(np.ones(4, np.float32)), O.fptr(np.full(4, 2, np.float32)), 4, 0.0)
    assert np.allclose(o, 2.0, rtol=1e-6)
    x = np.array([3, 4], np.float32)
    o2 = np.zeros(2, np.float32)
    L.or_l2norm(O.fptr(o2), O.fptr(x), 2, 1e-5)
    assert np.allclose(o2, [0.6, 0.8], rtol=1e-6)
    z4 = np.zeros(4, np.float32)
    L.or_l2norm(O.fptr(o), O.fptr(z4), 4, 1e-5)
    assert np.all(o == 0)
    s = np.array([0, 2, -20, 20], np.float32)
    L.or_silu_inplace(O.fptr(s), 4)
    assert np.allclose(s, [0, 2 / (1 + np.exp(-2)), -20 * np.exp(-20), 20], rtol=1e-4)
    g = np.array([0, 100, -100, 1, -1], np.float32)
    L.or_sigmoid_inplace(O.fptr(g), 5)
    assert np.allclose(g, [0.5, 1, 0, 1 / (1 + np.e ** -1), 1 / (1 + np.e)], rtol=1e-6, atol=1e-30)
    sp = np.array([0, 1, -50, 50, 100, 1000], np.float32)
    L.or_softplus_inplace(O.fptr(sp), 6)
    assert np.allclose(sp, [np.log(2), np.log1p(np.e), np.exp(-50), 50, 100, 1000], rtol=1e-5)
    sm = np.full(4, 1000, np.float32)
    L.or_softmax_inplace(O.fptr(sm), 4)
    assert np.allclose(sm, 0.25, rtol=1e-6)


def test_exp_lane_properties():
    """exp256_ps lane: exact at 0, rel err < 2e-6 of exp(float32 x) inside [-80, 80], 0 below the
    -88 clamp's 2^-127 floor (the exponent-bit construction gives +0 for k = -127)."""
    L = O.lib()
    assert L.or_exp8_lane(0.0) == 1.0
    for k in range(-20, 21):
        xf = float(np.float32(k * np.log(2)))
        assert L.or_exp8_lane(xf) == pytest.approx(np.exp(xf), rel=2e-6)
    xs = np.linspace(-80, 80, 2001)
    got = np.array([L.or_exp8_lane(float(v)) for v in xs], np.float64)
    assert np.max(np.abs(got - np.exp(xs.astype(np.float32).astype(np.float64))) / np.exp(xs)) < 2e-6
    assert L.or_exp8_lane(-1000.0) == 0.0


def test_argmax_ties_lowest_index():
    L = O.lib()
    a = np.array([1, 5, 5, 2, 5], np.float32)
    assert L.or_argmax(O.fptr(a), 5) == 1
    assert L.or_argmax(O.fptr(np.zeros(7, np.float32)), 7) == 0


# ---------------------------------------------------------------- GDN closed form
def gdn_fp64(T, cd, nk, nv, hk, hv, eps, qkv, br, ar, cw, dtb, sa, conv, ssm):
    """FP64 statement of the Gated DeltaNet step (model.c:494-524, 572-575, 891-916):
    S <- g S + beta (v - g S k) k^T ; o = (g S q + d (k.q)) / sqrt(hk)  computed as S' q / sqrt(hk)."""
    conv = conv.astype(np.float64).copy()
    S = ssm.astype(np.float64).reshape(nv, hv, hk).copy()
    outs = []
    for b in range(T):
        conv[:, :3] = conv[:, 1:]
        conv[:, 3] = qkv[b]
        y = (conv * cw.reshape(cd, 4)).sum(1)
        y = y / (1 + np.exp(-y))
        q = y[:nk * hk].reshape(nk, hk)
        k = y[nk * hk:2 * nk * hk].reshape(nk, hk)
        v = y[2 * nk * hk:].reshape(nv, hv)
        q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), eps)
        k = k / np.maximum(np.linalg.norm(k, axis=1, keepdims=True), eps)
        o = np.zeros((nv, hv))
        for h in range(nv):
            kh = h % nk
            beta = 1 / (1 + np.exp(-br[b, h]))
            a = ar[b, h] + dtb[h]
            g = np.exp(sa[h] * (a if a > 30 else np.log1p(np.exp(a))))
            Sg = g * S[h]
            d = (v[h] - Sg @ k[kh]) * beta
            S[h] = Sg + np.outer(d, k[kh])
            o[h] = S[h] @ q[kh] / np.sqrt(hk)
        outs.append(o.reshape(-1))
    return np.array(outs), conv, S.reshape(-1)


def test_oracle_gdn_vs_fp64_and_snapshots():
    """Config-3 parameterisation at reduced heads: oracle GDN block vs FP64 closed
    form, and snapshot b == state after running tokens 0..b alone."""
    host = host_lib()
    T, nk, nv, hk = 4, 2, 6, 128
    hv, cd, eps = hk, 2 * nk * hk + nv * hk, 1e-6
    rng = np.random.default_rng(5)
    qkv = rng.standard_normal((T, cd)).astype(np.float32)
    br = rng.standard_normal((T, nv)).astype(np.float32)
    ar = rng.standard_normal((T, nv)).astype(np.float32)
    cw = (0.5 * rng.standard_normal(cd * 4)).astype(np.float32)
    dtb = np.zeros(nv, np.float32)
    sa = -np.ones(nv, np.float32)
    conv0 = rng.standard_normal(cd * 4).astype(np.float32) * 0.1
    ssm0 = (0.01 * rng.standard_normal(nv * hv * hk)).astype(np.float32)
    L = O.lib()
    conv, ssm = conv0.copy(), ssm0.copy()
    out = np.zeros(T * nv * hv, np.float32)
    sc = np.zeros(T * cd * 4, np.float32)
    ss = np.zeros(T * nv * hv * hk, np.float32)
    L.or_gdn_block(T, cd, nk, nv, hk, hv, eps, O.fptr(qkv), O.fptr(br), O.fptr(ar), O.fptr(cw), O.fptr(dtb),
                   O.fptr(sa), O.fptr(conv), O.fptr(ssm), O.fptr(out), O.fptr(sc), O.fptr(ss))
    ref_o, ref_c, ref_s = gdn_fp64(T, cd, nk, nv, hk, hv, eps, qkv, br, ar, cw, dtb, sa, conv0.reshape(cd, 4), ssm0)
    assert np.abs(out.reshape(T, -1) - ref_o).max() / np.abs(ref_o).max() < 1e-5
    assert np.abs(ssm - ref_s).max() / np.abs(ref_s).max() < 1e-5
    assert np.array_equal(ss[-nv * hv * hk:], ssm) and np.array_equal(sc[-cd * 4:], conv)
    for b in range(T - 1):       # snapshot b == state after tokens 0..b run alone
        c2, s2 = conv0.copy(), ssm0.copy()
        o2 = np.zeros((b + 1) * nv * hv, np.float32)
        L.or_gdn_block(b + 1, cd, nk, nv, hk, hv, eps, O.fptr(qkv), O.fptr(br), O.fptr(ar), O.fptr(cw),
                       O.fptr(dtb), O.fptr(sa), O.fptr(c2), O.fptr(s2), O.fptr(o2), None, None)
        assert np.array_equal(ss[b * nv * hv * hk:(b + 1) * nv * hv * hk], s2)
        assert np.array_equal(sc[b * cd * 4:(b + 1) * cd * 4], c2)


# ---------------------------------------------------------------- model
@pytest.fixture(scope="module", params=["tiny", "tiny_mixed"])
def tiny_model(request):
    z = load(f"model_{request.param}.npz")
    host = host_lib()
    td = tempfile.mkdtemp()
    path = os.path.join(td, "m.gguf")
    host.write_tiny_gguf(path, int(z["seed"]), int(z["mixed"]))
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(z["gguf_sha256"]), \
        "generator no longer reproduces the fixture's GGUF"
    yield path, z
    os.remove(path)


def test_oracle_model_forward_bitexact(tiny_model):
    path, z = tiny_model
    V = 1024
    m = O.Model(path, int(z["n_ctx"]))
    p = z["prompt"]
    lb = m.forward_batch(p[:8], 0, 0)
    assert np.array_equal(lb.reshape(-1), z["batch_logits"])
    assert np.array_equal(m.h_save(8).reshape(-1), z["batch_hsave"])
    m.close()
    m = O.Model(path, int(z["n_ctx"]))
    seq = np.array([m.forward(int(p[i]), i) for i in range(8)])
    assert np.array_equal(seq.reshape(-1), z["seq_logits"])
    m.close()
    m = O.Model(path, int(z["n_ctx"]))
    m.forward_batch(p[:8], 0, 0)
    m.L.or_mtp_forward_batch(m.h, O.uptr(np.ascontiguousarray(p[:8])), 0, 8, 0)
    m.L.or_mtp_forward(m.h, int(p[8]), 8, 1)
    assert np.array_equal(m.arr(m.L.or_model_logits, V), z["mtp_logits"])
    assert np.array_equal(m.arr(m.L.or_model_mtp_h, m.E), z["mtp_h"])



def _tied_pair(mixed):
    """two tiny GGUFs that differ only in output.weight: absent (the lm_head falls back to
    token_embd, model.c:87-88) or present as an exact copy of token_embd"""
    host = host_lib()
    td = tempfile.mkdtemp()
    paths = []
    for tie in (1, 2):
        spec = host.spec_tiny(31, mixed)
        spec.tie_output = tie
        path = os.path.join(td, f"tie{tie}.gguf")
        host.write_gguf(spec, path)
        paths.append(path)
    return paths


@pytest.mark.parametrize("mixed", [0, 1])
def test_oracle_tied_output_equals_explicit_copy(mixed):
    """A model file without output.weight (model.c:87-88: the lm_head is token_embd) gives, bit for bit,
    the logits of the same model whose output.weight is an explicit copy of token_embd: batched and
    sequential forwards and the MTP draft logits.  (mixed: a Q4_K token_embd as the lm_head.)"""
    paths = _tied_pair(mixed)
    p = np.random.default_rng(5).integers(0, 1024, 9).astype(np.uint32)
    res = []
    for path in paths:
        m = O.Model(path, 64)
        lb = m.forward_batch(p[:8], 0, 0)
        m.L.or_mtp_forward_batch(m.h, O.uptr(np.ascontiguousarray(p[:8])), 0, 8, 0)
        m.L.or_mtp_forward(m.h, int(p[8]), 8, 1)
        ml = m.arr(m.L.or_model_logits, m.V)
        m.close()
        m = O.Model(path, 64)
        seq = np.array([m.forward(int(p[i]), i) for i in range(4)])
        m.close()
        res.append((lb, ml, seq))
    for a, b in zip(res[0], res[1]):
        assert np.array_equal(a, b)
    for path in paths:
        os.remove(path)

def test_oracle_rollback_bitexact(tiny_model):
    path, z = tiny_model
    p = z["prompt"]
    m = O.Model(path, int(z["n_ctx"]))
    for i in range(5):
        m.forward(int(p[i]), i)
    m.forward_batch(p[10:13], 5, 1)
    m.L.or_model_rollback_to(m.h, 1)
    m.L.or_model_set_pos(m.h, 8)
    lb = m.forward_batch(p[13:16], 7, 1)
    assert np.array_equal(lb.reshape(-1), z["rollback_logits"])


@pytest.mark.parametrize("k", [1, 2, 3, 5, 7])
def test_oracle_spec_stream_bitexact(tiny_model, k):
    """k<=2: the reference's own loop (batched verify + rollback); k>2: the reference's
    sequential-verify harness; both must equal the oracle's batched spec loop."""
    path, z = tiny_model
    m = O.Model(path, int(z["n_ctx"]), k_max=7)
    toks, js, st = m.generate_spec(z["prompt"][:20], 40, k)
    key = f"spec_k{k}" if k <= 2 else f"spec_seq_k{k}"
    assert np.array_equal(toks, z[key])
    assert np.array_equal(js, z[f"spec_j_k{k}" if k <= 2 else f"spec_seq_j_k{k}"][:len(js)])
    assert np.array_equal(toks, z["greedy"]), "spec stream must equal the greedy stream"


def test_oracle_greedy_stream_bitexact(tiny_model):
    path, z = tiny_model
    m = O.Model(path, int(z["n_ctx"]))
    assert np.array_equal(m.generate_greedy(z["prompt"][:20], 40), z["greedy"])


# ---------------------------------------------------------------- sampler (sampler.c:46-162)
def test_oracle_sampler_bitexact_vs_reference():
    """Three sampler_sample calls per case against the compiled reference: tokens, the generator
    state after each call and the penalised logits (greedy, top-k 1/2/5/40/128/256/300, K > vocab,
    nucleus 0.05..0.99, penalties 0.9..2.0 with repeated window tokens, seed 0)."""
    z = load("sampler.npz")
    for c, (V, temp, top_p, top_k, pen, seed, W) in enumerate(z["cases"]):
        s = O.sampler(temp, top_p, int(top_k), pen, int(seed))
        for step in range(3):
            lg = z[f"logits_{c}"].copy()
            tok = O.sample(s, lg, z[f"tokens_{c}"])
            assert tok == z[f"sampled_{c}"][step], (c, step)
            assert s.rng_state == z[f"state_{c}"][step], (c, step)
            if step == 0:
                assert np.array_equal(lg.view(np.uint32), z[f"penalised_{c}"].view(np.uint32)), c


def test_oracle_sampler_defaults_and_greedy():
    """sampler_init's defaults (sampler.c:46-56), and greedy = the first maximum of the penalised logits."""
    s = O.sampler(0.7, 0.9, 0, -1.0, 0)
    assert (s.top_k, s.repeat_penalty, s.repeat_last_n, s.rng_state) == (40, 1.0, 64, 0x123456789abcdef)
    rng = np.random.default_rng(5)
    lg = rng.standard_normal(300).astype(np.float32)
    lg[[17, 200]] = 9.0                                  # tie: the earlier index wins
    for temp, k in ((0.0, 40), (1.0, 1), (-2.0, 7)):
        s = O.sampler(temp, 1.0, k, 1.0, 3)
        st0 = s.rng_state
        assert O.sample(s, lg.copy(), []) == 17
        assert s.rng_state == st0, "greedy draws no random number"
    # penalty: 17 occurs twice in the window (9 / 1.5 / 1.5 = 4), 200 once (9 / 1.5 = 6)
    s = O.sampler(0.0, 1.0, 40, 1.5, 3)
    l2 = lg.copy()
    assert O.sample(s, l2, [17, 5, 17, 200]) == 200
    assert l2[17] == np.float32(np.float32(9.0 / 1.5) / np.float32(1.5)) and l2[200] == np.float32(9.0 / 1.5)
    neg = l2[5]
    assert neg == (lg[5] / np.float32(1.5) if lg[5] > 0 else lg[5] * np.float32(1.5))
    # only the last repeat_last_n = 64 tokens count
    l3 = lg.copy()
    O.sample(O.sampler(0.0, 1.0, 40, 1.5, 3), l3, [17] + [1] * 64)
    assert l3[17] == lg[17]


def _draws(temp, top_p, top_k, lg, n, seed=11):
    s = O.sampler(temp, top_p, top_k, 1.0, seed)
    return np.bincount([O.sample(s, lg.copy(), []) for _ in range(n)], minlength=len(lg))


def test_oracle_sampler_distribution():
    """Draw frequencies against the closed form: softmax(l / temp) restricted to the top-k largest logits
    and to the shortest descending prefix whose mass reaches top_p, renormalised (5-sigma bands)."""
    lg = np.array([2.0, 0.5, 1.5, -1.0, 1.0, 0.0, 2.5, -0.5], np.float32)
    order = np.argsort(-lg, kind="stable")
    n = 40000
    for temp, top_p, top_k in ((1.0, 1.0, 8), (0.5, 1.0, 8), (2.0, 1.0, 3), (1.0, 0.7, 8), (0.7, 0.8, 5)):
        z = lg[order[:top_k]].astype(np.float64) / temp
        p = np.exp(z - z.max())
        p /= p.sum()
        m = len(p)
        if top_p < 1.0:
            m = int(np.searchsorted(np.cumsum(p), top_p) + 1)
        q = np.zeros(len(lg))
        q[order[:m]] = p[:m] / p[:m].sum()
        f = _draws(temp, top_p, top_k, lg, n)
        assert np.all(f[q == 0] == 0), (temp, top_p, top_k)
        sig = np.sqrt(n * q * (1 - q)) + 1
        assert np.all(np.abs(f - n * q) < 5 * sig), (temp, top_p, top_k, f, n * q)


def test_oracle_sample_stream_bitexact(tiny_model):
    """The sampled decode of main.c:232-248 (prefill, then sample / forward) on the tiny models."""
    path, z = tiny_model
    for c, (temp, top_p, top_k, pen, seed) in enumerate(z["sample_cfg"].reshape(4, 5)):
        m = O.Model(path, int(z["n_ctx"]))
        s = O.sampler(temp, top_p, int(top_k), pen, int(seed))
        assert np.array_equal(m.generate_sample(z["prompt"][:20], 40, s), z[f"sample_c{c}"]), c
        m.close()


# ---------------------------------------------------------------- accepted drafts (j > 0)
@pytest.fixture(scope="module")
def accept_model():
    """The tiny model whose MTP drafts the backbone mostly accepts (synth variant 2)."""
    z = load("model_tiny_accept.npz")
    td = tempfile.mkdtemp()
    path = os.path.join(td, "accept.gguf")
    host_lib().write_tiny_gguf(path, int(z["seed"]), int(z["variant"]))
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(z["gguf_sha256"]), \
        "generator no longer reproduces the fixture's GGUF"
    yield path, z
    os.remove(path)


def accept_key(pre, force, k):
    if force:
        return f"{pre}spec_f{force}_k{k}"
    return f"{pre}spec_k{k}" if k <= 2 else f"{pre}spec_seq_k{k}"


def test_accept_fixture_spans_every_j():
    """The reference's own loops accept every number of drafts 0..k on this model (k = 1..7), the
    batched loop of main.c and the sequential-verify harness agree exactly (k <= 2), and every
    natural stream is the greedy stream (lossless speculation)."""
    z = load("model_tiny_accept.npz")
    for k in range(1, 8):
        assert set(np.unique(z[f"spec_seq_k{k}_j"]).tolist()) == set(range(k + 1)), k
    for pre in ("", "end_"):
        for k in (1, 2):
            for suf in ("", "_j", "_last", "_mtph"):
                assert np.array_equal(z[f"{pre}spec_k{k}{suf}"], z[f"{pre}spec_seq_k{k}{suf}"]), (pre, k, suf)
        g = z[f"{pre}greedy"]
        for k in range(1, 8):
            s = z[accept_key(pre, 0, k)]
            assert np.array_equal(s, g[:len(s)]), (pre, k)


@pytest.mark.parametrize("pre", ["", "end_"])
@pytest.mark.parametrize("force", [0, 1, 2])
@pytest.mark.parametrize("k", range(1, 8))
def test_oracle_spec_accept_bitexact(accept_model, pre, force, k):
    """The oracle's batched speculative loop (verify of k+1 tokens, rollback to j, re-anchor) against
    the reference: tokens, j of every cycle, the logits the next cycle starts from and the MTP state,
    bit for bit.  end_: a 57-position context that the loop runs into (main.c:210 stop)."""
    path, z = accept_model
    m = O.Model(path, int(z[pre + "n_ctx"]), k_max=7)
    toks, js, st = m.generate_spec(z["prompt"], int(z[pre + "n_predict"]), k, force_accept=force)
    key = accept_key(pre, force, k)
    assert np.array_equal(toks, z[key])
    assert np.array_equal(js, z[key + "_j"])
    last = m.arr(m.L.or_model_logits_b, (k + 1) * m.V).reshape(k + 1, m.V)[js[-1]]
    assert np.array_equal(last.view(np.uint32), z[key + "_last"].view(np.uint32))
    assert np.array_equal(m.arr(m.L.or_model_mtp_h, m.E).view(np.uint32), z[key + "_mtph"].view(np.uint32))
    if force == 1:
        assert np.all(js[:-1] == k)


@pytest.mark.parametrize("force,k", [(0, 3), (0, 7), (1, 3), (1, 7), (2, 3), (2, 4)])
def test_oracle_spec_state_equals_sequential_forward(accept_model, force, k):
    """What the mathematics fixes: after the cycles, the logits the loop continues from are the
    logits of a plain sequential model_forward over the prompt and every token the cycles verified
    and kept (cand[0..j] of each cycle), whatever the acceptance rule.  In the natural mode the kept
    tokens are the greedy stream (also past the emission cut of n_predict)."""
    path, z = accept_model
    key = accept_key("", force, k)
    toks, js = z[key], z[key + "_j"]
    kept = int(np.sum(js + 1))
    if force == 0:
        assert kept <= len(z["greedy"])
        toks = z["greedy"][:kept]
    assert kept == len(toks), "forced cases chosen where n_predict does not cut the last cycle"
    m = O.Model(path, int(z["n_ctx"]))
    seq = np.concatenate([z["prompt"], toks]).astype(np.uint32)
    for i, t in enumerate(seq):
        lg = m.forward(int(t), i)
    assert np.array_equal(lg.view(np.uint32), z[key + "_last"].view(np.uint32))
