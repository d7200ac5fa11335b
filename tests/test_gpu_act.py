"""GPU parity of the activation transforms fused into the GEMV input preparation
(qgpu_gemv_act_batch): RMSNorm, two-segment RMSNorm (MTP input), SiLU*up and
per-head gated RMSNorm, against the oracle's ops (pinned to the reference)
followed by the oracle's GEMV.  Bars: GEMV outputs within 1e-3 normwise; the
transformed fp32 rows (xout) within 1e-5.  Single-segment RMSNorm applies its
row factor to the GEMV output, so its xout holds x * w.

Also the K-split GEMV of narrow outputs: partial planes (qgpu_gemv_act_split)
summed by qgpu_add_partials or by the next RMSNorm preparation, which writes
the summed residual back in place, for every format of the matrix-core GEMV."""
import ctypes

import numpy as np
import pytest

import oracle_lib as O
from gpu_util import gpu, rel_err  # noqa: F401
from qwen_pkg import host_lib, pyqwen

pytestmark = pytest.mark.gpu
EPS = 1e-6


def o_rmsnorm(x, w):
    out = np.zeros_like(x)
    O.lib().or_rmsnorm(O.fptr(out), O.fptr(np.ascontiguousarray(x)), O.fptr(w), x.size, EPS)
    return out


def o_silu(x):
    y = np.ascontiguousarray(x, np.float32).copy()
    O.lib().or_silu_inplace(O.fptr(y), y.size)
    return y


def run(gpu, t, W, ne0, ne1, act, B, bufs):
    """one qgpu_gemv_act_batch call; returns (out, xout)"""
    T = gpu.tensor(W, t, ne0, ne1)
    ob = gpu.buf(B * ne1 * 4)
    xo = gpu.buf(B * ne0 * 4)
    act.xout, act.ldxo = xo.f32(), ne0
    Ws = (ctypes.c_void_p * 1)(T.h)
    outs = (pyqwen.F32P * 1)(ob.f32())
    lds = (ctypes.c_uint64 * 1)(ne1)
    gpu.ok(gpu.L.qgpu_gemv_act_batch(Ws, 1, ctypes.byref(act), B, outs, lds, 0))
    r = ob.download(np.float32).reshape(B, ne1), xo.download(np.float32).reshape(B, ne0)
    del bufs
    return r


@pytest.mark.parametrize("t", [23, 12, 14, 0])   # IQ4_XS, Q4_K, Q6_K (matrix-core digit path), F32 (VALU path via xout)
@pytest.mark.parametrize("B", [1, 4, 7])
@pytest.mark.parametrize("kind", ["rmsnorm", "rmsnorm2", "silu_mul", "gated"])
def test_act_transform_gemv(gpu, t, B, kind):
    print(f"\n[act] {kind} type={t} B={B}", flush=True)
    host = host_lib()
    ne0, ne1 = 1024, 384
    W = host.synth_matrix(t, ne0, ne1, 11, t, 0.02)
    rng = np.random.default_rng(B * 10 + t)
    x = (rng.standard_normal((B, ne0)) * 3).astype(np.float32)
    y = rng.standard_normal((B, ne0)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(ne0)).astype(np.float32)
    w2 = (1 + 0.1 * rng.standard_normal(ne0)).astype(np.float32)
    xb, yb, wb, w2b = gpu.put(x), gpu.put(y), gpu.put(w), gpu.put(w2)
    a = pyqwen.Act()
    a.x, a.ldx, a.eps = xb.f32(), ne0, EPS
    xo_ref = None
    if kind == "rmsnorm":
        a.kind, a.w = pyqwen.ACT_RMSNORM, wb.f32()
        xin = np.stack([o_rmsnorm(x[b], w) for b in range(B)])
        xo_ref = x * w                                 # row factor applied to the GEMV output
    elif kind == "rmsnorm2":                          # [x | y] halves, each with its own row norm
        h = ne0 // 2
        xs, ys = np.ascontiguousarray(x[:, :h]), np.ascontiguousarray(y[:, :h])
        xb, yb = gpu.put(xs), gpu.put(ys)
        a.x, a.ldx, a.y, a.ldy = xb.f32(), h, yb.f32(), h
        a.kind, a.w, a.w2, a.seg = pyqwen.ACT_RMSNORM, wb.f32(), w2b.f32(), h
        xin = np.stack([np.concatenate([o_rmsnorm(xs[b], w[:h]), o_rmsnorm(ys[b], w2[:h])]) for b in range(B)])
    elif kind == "silu_mul":
        a.kind, a.y, a.ldy = pyqwen.ACT_SILU_MUL, yb.f32(), ne0
        xin = o_silu(x) * y
    else:
        hd = 128
        a.kind, a.y, a.ldy, a.w, a.seg = pyqwen.ACT_GATED_NORM, yb.f32(), ne0, wb.f32(), hd
        xin = np.zeros_like(x)
        for b in range(B):
            for hh in range(ne0 // hd):
                sl = slice(hh * hd, (hh + 1) * hd)
                xin[b, sl] = o_rmsnorm(x[b, sl], w[:hd]) * o_silu(y[b, sl])
    out, xo = run(gpu, t, W, ne0, ne1, a, B, (xb, yb, wb, w2b))
    ex = rel_err(xo, xin if xo_ref is None else xo_ref)
    ref = O.gemv(t, W, ne0, ne1, xin, B)
    eo = rel_err(out, ref)
    print(f"  xout {ex:.2e}  gemv {eo:.2e}", flush=True)
    assert ex < 1e-5 and eo < 1e-3


@pytest.mark.parametrize("t", [23, 12, 8])          # IQ4_XS, Q4_K, Q8_0 (the 27B eh_proj formats)
@pytest.mark.parametrize("B", [1, 4, 7])
@pytest.mark.parametrize("shape,gather", [((1024, 384), False), ((1024, 384), True), ((2048, 4352), False)])
def test_act_two_segment_deferred(gpu, t, B, shape, gather):
    """The MTP input concat(enorm(e), hnorm(h)) without an fp32 copy (xout NULL): the preparation writes
    [x*w | y*w2] and per-super-block sums of squares, and the matrix-core GEMV sums each half's super-blocks
    apart and applies each half's row factor.  Against the oracle GEMV of the normalised rows (bar 1e-3
    normwise) and against the same call with xout (normalised digits, one factor per element): the two
    agree to the GEMV's rounding.  4352 rows = 272 tiles: the pair-split tail, whose halves are exactly the
    two segments.  gather: the first half from embedding rows (IQ4_XS), as the model's MTP input."""
    print(f"\n[act2] type={t} B={B} shape={shape} gather={gather}", flush=True)
    host = host_lib()
    ne0, ne1 = shape
    h = ne0 // 2
    W = host.synth_matrix(t, ne0, ne1, 13, t, 0.02)
    T = gpu.tensor(W, t, ne0, ne1)
    rng = np.random.default_rng(100 * B + t)
    ys = rng.standard_normal((B, h)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    w2 = (1 + 0.1 * rng.standard_normal(h)).astype(np.float32)
    yb, wb, w2b = gpu.put(ys), gpu.put(w), gpu.put(w2)
    if gather:
        V = 300
        Te = gpu.tensor(host.synth_matrix(23, h, V, 41, 7, 0.5), 23, h, V)
        tb = gpu.put(rng.integers(0, V, B).astype(np.uint32))
        xr = gpu.buf(B * h * 4)
        gpu.ok(gpu.L.qgpu_dequant_rows(Te.h, tb.u32(), B, xr.f32(), h))
        xs = xr.download(np.float32).reshape(B, h)
    else:
        xs = (rng.standard_normal((B, h)) * 3).astype(np.float32)
        xb = gpu.put(xs)
    xin = np.stack([np.concatenate([o_rmsnorm(xs[b], w), o_rmsnorm(ys[b], w2)]) for b in range(B)])

    def call(with_xout):
        a = pyqwen.Act()
        a.kind, a.w, a.w2, a.seg, a.eps = pyqwen.ACT_RMSNORM, wb.f32(), w2b.f32(), h, EPS
        a.y, a.ldy, a.ldx = yb.f32(), h, h
        if gather:
            a.embd, a.tok = Te.h, tb.u32()
        else:
            a.x = xb.f32()
        xo = gpu.buf(B * ne0 * 4)
        if with_xout:
            a.xout, a.ldxo = xo.f32(), ne0
        ob = gpu.buf(B * ne1 * 4)
        gpu.ok(gpu.L.qgpu_gemv_act_batch((ctypes.c_void_p * 1)(T.h), 1, ctypes.byref(a), B,
                                         (pyqwen.F32P * 1)(ob.f32()), (ctypes.c_uint64 * 1)(ne1), 0))
        return ob.download(np.float32).reshape(B, ne1)

    got, with_xo = call(False), call(True)
    ref = O.gemv(t, W, ne0, ne1, xin, B)
    e, e2, d = rel_err(got, ref), rel_err(with_xo, ref), rel_err(got, with_xo)
    print(f"  deferred {e:.2e}  with xout {e2:.2e}  between {d:.2e}", flush=True)
    assert e < 1e-3 and e2 < 1e-3 and d < 1e-5
    assert np.array_equal(got, call(False))            # deterministic


def test_act_rejects_bad_args(gpu):
    host = host_lib()
    W = host.synth_matrix(23, 512, 32, 3, 3, 0.02)
    T = gpu.tensor(W, 23, 512, 32)
    xb, ob, wb = gpu.buf(4 * 512 * 2), gpu.buf(4 * 32 * 2), gpu.buf(4 * 512)
    Ws = (ctypes.c_void_p * 1)(T.h)
    outs = (pyqwen.F32P * 1)(ob.f32())
    lds = (ctypes.c_uint64 * 1)(32)
    a = pyqwen.Act()
    a.kind, a.x, a.ldx, a.eps = pyqwen.ACT_RMSNORM, xb.f32(), 512, EPS
    assert gpu.L.qgpu_gemv_act_batch(Ws, 1, ctypes.byref(a), 2, outs, lds, 0) != 0      # no weight
    a.w, a.seg = wb.f32(), 128                                                             # seg not ne0 or ne0/2
    assert gpu.L.qgpu_gemv_act_batch(Ws, 1, ctypes.byref(a), 2, outs, lds, 0) != 0
    a.kind, a.seg, a.y, a.ldy = pyqwen.ACT_GATED_NORM, 96, xb.f32(), 512                   # head size 96
    assert gpu.L.qgpu_gemv_act_batch(Ws, 1, ctypes.byref(a), 2, outs, lds, 0) != 0
    a.kind = 9
    assert gpu.L.qgpu_gemv_act_batch(Ws, 1, ctypes.byref(a), 2, outs, lds, 0) != 0
    gpu.sync()


def _split(gpu, T, a, B, ne1, ks):
    pb = gpu.buf(ks * B * ne1 * 4)
    gpu.ok(gpu.L.qgpu_gemv_act_split(T.h, ctypes.byref(a), B, pb.f32(), ne1, ks))
    return pb, pb.download(np.float32).reshape(ks, B, ne1)


@pytest.mark.parametrize("t", [23, 12, 13, 14, 8])     # every format of the matrix-core GEMV
@pytest.mark.parametrize("B", [1, 4, 6])
def test_split_gemv_partials(gpu, t, B):
    """K-split planes of a narrow GEMV sum to the oracle GEMV; qgpu_add_partials adds them in order."""
    print(f"\n[split] type={t} B={B}", flush=True)
    host = host_lib()
    ne0, ne1 = 5120, 320
    W = host.synth_matrix(t, ne0, ne1, 21, 4, 0.02)
    T = gpu.tensor(W, t, ne0, ne1)
    ks = gpu.L.qgpu_gemv_split_ks(T.h)
    assert 2 <= ks <= 8
    x = np.random.default_rng(B).standard_normal((B, ne0)).astype(np.float32)
    xb = gpu.put(x)
    a = pyqwen.Act()
    a.kind, a.x, a.ldx = pyqwen.ACT_COPY, xb.f32(), ne0
    pb, planes = _split(gpu, T, a, B, ne1, ks)
    ref = O.gemv(t, W, ne0, ne1, x, B)
    e = rel_err(planes.sum(0), ref)
    print(f"  ks={ks} rel err {e:.2e}", flush=True)
    assert e < 2e-5
    # y = r + (p0 + p1 + ...), in place
    r = np.random.default_rng(B + 50).standard_normal((B, ne1)).astype(np.float32)
    rb = gpu.put(r)
    gpu.ok(gpu.L.qgpu_add_partials(rb.f32(), ne1, rb.f32(), ne1, pb.f32(), ne1, ks, ne1, B))
    ps = planes[0].copy()
    for q in range(1, ks):
        ps = (ps + planes[q]).astype(np.float32)
    assert np.array_equal(rb.download(np.float32).reshape(B, ne1), (r + ps).astype(np.float32))


@pytest.mark.parametrize("tp", [23, 14])                 # producer format
@pytest.mark.parametrize("tc", [23, 13, 8])              # consumer format (deferred row factor in the epilogue)
@pytest.mark.parametrize("B", [1, 4, 7])
def test_rmsnorm_consumes_partials(gpu, tp, tc, B):
    """The residual's pending partial planes are added by the next RMSNorm preparation (written back in
    place) and the GEMV that follows sees rmsnorm(R + sum of planes)."""
    print(f"\n[rms-partials] producer={tp} consumer={tc} B={B}", flush=True)
    host = host_lib()
    E, n_out = 1024, 384
    Wd = host.synth_matrix(tp, 4096, E, 31, 5, 0.02)          # narrow producer: 4096 -> 1024 (64 tiles)
    Td = gpu.tensor(Wd, tp, 4096, E)
    Wn = host.synth_matrix(tc, E, n_out, 32, 6, 0.02)          # consumer: 1024 -> 384
    Tn = gpu.tensor(Wn, tc, E, n_out)
    rng = np.random.default_rng(100 + B)
    h = rng.standard_normal((B, 4096)).astype(np.float32)
    R = (3 * rng.standard_normal((B, E))).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    hb, Rb, wb = gpu.put(h), gpu.put(R), gpu.put(w)
    a = pyqwen.Act()
    a.kind, a.x, a.ldx = pyqwen.ACT_COPY, hb.f32(), 4096
    ks = gpu.L.qgpu_gemv_split_ks(Td.h)
    assert ks > 1
    pb, planes = _split(gpu, Td, a, B, E, ks)
    ps = planes[0].copy()
    for q in range(1, ks):
        ps = (ps + planes[q]).astype(np.float32)
    R_new = (R + ps).astype(np.float32)
    an = pyqwen.Act()
    an.kind, an.x, an.ldx, an.w, an.eps = pyqwen.ACT_RMSNORM, Rb.f32(), E, wb.f32(), EPS
    an.part, an.ldp, an.n_part, an.xnew, an.ldxn = pb.f32(), E, ks, Rb.f32(), E
    ob = gpu.buf(B * n_out * 4)
    Ws = (ctypes.c_void_p * 1)(Tn.h)
    outs = (pyqwen.F32P * 1)(ob.f32())
    lds = (ctypes.c_uint64 * 1)(n_out)
    gpu.ok(gpu.L.qgpu_gemv_act_batch(Ws, 1, ctypes.byref(an), B, outs, lds, 0))
    assert np.array_equal(Rb.download(np.float32).reshape(B, E), R_new)
    xin = np.stack([o_rmsnorm(R_new[b], w) for b in range(B)])
    e = rel_err(ob.download(np.float32).reshape(B, n_out), O.gemv(tc, Wn, E, n_out, xin, B))
    print(f"  ks={ks} gemv rel err {e:.2e}", flush=True)
    assert e < 1e-4
    # partial planes are rejected by every transform but single-segment RMSNorm
    a2 = pyqwen.Act()
    a2.kind, a2.x, a2.ldx, a2.part, a2.ldp, a2.n_part = pyqwen.ACT_COPY, Rb.f32(), E, pb.f32(), E, ks
    assert gpu.L.qgpu_gemv_act_batch(Ws, 1, ctypes.byref(a2), B, outs, lds, 0) != 0
    gpu.sync()


@pytest.mark.parametrize("B", [1, 4, 8])
def test_act_batch_ks_planes(gpu, B):
    """qgpu_gemv_act_batch_ks, the grouped GEMV with a K split per matrix (the GDN input projection cuts
    its two narrow gate matrices so): matrices with ks = 1 give the outputs of qgpu_gemv_act_batch bit
    for bit; a matrix with ks > 1 gives ks partial planes whose sum (in plane order) is the oracle GEMV of
    the RMSNorm input within 1e-3, and qgpu_gemv_act_batch's output within 2e-5 (the deferred row factor
    applies to every plane).  Mixed formats: one launch per format, each with its own split."""
    print(f"\n[act-ks] B={B}", flush=True)
    host = host_lib()
    E = 2048
    mats = [(23, 384, 1), (14, 256, 1), (23, 48, 8), (8, 48, 3)]       # (type, rows, K ranges)
    Ws_h = [host.synth_matrix(t, E, r, 41 + i, t, 0.02) for i, (t, r, _) in enumerate(mats)]
    Ts = [gpu.tensor(W, t, E, r) for W, (t, r, _) in zip(Ws_h, mats)]
    rng = np.random.default_rng(70 + B)
    x = (rng.standard_normal((B, E)) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    xb, wb = gpu.put(x), gpu.put(w)
    a = pyqwen.Act()
    a.kind, a.x, a.ldx, a.w, a.eps = pyqwen.ACT_RMSNORM, xb.f32(), E, wb.f32(), EPS
    n = len(mats)
    Ws = (ctypes.c_void_p * n)(*[T.h for T in Ts])
    lds = (ctypes.c_uint64 * n)(*[r for _, r, _ in mats])
    plain = [gpu.buf(B * r * 4) for _, r, _ in mats]
    split = [gpu.buf(k * B * r * 4) for _, r, k in mats]
    gpu.ok(gpu.L.qgpu_gemv_act_batch(Ws, n, ctypes.byref(a), B, (pyqwen.F32P * n)(*[b.f32() for b in plain]),
                                     lds, 0))
    ks = (ctypes.c_int * n)(*[k for _, _, k in mats])
    gpu.ok(gpu.L.qgpu_gemv_act_batch_ks(Ws, n, ctypes.byref(a), B, (pyqwen.F32P * n)(*[b.f32() for b in split]),
                                        lds, ks))
    xin = np.stack([o_rmsnorm(x[b], w) for b in range(B)])
    for j, (t, r, k) in enumerate(mats):
        p = plain[j].download(np.float32).reshape(B, r)
        s = split[j].download(np.float32).reshape(k, B, r)
        if k == 1:
            assert np.array_equal(s[0], p), j
            continue
        tot = s[0].copy()
        for q in range(1, k):
            tot = (tot + s[q]).astype(np.float32)
        e_or = rel_err(tot, O.gemv(t, Ws_h[j], E, r, xin, B))
        e_pl = rel_err(tot, p)
        print(f"  matrix {j} type {t} ks={k}: vs oracle {e_or:.2e}, vs unsplit {e_pl:.2e}", flush=True)
        assert e_or < 1e-3 and e_pl < 2e-5, (j, e_or, e_pl)
    # rejected: a K range count of 0, above 32 or above the super-blocks of a row, a split of an fp32 matrix
    for bad in ([1, 1, 0, 1], [1, 1, 33, 1], [1, 1, 9, 1]):
        kb = (ctypes.c_int * n)(*bad)
        assert gpu.L.qgpu_gemv_act_batch_ks(Ws, n, ctypes.byref(a), B,
                                            (pyqwen.F32P * n)(*[b.f32() for b in split]), lds, kb) != 0, bad
    Wf = host.synth_matrix(0, E, 48, 49, 0, 0.02)
    Tf = gpu.tensor(Wf, 0, E, 48)
    Wf_s = (ctypes.c_void_p * 1)(Tf.h)
    assert gpu.L.qgpu_gemv_act_batch_ks(Wf_s, 1, ctypes.byref(a), B, (pyqwen.F32P * 1)(split[2].f32()),
                                        (ctypes.c_uint64 * 1)(48), (ctypes.c_int * 1)(2)) != 0
    gpu.sync()


@pytest.mark.parametrize("form", ["single", "two_segment"])
@pytest.mark.parametrize("B", [1, 4, 8])
def test_rmsnorm_embedding_gather(gpu, form, B):
    """RMSNorm whose rows are gathered from a packed IQ4_XS embedding (embd, tok) gives the bits of
    qgpu_dequant_rows followed by the same transform: GEMV outputs, xout, and (single segment, the
    first preparation of a forward) the rows written to xnew; an id past the last row is a zero row."""
    print(f"\n[embd-gather] {form} B={B}", flush=True)
    host = host_lib()
    E, V, n_out = 1024, 300, 384
    Te = gpu.tensor(host.synth_matrix(23, E, V, 41, 7, 0.5), 23, E, V)
    ne0 = E if form == "single" else 2 * E
    Tn = gpu.tensor(host.synth_matrix(23, ne0, n_out, 42, 8, 0.02), 23, ne0, n_out)
    rng = np.random.default_rng(B)
    tok = rng.integers(0, V, B).astype(np.uint32)
    if B > 1:
        tok[-1] = V + 5
    tb = gpu.put(tok)
    xr = gpu.buf(B * E * 4)
    gpu.ok(gpu.L.qgpu_dequant_rows(Te.h, tb.u32(), B, xr.f32(), E))
    w = (1 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    w2 = (1 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    h = rng.standard_normal((B, E)).astype(np.float32)
    wb, w2b, hb = gpu.put(w), gpu.put(w2), gpu.put(h)

    def call(gather):
        a = pyqwen.Act()
        a.kind, a.ldx, a.w, a.eps = pyqwen.ACT_RMSNORM, E, wb.f32(), EPS
        if gather:
            a.embd, a.tok = Te.h, tb.u32()
        else:
            a.x = xr.f32()
        if form == "two_segment":
            a.y, a.ldy, a.w2, a.seg = hb.f32(), E, w2b.f32(), E
        xo, ob = gpu.buf(B * ne0 * 4), gpu.buf(B * n_out * 4)
        a.xout, a.ldxo = xo.f32(), ne0
        xn = gpu.buf(B * E * 4)
        if form == "single":
            a.xnew, a.ldxn = xn.f32(), E
        gpu.ok(gpu.L.qgpu_gemv_act_batch((ctypes.c_void_p * 1)(Tn.h), 1, ctypes.byref(a), B,
                                         (pyqwen.F32P * 1)(ob.f32()), (ctypes.c_uint64 * 1)(n_out), 0))
        return ob.download(np.float32), xo.download(np.float32), xn.download(np.float32)

    plain, gath = call(False), call(True)
    assert np.array_equal(gath[0], plain[0]) and np.array_equal(gath[1], plain[1])
    rows = xr.download(np.float32).reshape(B, E)
    if form == "single":
        assert np.array_equal(gath[2].reshape(B, E), rows)
    if B > 1:
        assert not rows[-1].any()
    assert np.isfinite(plain[0]).all() and np.abs(plain[0]).max() > 0
    if form == "two_segment":        # an embedding narrower than the single-segment row: rejected
        a = pyqwen.Act()
        a.kind, a.w, a.eps, a.embd, a.tok = pyqwen.ACT_RMSNORM, wb.f32(), EPS, Te.h, tb.u32()
        assert gpu.L.qgpu_gemv_act_batch((ctypes.c_void_p * 1)(Tn.h), 1, ctypes.byref(a), B,
                                         (pyqwen.F32P * 1)(gpu.buf(B * n_out * 4).f32()),
                                         (ctypes.c_uint64 * 1)(n_out), 0) != 0
    gpu.sync()
