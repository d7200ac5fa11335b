"""GPU parity of the Gated DeltaNet block, the gated GQA attention and the whole
hybrid model (batched verify, single-token decode, MTP draft, rollback and the
on-device greedy speculative loop), through the C-ABI (libqgpu) and the
reference-compatible model API (libqwen).

Checkers: the oracle (CPU restatement, bit-exact with the reference) and the
golden vectors produced from the compiled reference (tests/golden).
Bars: GEMV/GDN outputs within 1e-3 relative (normwise, max|d|/max|ref|);
greedy token streams identical wherever the reference top-2 gap > 1e-2 (every
gap of the fixtures is above 0.3, so the streams must be identical).
"""
import ctypes
import hashlib
import os
import tempfile
import time

import numpy as np
import pytest

import oracle_lib as O
from gpu_util import gpu, rel_err  # noqa: F401
from qwen_pkg import host_lib, pyqwen

pytestmark = pytest.mark.gpu
NSLOT = 9


def load(name):
    return np.load(os.path.join(O.GOLDEN, name), allow_pickle=False)


# ---------------------------------------------------------------- GDN block (config 3)
@pytest.mark.parametrize("fused", [False, True])
def test_gdn_block_config3_vs_oracle_with_snapshots_and_rollback(gpu, fused):
    print(f"\n[gdn] config 3: 48 v-heads x 128x128, 16 k-heads, T=4, fused={fused}", flush=True)
    T, nk, nv, hk = 4, 16, 48, 128
    cd, eps = 2 * nk * hk + nv * hk, 1e-6
    host = host_lib()
    qkv = host.synth_normal(T * cd, 3, 1).reshape(T, cd)
    br = host.synth_normal(T * nv, 3, 2).reshape(T, nv)
    ar = host.synth_normal(T * nv, 3, 3).reshape(T, nv)
    cw = host.synth_normal(cd * 4, 3, 4, 0.0, 0.5)
    conv0 = host.synth_normal(cd * 4, 3, 5, 0.0, 0.5)
    ssm0 = host.synth_normal(nv * hk * hk, 3, 6, 0.0, 0.01)
    dtb = np.zeros(nv, np.float32)
    sa = -np.ones(nv, np.float32)
    # oracle
    L = O.lib()
    oc, os_ = conv0.copy(), ssm0.copy()
    oout = np.zeros(T * nv * hk, np.float32)
    snap_c = np.zeros(T * cd * 4, np.float32)
    snap_s = np.zeros(T * nv * hk * hk, np.float32)
    L.or_gdn_block(T, cd, nk, nv, hk, hk, eps, O.fptr(qkv), O.fptr(br), O.fptr(ar), O.fptr(cw), O.fptr(dtb),
                   O.fptr(sa), O.fptr(oc), O.fptr(os_), O.fptr(oout), O.fptr(snap_c), O.fptr(snap_s))
    # GPU: ring of NSLOT slots, current slot 5 (exercises the wrap-around)
    cur0 = 5
    cstride, sstride = cd * 4, nv * hk * hk
    cring = gpu.put(np.zeros(NSLOT * cstride, np.float32))
    sring = gpu.put(np.zeros(NSLOT * sstride, np.float32))
    cring.upload(conv0, cur0 * cstride * 4)
    sring.upload(ssm0, cur0 * sstride * 4)
    curb = gpu.put(np.array([cur0], np.int32))
    xb, yb, cwb = gpu.put(qkv), gpu.buf(T * cd * 4), gpu.put(cw)
    dtbb, sab = gpu.put(dtb), gpu.put(sa)
    ob = gpu.buf(T * nv * hk * 4)
    bb, ab = gpu.put(br), gpu.put(ar)

    def run(xbuf, ntok, bbuf, abuf):
        if fused:
            gpu.ok(gpu.L.qgpu_gdn_fused(xbuf.f32(), cd, ntok, cd, cwb.f32(), cring.f32(), cstride, bbuf.f32(),
                                        abuf.f32(), nv, dtbb.f32(), sab.f32(), sring.f32(), sstride, NSLOT,
                                        curb.i32(), nk, nv, hk, eps, ob.f32(), nv * hk))
        else:
            gpu.ok(gpu.L.qgpu_gdn_conv(xbuf.f32(), cd, ntok, cd, cwb.f32(), cring.f32(), cstride, NSLOT, curb.i32(),
                                       yb.f32(), cd))
            gpu.ok(gpu.L.qgpu_gdn_recurrence(yb.f32(), cd, bbuf.f32(), abuf.f32(), nv, dtbb.f32(), sab.f32(),
                                             sring.f32(), sstride, NSLOT, curb.i32(), ntok, nk, nv, hk, eps, ob.f32(),
                                             nv * hk))
    run(xb, T, bb, ab)
    got = ob.download(np.float32).reshape(T, -1)
    for b in range(T):
        e = rel_err(got[b], oout.reshape(T, -1)[b])
        print(f"  token {b}: output rel err {e:.2e}", flush=True)
        assert e < 1e-3, (b, e)
    cr = cring.download(np.float32).reshape(NSLOT, -1)
    sr = sring.download(np.float32).reshape(NSLOT, -1)
    assert np.array_equal(cr[cur0], conv0) and np.array_equal(sr[cur0], ssm0), "current slot must not be written"
    for b in range(T):
        slot = (cur0 + 1 + b) % NSLOT
        ec, es = rel_err(cr[slot], snap_c.reshape(T, -1)[b]), rel_err(sr[slot], snap_s.reshape(T, -1)[b])
        print(f"  snapshot {b} in slot {slot}: conv {ec:.2e} state {es:.2e}", flush=True)
        assert ec == 0.0 and es < 1e-3, (b, ec, es)
    # rollback to accepted position 2 = pointer select, then one more token continues from there
    gpu.ok(gpu.L.qgpu_set_i32(curb.i32(), (cur0 + 1 + 2) % NSLOT))
    x1 = host.synth_normal(cd, 3, 7).reshape(1, cd)
    b1, a1 = host.synth_normal(nv, 3, 8), host.synth_normal(nv, 3, 9)
    x1b, b1b, a1b = gpu.put(x1), gpu.put(b1), gpu.put(a1)
    run(x1b, 1, b1b, a1b)
    oc2 = snap_c.reshape(T, -1)[2].copy()
    os2 = snap_s.reshape(T, -1)[2].copy()
    o2 = np.zeros(nv * hk, np.float32)
    L.or_gdn_block(1, cd, nk, nv, hk, hk, eps, O.fptr(x1), O.fptr(b1), O.fptr(a1), O.fptr(cw), O.fptr(dtb),
                   O.fptr(sa), O.fptr(oc2), O.fptr(os2), O.fptr(o2), None, None)
    assert rel_err(ob.download(np.float32, nv * hk), o2) < 1e-3


@pytest.mark.parametrize("planes", [1, 3, 20])
def test_gdn_fused_gate_planes(gpu, planes):
    """qgpu_gdn_fused_planes: the gate inputs (beta, alpha) given as partial planes, summed in plane order
    per (token, head), give the outputs and the state/conv snapshots of qgpu_gdn_fused on the summed
    inputs bit for bit, and the oracle's within 1e-3 (config-3 shapes, T = 4)."""
    print(f"\n[gdn-planes] {planes} gate planes", flush=True)
    T, nk, nv, hk = 4, 16, 48, 128
    cd, eps = 2 * nk * hk + nv * hk, 1e-6
    host = host_lib()
    qkv = host.synth_normal(T * cd, 4, 1).reshape(T, cd)
    cw = host.synth_normal(cd * 4, 4, 4, 0.0, 0.5)
    conv0 = host.synth_normal(cd * 4, 4, 5, 0.0, 0.5)
    ssm0 = host.synth_normal(nv * hk * hk, 4, 6, 0.0, 0.01)
    dtb = np.full(nv, 0.1, np.float32)
    sa = -np.ones(nv, np.float32)
    rng = np.random.default_rng(planes)
    bp = (rng.standard_normal((planes, T, nv)) / np.sqrt(planes)).astype(np.float32)
    ap = (rng.standard_normal((planes, T, nv)) / np.sqrt(planes)).astype(np.float32)

    def psum(p):
        s = p[0].copy()
        for q in range(1, len(p)):
            s = (s + p[q]).astype(np.float32)
        return s
    br, ar = psum(bp), psum(ap)
    L = O.lib()
    oc, os_ = conv0.copy(), ssm0.copy()
    oout = np.zeros(T * nv * hk, np.float32)
    L.or_gdn_block(T, cd, nk, nv, hk, hk, eps, O.fptr(qkv), O.fptr(br), O.fptr(ar), O.fptr(cw), O.fptr(dtb),
                   O.fptr(sa), O.fptr(oc), O.fptr(os_), O.fptr(oout), None, None)
    cur0 = 2
    cstride, sstride = cd * 4, nv * hk * hk
    cring = gpu.put(np.zeros(NSLOT * cstride, np.float32))
    sring = gpu.put(np.zeros(NSLOT * sstride, np.float32))
    cring.upload(conv0, cur0 * cstride * 4)
    sring.upload(ssm0, cur0 * sstride * 4)
    curb = gpu.put(np.array([cur0], np.int32))
    xb, cwb, dtbb, sab = gpu.put(qkv), gpu.put(cw), gpu.put(dtb), gpu.put(sa)
    ob = gpu.buf(T * nv * hk * 4)
    # summed inputs through qgpu_gdn_fused (the current slot is read, never written: both runs start there)
    bb, ab = gpu.put(br), gpu.put(ar)
    gpu.ok(gpu.L.qgpu_gdn_fused(xb.f32(), cd, T, cd, cwb.f32(), cring.f32(), cstride, bb.f32(), ab.f32(), nv,
                                dtbb.f32(), sab.f32(), sring.f32(), sstride, NSLOT, curb.i32(), nk, nv, hk, eps,
                                ob.f32(), nv * hk))
    o1 = ob.download(np.float32)
    c1, s1 = cring.download(np.float32), sring.download(np.float32)
    bpb, apb = gpu.put(bp), gpu.put(ap)
    gpu.ok(gpu.L.qgpu_gdn_fused_planes(xb.f32(), cd, T, cd, cwb.f32(), cring.f32(), cstride, bpb.f32(), apb.f32(),
                                       nv, planes, T * nv, dtbb.f32(), sab.f32(), sring.f32(), sstride, NSLOT,
                                       curb.i32(), nk, nv, hk, eps, ob.f32(), nv * hk))
    o2 = ob.download(np.float32)
    assert np.array_equal(o1, o2)
    assert np.array_equal(c1, cring.download(np.float32)) and np.array_equal(s1, sring.download(np.float32))
    e = rel_err(o2, oout)
    print(f"  output vs oracle {e:.2e}", flush=True)
    assert e < 1e-3
    # plane counts outside 1..32, or 32 planes of 9 tokens (> 256 gate loads), are rejected
    for npl in (0, 33):
        assert gpu.L.qgpu_gdn_fused_planes(xb.f32(), cd, T, cd, cwb.f32(), cring.f32(), cstride, bpb.f32(),
                                           apb.f32(), nv, npl, T * nv, dtbb.f32(), sab.f32(), sring.f32(), sstride,
                                           NSLOT, curb.i32(), nk, nv, hk, eps, ob.f32(), nv * hk) != 0, npl
    assert gpu.L.qgpu_gdn_fused_planes(xb.f32(), cd, T, cd, cwb.f32(), cring.f32(), cstride, bpb.f32(), apb.f32(),
                                       nv, 2, T * nv - 1, dtbb.f32(), sab.f32(), sring.f32(), sstride, NSLOT,
                                       curb.i32(), nk, nv, hk, eps, ob.f32(), nv * hk) != 0   # planes overlap
    gpu.sync()

@pytest.mark.parametrize("seq", [((8, 3), (8, 7), (1, 0)), ((6, 5), (4, 0), (8, 2)), ((5, 0), (5, 4), (3, 1)),
                                 ((8, 7), (8, 7), (8, 7))])
def test_gdn_factor_form_equals_snapshots(gpu, seq):
    """qgpu_gdn_fused_factor: three calls (B tokens, then a rollback to the state after token j), the first two
    keeping the state in rank-1 factor form and the third taking snapshots, give the outputs of every call, the
    third call's state snapshots and the conv snapshots of the snapshot-only sequence (qgpu_gdn_fused_planes)
    bit for bit; qgpu_gdn_materialize after the second call writes the state the snapshot sequence selects.
    Config-3 shapes (48 v-heads, 16 k-heads, 128x128 states); ring slots wrap around."""
    print(f"\n[gdn-factor] calls (B, j): {seq}", flush=True)
    nk, nv, hk = 16, 48, 128
    cd, eps = 2 * nk * hk + nv * hk, 1e-6
    host = host_lib()
    cw = host.synth_normal(cd * 4, 5, 4, 0.0, 0.5)
    conv0 = host.synth_normal(cd * 4, 5, 5, 0.0, 0.5)
    ssm0 = host.synth_normal(nv * hk * hk, 5, 6, 0.0, 0.01)
    dtb = np.full(nv, 0.1, np.float32)
    sa = -np.ones(nv, np.float32)
    cstride, sstride = cd * 4, nv * hk * hk
    ftok = ((nv + nk) * hk + nv + 3) // 4 * 4
    cwb, dtbb, sab = gpu.put(cw), gpu.put(dtb), gpu.put(sa)
    cur0 = 6
    rings = []
    for _ in range(2):
        cring = gpu.put(np.zeros(NSLOT * cstride, np.float32))
        sring = gpu.put(np.zeros(NSLOT * sstride, np.float32))
        cring.upload(conv0, cur0 * cstride * 4)
        sring.upload(ssm0, cur0 * sstride * 4)
        rings.append((cring, sring))
    fbuf = gpu.put(np.zeros(2 * 8 * ftok, np.float32))
    fst = gpu.put(np.zeros(2, np.int32))
    curs = [gpu.put(np.array([cur0], np.int32)) for _ in range(2)]
    ob = gpu.buf(8 * nv * hk * 4)
    cur, pend, par = cur0, 0, 0
    for call, (B, j) in enumerate(seq):
        x = host.synth_normal(B * cd, 6, call).reshape(B, cd)
        br = host.synth_normal(B * nv, 6, 10 + call).reshape(B, nv)
        ar = host.synth_normal(B * nv, 6, 20 + call).reshape(B, nv)
        xb, bb, ab = gpu.put(x), gpu.put(br), gpu.put(ar)
        cring, sring = rings[0]
        gpu.ok(gpu.L.qgpu_gdn_fused_planes(xb.f32(), cd, B, cd, cwb.f32(), cring.f32(), cstride, bb.f32(), ab.f32(), nv,
                                           1, 0, dtbb.f32(), sab.f32(), sring.f32(), sstride, NSLOT, curs[0].i32(), nk,
                                           nv, hk, eps, ob.f32(), nv * hk))
        o_snap = ob.download(np.float32, B * nv * hk)
        factor = call < 2
        fst.upload(np.array([pend, par], np.int32))
        cring, sring = rings[1]
        gpu.ok(gpu.L.qgpu_gdn_fused_factor(xb.f32(), cd, B, cd, cwb.f32(), cring.f32(), cstride, bb.f32(), ab.f32(),
                                           nv, 1, 0, dtbb.f32(), sab.f32(), sring.f32(), sstride, NSLOT, curs[1].i32(),
                                           nk, nv, hk, eps, ob.f32(), nv * hk, fbuf.f32(), ftok, fst.i32(),
                                           1 if factor else 0))
        o_fac = ob.download(np.float32, B * nv * hk)
        assert np.array_equal(o_snap, o_fac), f"call {call}: outputs differ"
        # conv snapshots are written in both forms
        ca, cb = rings[0][0].download(np.float32).reshape(NSLOT, -1), rings[1][0].download(np.float32).reshape(NSLOT, -1)
        for b in range(B):
            assert np.array_equal(ca[(cur + 1 + b) % NSLOT], cb[(cur + 1 + b) % NSLOT]), (call, b)
        if factor:
            pend, par = j + 1, par ^ 1
        else:
            sa_, sb_ = rings[0][1].download(np.float32).reshape(NSLOT, -1), rings[1][1].download(np.float32).reshape(NSLOT, -1)
            for b in range(B):
                assert np.array_equal(sa_[(cur + 1 + b) % NSLOT], sb_[(cur + 1 + b) % NSLOT]), (call, b)
            pend = 0
        cur = (cur + 1 + j) % NSLOT
        for cb_ in curs:
            gpu.ok(gpu.L.qgpu_set_i32(cb_.i32(), cur))
        if call == 1:
            # the state the snapshot sequence selects, written from the kept factors
            fst.upload(np.array([pend, par], np.int32))
            mat = gpu.put(rings[1][1].download(np.float32))
            gpu.ok(gpu.L.qgpu_gdn_materialize(mat.f32(), sstride, NSLOT, curs[1].i32(), nk, nv, hk, fbuf.f32(), ftok,
                                              fst.i32()))
            want = rings[0][1].download(np.float32).reshape(NSLOT, -1)[cur]
            assert np.array_equal(mat.download(np.float32).reshape(NSLOT, -1)[cur], want)
            mat.close()
        print(f"  call {call}: B={B} ({'factor' if factor else 'snapshot'} form) identical; rollback to {j}",
              flush=True)
    gpu.sync()


def test_rmsnorm_gated(gpu):
    rng = np.random.default_rng(1)
    rows, n = 12, 128
    x = rng.standard_normal((rows, n)).astype(np.float32)
    z = rng.standard_normal((rows, n)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    xb, zb, wb = gpu.put(x), gpu.put(z), gpu.put(w)
    gpu.ok(gpu.L.qgpu_rmsnorm_gated(xb.f32(), xb.f32(), zb.f32(), wb.f32(), n, rows, n, 1e-6))
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * w * (z / (1 + np.exp(-z.astype(np.float64))))
    assert rel_err(xb.download(np.float32).reshape(rows, n), ref) < 1e-5


# ---------------------------------------------------------------- attention
def attn_fp64(q, k, v, qw, kw, kc, vc, pos, B, nh, nkv, hd, rope_dim, theta, eps):
    """FP64 statement of model.c:318-406, 784-810 for B query tokens."""
    half = rope_dim // 2
    kc, vc = kc.astype(np.float64).copy(), vc.astype(np.float64).copy()

    def norm(x, w):
        x = x.astype(np.float64)
        return x / np.sqrt((x ** 2).mean() + eps) * w

    def rope(x, p):
        i = np.arange(half)
        ang = np.float32(p) * np.power(np.float32(theta), (-2.0 * i / rope_dim).astype(np.float32))
        c, s = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
        y = x.copy()
        y[:half] = x[:half] * c - x[half:2 * half] * s
        y[half:2 * half] = x[:half] * s + x[half:2 * half] * c
        return y

    qr = np.zeros((B, nh, hd))
    for b in range(B):
        for h in range(nh):
            qr[b, h] = rope(norm(q[b, h * 2 * hd:h * 2 * hd + hd], qw), pos + b)
        for g in range(nkv):
            kc[pos + b, g] = rope(norm(k[b, g * hd:(g + 1) * hd], kw), pos + b)
            vc[pos + b, g] = v[b, g * hd:(g + 1) * hd]
    out = np.zeros((B, nh * hd))
    per = nh // nkv
    for b in range(B):
        for h in range(nh):
            g = h // per
            s = kc[:pos + b + 1, g] @ qr[b, h] / np.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            gate = q[b, h * 2 * hd + hd:(h + 1) * 2 * hd].astype(np.float64)
            out[b, h * hd:(h + 1) * hd] = (p @ vc[:pos + b + 1, g]) / (1 + np.exp(-gate))
    return out, kc, vc


ATT_DIMS = (24, 4, 256, 64, 1e7, 1e-6, 512)      # n_head, n_kv, head_dim, rope_dim, theta, eps, n_ctx


def _attn_inputs(pos, B, n_ctx=ATT_DIMS[6]):
    nh, nkv, hd, rope_dim, theta, eps, _ = ATT_DIMS
    rng = np.random.default_rng(pos + B)
    q = rng.standard_normal((B, nh * 2 * hd)).astype(np.float32)
    k = rng.standard_normal((B, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((B, nkv * hd)).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kc = np.zeros((n_ctx, nkv, hd), np.float32)
    vc = np.zeros((n_ctx, nkv, hd), np.float32)
    kc[:pos] = rng.standard_normal((pos, nkv, hd)).astype(np.float32)
    vc[:pos] = rng.standard_normal((pos, nkv, hd)).astype(np.float32)
    half = rope_dim // 2
    i = np.arange(half)
    ang = np.arange(n_ctx, dtype=np.float32)[:, None] * np.power(np.float32(theta), (-2.0 * i / rope_dim).astype(np.float32))[None]
    rc, rs = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    return q, k, v, qw, kw, kc, vc, rc, rs


@pytest.mark.parametrize("pos,B,n_ctx", [(0, 1, 512), (37, 4, 512), (300, 8, 512), (95, 3, 512), (31, 2, 512),
                                         (504, 8, 512), (17, 6, 512), (497, 8, 512),
                                         (3000, 8, 4096), (4090, 5, 4096), (2047, 1, 4096)])
def test_attention_vs_fp64(gpu, pos, B, n_ctx):
    """Spans of one to several tiles: 512 positions give one tile per span, 4096 up to four."""
    print(f"\n[attn] pos={pos} B={B} n_ctx={n_ctx}", flush=True)
    nh, nkv, hd, rope_dim, theta, eps, _ = ATT_DIMS
    q, k, v, qw, kw, kc, vc, rc, rs = _attn_inputs(pos, B, n_ctx)
    ref, kref, vref = attn_fp64(q, k, v, qw, kw, kc, vc, pos, B, nh, nkv, hd, rope_dim, theta, eps)
    qb, kb, vb = gpu.put(q), gpu.put(k), gpu.put(v)
    kcb, vcb = gpu.put(kc), gpu.put(vc)
    posb = gpu.put(np.array([pos], np.int32))
    qwb, kwb, rcb, rsb = gpu.put(qw), gpu.put(kw), gpu.put(rc), gpu.put(rs)
    gpu.ok(gpu.L.qgpu_attn_prep(qb.f32(), nh * 2 * hd, kb.f32(), vb.f32(), nkv * hd, qwb.f32(), kwb.f32(),
                                kcb.f32(), vcb.f32(), rcb.f32(), rsb.f32(), rope_dim, posb.i32(), B, nh, nkv, hd, eps))
    ob = gpu.buf(B * nh * hd * 4)
    gpu.ok(gpu.L.qgpu_attn_decode(qb.f32(), nh * 2 * hd, kcb.f32(), vcb.f32(), posb.i32(), n_ctx, B, nh, nkv, hd,
                                  ob.f32(), nh * hd))
    got = ob.download(np.float32).reshape(B, nh * hd)
    assert rel_err(got, ref) < 1e-4
    kcg = kcb.download(np.float32).reshape(n_ctx, nkv, hd)
    assert rel_err(kcg[pos:pos + B], kref[pos:pos + B]) < 1e-5
    assert np.array_equal(vcb.download(np.float32).reshape(n_ctx, nkv, hd)[pos:pos + B], v.reshape(B, nkv, hd))
    # fused form (norm + RoPE + cache write inside the attention kernel), tight context bound
    qb2, kcb2, vcb2 = gpu.put(q), gpu.put(kc), gpu.put(vc)
    ob2 = gpu.buf(B * nh * hd * 4)
    gpu.ok(gpu.L.qgpu_attn_fused(qb2.f32(), nh * 2 * hd, kb.f32(), vb.f32(), nkv * hd, qwb.f32(), kwb.f32(),
                                 kcb2.f32(), vcb2.f32(), rcb.f32(), rsb.f32(), rope_dim, posb.i32(), pos + B, B, nh,
                                 nkv, hd, eps, ob2.f32(), nh * hd))
    got2 = ob2.download(np.float32).reshape(B, nh * hd)
    print(f"  decode {rel_err(got, ref):.2e} fused {rel_err(got2, ref):.2e}", flush=True)
    assert rel_err(got2, ref) < 1e-4
    assert np.array_equal(qb2.download(np.float32).reshape(B, -1), q), "fused attention must not modify q"
    kcg2 = kcb2.download(np.float32).reshape(n_ctx, nkv, hd)
    assert rel_err(kcg2[pos:pos + B], kref[pos:pos + B]) < 1e-5
    assert np.array_equal(kcg2[:pos], kc[:pos]) and np.array_equal(kcg2[pos + B:], kc[pos + B:])
    assert np.array_equal(vcb2.download(np.float32).reshape(n_ctx, nkv, hd)[pos:pos + B], v.reshape(B, nkv, hd))


@pytest.mark.parametrize("t", [23, 14])
@pytest.mark.parametrize("pos,B", [(0, 1), (300, 4), (95, 7), (504, 8)])
def test_attention_prepares_o_projection(gpu, t, pos, B):
    """qgpu_attn_fused_act writes the rows of qgpu_attn_fused and the digit planes the COPY preparation
    writes from them: the o-projection through qgpu_gemv_prepared(_split) equals qgpu_gemv_act_split /
    qgpu_gemv_act_batch on the rows, bit for bit."""
    import ctypes
    print(f"\n[attn-act] type={t} pos={pos} B={B}", flush=True)
    nh, nkv, hd, rope_dim, theta, eps, n_ctx = ATT_DIMS
    q, k, v, qw, kw, kc, vc, rc, rs = _attn_inputs(pos, B)
    host = host_lib()
    ne0, ne1 = nh * hd, 320
    W = host.synth_matrix(t, ne0, ne1, 41, 7, 0.02)
    T = gpu.tensor(W, t, ne0, ne1)
    ks = gpu.L.qgpu_gemv_split_ks(T.h)
    assert ks > 1
    qb, kb, vb = gpu.put(q), gpu.put(k), gpu.put(v)
    posb = gpu.put(np.array([pos], np.int32))
    qwb, kwb, rcb, rsb = gpu.put(qw), gpu.put(kw), gpu.put(rc), gpu.put(rs)

    def attn(fn, rows=True):
        kcb, vcb, ob = gpu.put(kc), gpu.put(vc), gpu.buf(B * ne0 * 4)
        gpu.ok(fn(qb.f32(), nh * 2 * hd, kb.f32(), vb.f32(), nkv * hd, qwb.f32(), kwb.f32(), kcb.f32(), vcb.f32(),
                  rcb.f32(), rsb.f32(), rope_dim, posb.i32(), n_ctx, B, nh, nkv, hd, eps,
                  ob.f32() if rows else None, ne0))
        return ob, kcb.download(np.float32), vcb.download(np.float32)

    pa, pb = gpu.buf(ks * B * ne1 * 4), gpu.buf(ks * B * ne1 * 4)
    ya, yb = gpu.buf(B * ne1 * 4), gpu.buf(B * ne1 * 4)
    # the reference sequence: attention rows, then the COPY preparation inside the GEMV calls
    oa, kca, vca = attn(gpu.L.qgpu_attn_fused)
    a = pyqwen.Act()
    a.kind, a.x, a.ldx = pyqwen.ACT_COPY, oa.f32(), ne0
    gpu.ok(gpu.L.qgpu_gemv_act_split(T.h, ctypes.byref(a), B, pa.f32(), ne1, ks))
    Ws = (ctypes.c_void_p * 1)(T.h)
    gpu.ok(gpu.L.qgpu_gemv_act_batch(Ws, 1, ctypes.byref(a), B, (pyqwen.F32P * 1)(ya.f32()),
                                     (ctypes.c_uint64 * 1)(ne1), 0))
    # the prepared sequence
    ob1, kcb1, vcb1 = attn(gpu.L.qgpu_attn_fused_act)
    gpu.ok(gpu.L.qgpu_gemv_prepared_split(T.h, B, pb.f32(), ne1, ks))
    ob2, _, _ = attn(gpu.L.qgpu_attn_fused_act)
    gpu.ok(gpu.L.qgpu_gemv_prepared(T.h, B, yb.f32(), ne1, 0))
    # with no fp32 rows asked for (out NULL, as the model calls it): the same digit planes
    yc = gpu.buf(B * ne1 * 4)
    attn(gpu.L.qgpu_attn_fused_act, rows=False)
    gpu.ok(gpu.L.qgpu_gemv_prepared(T.h, B, yc.f32(), ne1, 0))
    assert np.array_equal(yc.download(np.float32), ya.download(np.float32))
    assert gpu.L.qgpu_attn_fused(qb.f32(), nh * 2 * hd, kb.f32(), vb.f32(), nkv * hd, qwb.f32(), kwb.f32(),
                                 gpu.put(kc).f32(), gpu.put(vc).f32(), rcb.f32(), rsb.f32(), rope_dim, posb.i32(),
                                 n_ctx, B, nh, nkv, hd, eps, None, ne0) == -1      # rows required without digits
    rows = oa.download(np.float32)
    assert np.array_equal(ob1.download(np.float32), rows) and np.array_equal(ob2.download(np.float32), rows)
    assert np.array_equal(kcb1, kca) and np.array_equal(vcb1, vca)
    assert np.array_equal(pb.download(np.float32), pa.download(np.float32))
    assert np.array_equal(yb.download(np.float32), ya.download(np.float32))
    ref = O.gemv(t, W, ne0, ne1, rows.reshape(B, ne0), B)
    e = rel_err(ya.download(np.float32).reshape(B, ne1), ref)
    print(f"  ks={ks} prepared == act path; gemv rel err {e:.2e}", flush=True)
    assert e < 2e-5


def test_attention_head_split_bound(gpu):
    """qgpu_attn_split_bound: the head split only where it takes fewer row tiles (6 query heads per kv
    head x 3..8 tokens), and only up to the live context where the doubled span blocks still fit the
    compute units once: 2 n_kv nsl <= CUs, with nsl spans of max(ceil(tiles / 64), 2) tiles; on 256 CUs
    and 4 kv heads that is 64 tiles, 1024 positions."""
    nh, nkv, n_ctx = 24, 4, 8704
    b = {B: gpu.L.qgpu_attn_split_bound(n_ctx, B, nh, nkv) for B in range(1, 9)}
    n_cu = gpu.device_info()[1]
    print(f"\n[attn-split] bounds {b} on {n_cu} CUs", flush=True)
    assert b[1] == b[2] == 0
    # the largest tile count t such that every live context of 1..t tiles has 2 n_kv nsl <= CUs
    t = 0
    while t < n_ctx // 16:
        ntl = t + 1
        tps = max(-(-ntl // min(ntl, 64)), 2)
        if 2 * nkv * -(-ntl // tps) > n_cu:
            break
        t = ntl
    want = min(16 * t, n_ctx)
    if n_cu == 256:
        assert want == 1024
    assert all(b[B] == want for B in range(3, 9))
    assert gpu.L.qgpu_attn_split_bound(300, 4, nh, nkv) == min(300, want)   # never past the context
    assert gpu.L.qgpu_attn_split_bound(n_ctx, 4, 20, 4) == 0                 # 5 heads per kv head: no even split


@pytest.mark.parametrize("pos,B", [(0, 3), (37, 4), (500, 5), (801, 4), (1000, 4), (200, 1), (3000, 4),
                                   (300, 8), (700, 6), (1010, 7), (3000, 8)])
def test_attention_head_split_bit_identical(gpu, pos, B):
    """qgpu_attn_fused_act_live with a live-context bound (two span blocks per kv head, half of its query
    heads each, while the bound allows) writes the same bits as qgpu_attn_fused_act: output rows, o-projection
    digit planes (through the prepared GEMV) and cache rows; a bound past the split's limit, or none, takes the
    one-block path.  Bad bounds are rejected."""
    print(f"\n[attn-split] pos={pos} B={B}", flush=True)
    nh, nkv, hd, rope_dim, theta, eps, _ = ATT_DIMS
    n_ctx = 4096
    q, k, v, qw, kw, kc, vc, rc, rs = _attn_inputs(pos, B, n_ctx)
    host = host_lib()
    ne0, ne1 = nh * hd, 320
    W = host.synth_matrix(23, ne0, ne1, 43, 9, 0.02)
    T = gpu.tensor(W, 23, ne0, ne1)
    qb, kb, vb = gpu.put(q), gpu.put(k), gpu.put(v)
    posb = gpu.put(np.array([pos], np.int32))
    qwb, kwb, rcb, rsb = gpu.put(qw), gpu.put(kw), gpu.put(rc), gpu.put(rs)
    bound = gpu.L.qgpu_attn_split_bound(n_ctx, B, nh, nkv)

    def run(live):
        kcb, vcb, ob, yb = gpu.put(kc), gpu.put(vc), gpu.buf(B * ne0 * 4), gpu.buf(B * ne1 * 4)
        args = (qb.f32(), nh * 2 * hd, kb.f32(), vb.f32(), nkv * hd, qwb.f32(), kwb.f32(), kcb.f32(), vcb.f32(),
                rcb.f32(), rsb.f32(), rope_dim, posb.i32(), n_ctx, B, nh, nkv, hd, eps, ob.f32(), ne0)
        if live is None:
            gpu.ok(gpu.L.qgpu_attn_fused_act(*args))
        else:
            gpu.ok(gpu.L.qgpu_attn_fused_act_live(*args, live))
        gpu.ok(gpu.L.qgpu_gemv_prepared(T.h, B, yb.f32(), ne1, 0))
        return [x.download(np.float32) for x in (ob, yb, kcb, vcb)]

    ref = run(None)
    lives = [0, pos + B, max(bound, pos + B), n_ctx]
    for live in lives:
        got = run(live)
        split = 0 < live <= bound
        print(f"  live {live} (bound {bound}, split {split}): identical", flush=True)
        for a, b_ in zip(got, ref):
            assert np.array_equal(a, b_), (live, bound)
    ob = gpu.buf(B * ne0 * 4)
    for bad in (B - 1, n_ctx + 1):
        if bad < 1:
            continue
        rc_ = gpu.L.qgpu_attn_fused_act_live(qb.f32(), nh * 2 * hd, kb.f32(), vb.f32(), nkv * hd, qwb.f32(),
                                             kwb.f32(), gpu.put(kc).f32(), gpu.put(vc).f32(), rcb.f32(), rsb.f32(),
                                             rope_dim, posb.i32(), n_ctx, B, nh, nkv, hd, eps, ob.f32(), ne0, bad)
        assert rc_ == -1                       # QGPU_E_ARG
    if B >= 3 and pos + B <= 1024:
        assert bound > 0            # the split path ran above


def test_spec_accept_kernel(gpu):
    cand = gpu.put(np.array([7, 3, 9, 4, 0, 0, 0, 0], np.uint32))
    for vt, k, fj, j in (([3, 9, 4, 11], 3, -1, 3), ([3, 8, 4, 11], 3, -1, 1), ([5, 9, 4, 11], 3, -1, 0),
                         ([12], 0, -1, 0), ([5, 9, 4, 11], 3, 2, 2), ([3, 9, 4, 11], 3, 9, 3)):
        vb = gpu.put(np.array(vt + [0] * (8 - len(vt)), np.uint32))
        pos, cur = gpu.put(np.array([100], np.int32)), gpu.put(np.array([7], np.int32))
        out = gpu.buf(16 * 4)
        gpu.ok(gpu.L.qgpu_spec_accept(cand.u32(), vb.u32(), k, fj, pos.i32(), cur.i32(), NSLOT, out.u32()))
        o = out.download(np.uint32)
        assert o[0] == j and list(o[1:j + 2]) == [7, 3, 9, 4][:j + 1] and o[j + 2] == vt[j]
        assert pos.download(np.int32)[0] == 100 + j + 1 and cur.download(np.int32)[0] == (7 + 1 + j) % NSLOT
        # the same with the incoming position and slot as values (the outputs start as other values)
        pos2, cur2, out2 = gpu.put(np.array([-5], np.int32)), gpu.put(np.array([3], np.int32)), gpu.buf(16 * 4)
        gpu.ok(gpu.L.qgpu_spec_accept_at(cand.u32(), vb.u32(), k, fj, 100, 7, pos2.i32(), cur2.i32(), NSLOT,
                                         out2.u32()))
        assert np.array_equal(out2.download(np.uint32)[:j + 3], o[:j + 3])     # out[0 .. j+2] are written
        assert pos2.download(np.int32)[0] == 100 + j + 1 and cur2.download(np.int32)[0] == (7 + 1 + j) % NSLOT
        # the same, handing the re-anchor its inputs: hidden row j, token cand[j], and the next
        # cand[0] = vtok[j] written into the candidate buffer itself
        rows = np.random.default_rng(j).standard_normal((8, 48)).astype(np.float32)
        rb, hb, tb = gpu.put(rows), gpu.put(np.full(40, np.nan, np.float32)), gpu.put(np.zeros(4, np.uint32))
        c3 = gpu.put(np.array([7, 3, 9, 4, 0, 0, 0, 0], np.uint32))
        pos3, cur3, out3 = gpu.put(np.array([-5], np.int32)), gpu.put(np.array([3], np.int32)), gpu.buf(16 * 4)
        gpu.ok(gpu.L.qgpu_spec_accept_anchor(c3.u32(), vb.u32(), k, fj, 99, 7, pos3.i32(), cur3.i32(), NSLOT,
                                             out3.u32(), rb.f32(), 48, 40, hb.f32(), tb.u32(), c3.u32()))
        assert np.array_equal(out3.download(np.uint32)[:j + 3], o[:j + 3])
        assert pos3.download(np.int32)[0] == 99 + j + 1 and cur3.download(np.int32)[0] == (7 + 1 + j) % NSLOT
        assert np.array_equal(hb.download(np.float32), rows[j, :40])
        assert tb.download(np.uint32)[0] == [7, 3, 9, 4][j]
        assert list(c3.download(np.uint32)) == [vt[j], 3, 9, 4, 0, 0, 0, 0]
    ob = gpu.buf(16 * 4)
    p_, c_ = gpu.put(np.array([0], np.int32)), gpu.put(np.array([0], np.int32))
    assert gpu.L.qgpu_spec_accept_anchor(cand.u32(), cand.u32(), 1, -1, 5, 0, p_.i32(), c_.i32(), NSLOT, ob.u32(),
                                         None, 8, 8, ob.f32(), None, None) != 0   # a row copy without rows
    for p0, c0 in ((-1, 0), (5, -1), (5, NSLOT)):                  # rejected: no valid incoming position / slot
        assert gpu.L.qgpu_spec_accept_at(cand.u32(), cand.u32(), 1, -1, p0, c0, p_.i32(), c_.i32(), NSLOT,
                                         ob.u32()) != 0


def test_spec_accept_into_host_memory(gpu):
    """The acceptance result written by the kernel straight into qgpu_host_malloc memory:
    out[0] (j) leaves the host's sentinel once the rest is there, read without a copy."""
    p = ctypes.c_void_p()
    gpu.ok(gpu.L.qgpu_host_malloc(ctypes.byref(p), 64 * 4))
    try:
        h = np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint32)), (64,))
        cand = gpu.put(np.array([7, 3, 9, 4, 0, 0, 0, 0], np.uint32))
        vb = gpu.put(np.array([3, 8, 4, 11, 0, 0, 0, 0], np.uint32))          # first mismatch at 1
        pos, cur = gpu.put(np.array([0], np.int32)), gpu.put(np.array([0], np.int32))
        h[:] = 0xFFFFFFFF
        gpu.ok(gpu.L.qgpu_spec_accept_anchor(cand.u32(), vb.u32(), 3, -1, 50, 2, pos.i32(), cur.i32(), NSLOT,
                                             ctypes.cast(p, ctypes.POINTER(ctypes.c_uint32)), None, 0, 0, None,
                                             None, None))
        t0 = time.time()
        while h[0] == 0xFFFFFFFF and time.time() - t0 < 10:
            pass
        gpu.sync()
        assert list(h[:4]) == [1, 7, 3, 8] and h[4] == 0xFFFFFFFF
        assert pos.download(np.int32)[0] == 52 and cur.download(np.int32)[0] == 4
    finally:
        gpu.ok(gpu.L.qgpu_host_free(p))


# ---------------------------------------------------------------- tiny hybrid model
@pytest.fixture(scope="module", params=["tiny", "tiny_mixed"])
def tiny(request):
    z = load(f"model_{request.param}.npz")
    td = tempfile.mkdtemp()
    path = os.path.join(td, "m.gguf")
    host_lib().write_tiny_gguf(path, int(z["seed"]), int(z["mixed"]))
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(z["gguf_sha256"])
    yield path, z
    os.remove(path)


def test_model_forward_batch_and_sequential_vs_reference(gpu, tiny):
    path, z = tiny
    print(f"\n[model] {os.path.basename(path)} forward", flush=True)
    V = 1024
    p = z["prompt"]
    m = pyqwen.Model(path, int(z["n_ctx"]))
    lb = m.forward_batch(p[:8], 0, 0)
    ref = z["batch_logits"].reshape(8, V)
    for b in range(8):
        assert rel_err(lb[b], ref[b]) < 1e-3, b
        assert lb[b].argmax() == ref[b].argmax()
    assert rel_err(m.h_save(8), z["batch_hsave"].reshape(8, -1)) < 1e-3
    # MTP prefill + one draft with logits (mtp_forward_batch then mtp_forward)
    m.mtp_forward_batch(p[:8], 0)
    ml = m.mtp_forward(int(p[8]), 8)
    assert rel_err(ml, z["mtp_logits"]) < 1e-3 and ml.argmax() == z["mtp_logits"].argmax()
    m.close()
    m = pyqwen.Model(path, int(z["n_ctx"]))
    seq = np.array([m.forward(int(p[i]), i) for i in range(8)])
    sref = z["seq_logits"].reshape(8, V)
    for b in range(8):
        assert rel_err(seq[b], sref[b]) < 1e-3, b
    m.close()



@pytest.mark.parametrize("mixed", [0, 1])
def test_model_tied_output_vs_oracle(gpu, mixed):
    """A model file without output.weight: model_init falls back to token_embd as the lm_head
    (model.c:87-88) and uploads it once.  Batched, sequential and MTP logits match the oracle on the
    same file within 1e-3 (same argmax), and equal the GPU's own logits for the file whose
    output.weight is an explicit copy of token_embd, bit for bit."""
    host = host_lib()
    td = tempfile.mkdtemp()
    p = np.random.default_rng(5).integers(0, 1024, 9).astype(np.uint32)
    got = []
    for tie in (1, 2):
        spec = host.spec_tiny(31, mixed)
        spec.tie_output = tie
        path = os.path.join(td, f"tie{tie}.gguf")
        host.write_gguf(spec, path)
        m = pyqwen.Model(path, 64)
        lb = m.forward_batch(p[:8], 0, 0)
        m.mtp_forward_batch(p[:8], 0)
        ml = m.mtp_forward(int(p[8]), 8)
        m.close()
        m = pyqwen.Model(path, 64)
        seq = np.array([m.forward(int(p[i]), i) for i in range(4)])
        m.close()
        got.append((lb, ml, seq))
        if tie == 1:
            o = O.Model(path, 64)
            olb = o.forward_batch(p[:8], 0, 0)
            o.L.or_mtp_forward_batch(o.h, O.uptr(np.ascontiguousarray(p[:8])), 0, 8, 0)
            o.L.or_mtp_forward(o.h, int(p[8]), 8, 1)
            oml = o.arr(o.L.or_model_logits, o.V)
            o.close()
            o = O.Model(path, 64)
            oseq = np.array([o.forward(int(p[i]), i) for i in range(4)])
            o.close()
            for b in range(8):
                assert rel_err(lb[b], olb[b]) < 1e-3 and lb[b].argmax() == olb[b].argmax(), b
            assert rel_err(ml, oml) < 1e-3 and ml.argmax() == oml.argmax()
            for b in range(4):
                assert rel_err(seq[b], oseq[b]) < 1e-3, b
            print(f"\n[tied] mixed={mixed}: batch rel err {rel_err(lb, olb):.2e}", flush=True)
        os.remove(path)
    for a, b in zip(got[0], got[1]):
        assert np.array_equal(a, b)

def test_model_forward_section_profile(gpu, tiny):
    """The reference's --profile counters (model.c:697-742): with profiling on, model_forward adds
    the device time of the embedding, the GDN layers, the attention layers and the head; the
    logits are those of the run without profiling; with it off only the call count moves."""
    path, z = tiny
    p = z["prompt"]
    m = pyqwen.Model(path, int(z["n_ctx"]))
    plain = np.array([m.forward(int(p[i]), i) for i in range(6)])
    c0 = m.prof_counters()
    m.reset()
    m.set_profile(1)
    t0 = time.perf_counter()
    prof = np.array([m.forward(int(p[i]), i) for i in range(6)])
    wall = time.perf_counter() - t0
    c1 = m.prof_counters()
    assert np.array_equal(plain, prof)
    d = {k: c1[k] - c0[k] for k in c1}
    print(f"  sections over 6 calls: {d}", flush=True)
    assert d["calls"] == 6
    for k in ("embed", "gdn", "attn", "head"):
        assert d[k] > 0, k
    assert d["embed"] + d["gdn"] + d["attn"] + d["head"] < wall
    assert d["gdn"] > d["embed"]
    m.set_profile(0)
    m.forward(int(p[6]), 6)
    c2 = m.prof_counters()
    assert c2["calls"] == c1["calls"] + 1 and all(c2[k] == c1[k] for k in ("embed", "gdn", "attn", "head"))
    m.close()


def test_model_rollback_vs_reference(gpu, tiny):
    path, z = tiny
    p = z["prompt"]
    m = pyqwen.Model(path, int(z["n_ctx"]))
    for i in range(5):
        m.forward(int(p[i]), i)
    m.forward_batch(p[10:13], 5)
    m.rollback_to(1)
    m.pos = 8
    lb = m.forward_batch(p[13:16], 7)
    ref = z["rollback_logits"].reshape(3, -1)
    for b in range(3):
        assert rel_err(lb[b], ref[b]) < 1e-3 and lb[b].argmax() == ref[b].argmax(), b


def test_gdn_factor_form_model_matches_snapshots(gpu, tiny):
    """The model with the GDN factor form for batches of 5..8 tokens (the default) against the same model
    with snapshots everywhere (QWEN_GDN_FACTOR_MIN_B=9): batches of 8, 6 and 5 with rollbacks between them,
    single-token steps after a factor-form batch (the kept tokens applied in a snapshot-form call), the step
    timer after a factor-form batch (which writes the selected state out and then allows only b = 0), and a
    last batch: every logit row and hidden state bit-identical."""
    path, z = tiny
    p = z["prompt"]
    models = []
    for fmin in ("9", None):
        if fmin is None:
            os.environ.pop("QWEN_GDN_FACTOR_MIN_B", None)
        else:
            os.environ["QWEN_GDN_FACTOR_MIN_B"] = fmin
        try:
            models.append(pyqwen.Model(path, int(z["n_ctx"])))
        finally:
            os.environ.pop("QWEN_GDN_FACTOR_MIN_B", None)
    snap, fac = models

    def both(fn):
        a, b = fn(snap), fn(fac)
        assert snap.status() == 0 and fac.status() == 0
        return a, b
    pos = 0
    for i in range(3):
        a, b = both(lambda m: m.forward(int(p[i]), i))
        assert np.array_equal(a, b)
    pos = 3
    for B, j in ((8, 3), (6, 5), (5, 0), (8, 7)):
        a, b = both(lambda m: m.forward_batch(p[pos:pos + B], pos))
        assert np.array_equal(a, b), (B, j)
        assert np.array_equal(snap.h_save(B), fac.h_save(B)), (B, j)
        both(lambda m: m.rollback_to(j))
        pos += j + 1
        both(lambda m: setattr(m, "pos", pos))
        print(f"  batch of {B} at {pos - j - 1}, rollback to {j}: identical", flush=True)
    a, b = both(lambda m: m.forward(int(p[pos]), pos))      # applies the 8 kept tokens of the last batch
    assert np.array_equal(a, b)
    pos += 1
    a, b = both(lambda m: m.forward_batch(p[pos:pos + 6], pos))
    assert np.array_equal(a, b)
    pos += 6
    both(lambda m: m.time_steps(5, 2))                        # writes the selected state out (factor form)
    fac.rollback_to(0)
    assert fac.status() == -1                                 # the other states of that batch are gone
    for m in models:
        m.pos = pos
    a, b = both(lambda m: m.forward_batch(p[pos:pos + 4], pos))
    assert np.array_equal(a, b)
    both(lambda m: m.rollback_to(1))                          # a snapshot-form batch: any b again
    pos += 2
    a, b = both(lambda m: m.forward(int(p[pos]), pos))
    assert np.array_equal(a, b)
    for m in models:
        m.close()


def test_model_rollback_rejects_states_not_written(gpu, tiny):
    """model_rollback_to(b) selects the state after token b of the last batch: b at or past that
    batch's B is refused on the host (status -1, ring index unchanged), and a valid rollback after
    it still gives the reference's logits."""
    path, z = tiny
    p = z["prompt"]
    m = pyqwen.Model(path, int(z["n_ctx"]))
    for i in range(5):
        m.forward(int(p[i]), i)
    m.forward_batch(p[10:13], 5)
    for b in (3, 7, 8):
        m.rollback_to(b)
        assert m.status() == -1, b
    m.rollback_to(1)
    assert m.status() == 0
    m.pos = 8
    lb = m.forward_batch(p[13:16], 7)
    ref = z["rollback_logits"].reshape(3, -1)
    for b in range(3):
        assert rel_err(lb[b], ref[b]) < 1e-3 and lb[b].argmax() == ref[b].argmax(), b
    m.forward(int(p[0]), 10)                         # a decode step writes one state
    m.rollback_to(1)
    assert m.status() == -1
    m.rollback_to(0)
    assert m.status() == 0
    m.reset()
    m.rollback_to(0)                                 # nothing written since the reset
    assert m.status() == -1
    m.close()


@pytest.mark.parametrize("k", [1, 2, 3, 5, 7])
def test_model_spec_stream_vs_reference(gpu, tiny, k):
    """On-device greedy MTP speculative decode == the reference's spec stream == greedy stream."""
    path, z = tiny
    m = pyqwen.Model(path, int(z["n_ctx"]))
    toks, js, st = m.generate_spec(z["prompt"][:20], 40, k)
    key = f"spec_k{k}" if k <= 2 else f"spec_seq_k{k}"
    assert np.array_equal(toks, z[key])
    assert np.array_equal(js, z[f"spec_j_k{k}" if k <= 2 else f"spec_seq_j_k{k}"][:len(js)])
    assert np.array_equal(toks, z["greedy"])


def test_model_greedy_stream_vs_reference(gpu, tiny):
    path, z = tiny
    m = pyqwen.Model(path, int(z["n_ctx"]))
    toks, st = m.generate_greedy(z["prompt"][:20], 40)
    assert np.array_equal(toks, z["greedy"])


@pytest.mark.parametrize("k,mode", [(3, 1), (7, 1), (3, 2), (7, 2)])
def test_model_forced_acceptance_vs_oracle(gpu, tiny, k, mode):
    """Fixed acceptance (mode 1: j = k every cycle; mode 2: j = cycle mod (k+1), every
    rollback depth in turn) against the oracle running the same loop on the CPU."""
    path, z = tiny
    m = pyqwen.Model(path, int(z["n_ctx"]))
    toks, js, st = m.generate_spec(z["prompt"][:20], 48, k, force_accept=mode)
    om = O.Model(path, int(z["n_ctx"]), k_max=7)
    otoks, ojs, ost = om.generate_spec(z["prompt"][:20], 48, k, force_accept=mode)
    assert np.array_equal(toks, otoks)
    assert np.array_equal(js, ojs)
    want = np.full(len(js), k) if mode == 1 else np.arange(len(js)) % (k + 1)
    assert np.array_equal(js, want)


def test_model_init_rejects_bad_files(gpu):
    host = host_lib()
    td = tempfile.mkdtemp()
    bad = os.path.join(td, "bad.gguf")
    with open(bad, "wb") as f:
        f.write(b"NOTGGUF" + b"\0" * 64)
    with pytest.raises(pyqwen.QgpuError):
        pyqwen.Model(bad, 64)
    path = os.path.join(td, "t.gguf")
    host.write_tiny_gguf(path, 1, 0)
    data = bytearray(open(path, "rb").read())
    i = data.find(b"blk.1.ffn_up.weight")
    data[i:i + 3] = b"xxx"                                   # missing tensor
    open(bad, "wb").write(bytes(data))
    with pytest.raises(pyqwen.QgpuError):
        pyqwen.Model(bad, 64)


@pytest.mark.parametrize("mode", [0, 1])
def test_model_spec_begin_run_resumes(gpu, tiny, mode):
    """begin + several run() calls of a few cycles each == one uninterrupted generation."""
    path, z = tiny
    m = pyqwen.Model(path, int(z["n_ctx"]))
    m.spec_begin(z["prompt"][:20], 3)
    parts = []
    for cyc in (1, 5, 2, 12):
        t, j, st = m.spec_run(3, cyc, force_accept=mode)
        assert st.n_cycles == cyc and len(t) == cyc * (1 + (3 if mode == 1 else 0))
        parts.append(t)
    m.close()
    got = np.concatenate(parts)
    m = pyqwen.Model(path, int(z["n_ctx"]))
    toks, js, st = m.generate_spec(z["prompt"][:20], len(got), 3, force_accept=mode)
    assert np.array_equal(got, toks)


@pytest.mark.parametrize("k", [3, 5])
@pytest.mark.parametrize("mode", [0, 2])
def test_model_graphs_match_eager(gpu, tiny, mode, k):
    """Replayed launch sequences (HIP graphs) give bit-identical streams and
    logits to kernel-by-kernel launches: every cycle replays the draft, verify and
    anchor graphs at new positions and ring slots, with host reads between replays,
    then a host-API forward runs after the device loop.  k = 5 verifies 6 tokens, so its
    GDN states are in factor form (the kept tokens and factor buffer read from device memory)."""
    path, z = tiny
    res = []
    for graphs in (False, True):
        m = pyqwen.Model(path, int(z["n_ctx"]))
        m.set_graphs(graphs)
        toks, js, st = m.generate_spec(z["prompt"][:20], 40, k, force_accept=mode)
        lb = m.forward_batch(z["prompt"][20:24], m.pos, 1)
        res.append((toks.copy(), js.copy(), lb.copy()))
        m.close()
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1], res[1][1])
    assert np.array_equal(res[0][2], res[1][2])


# ---------------------------------------------------------------- accepted drafts (j > 0)
@pytest.fixture(scope="module")
def accept():
    """The tiny model whose MTP drafts the backbone mostly accepts (synth variant 2); the
    fixture holds the reference's streams for every j in 0..k."""
    z = load("model_tiny_accept.npz")
    td = tempfile.mkdtemp()
    path = os.path.join(td, "accept.gguf")
    host_lib().write_tiny_gguf(path, int(z["seed"]), int(z["variant"]))
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(z["gguf_sha256"])
    yield path, z
    os.remove(path)


def accept_key(pre, force, k):
    if force:
        return f"{pre}spec_f{force}_k{k}"
    return f"{pre}spec_k{k}" if k <= 2 else f"{pre}spec_seq_k{k}"


@pytest.mark.parametrize("pre", ["", "end_"])
@pytest.mark.parametrize("force", [0, 1, 2])
@pytest.mark.parametrize("k", range(1, 8))
def test_model_spec_accept_vs_reference(gpu, accept, pre, force, k):
    """The device loop against the reference with drafts accepted (j over 0..k): tokens and j of
    every cycle identical; the logits the next cycle starts from (logits_b row j of the last cycle)
    and the MTP state within 1e-3.  force 1/2 are the forced-acceptance modes, pinned by the
    reference's sequential-verify harness; end_ runs into the end of a 57-position context."""
    path, z = accept
    print(f"\n[accept] n_ctx={int(z[pre + 'n_ctx'])} force={force} k={k}", flush=True)
    key = accept_key(pre, force, k)
    m = pyqwen.Model(path, int(z[pre + "n_ctx"]))
    toks, js, st = m.generate_spec(z["prompt"], int(z[pre + "n_predict"]), k, force_accept=force)
    assert m.status() == 0
    assert np.array_equal(toks, z[key])
    assert np.array_equal(js, z[key + "_j"])
    jl = int(js[-1])
    last = m.field("logits_b", (jl + 1) * m.V).reshape(jl + 1, m.V)[jl]
    ref = z[key + "_last"]
    assert rel_err(last, ref) < 1e-3 and last.argmax() == ref.argmax()
    assert rel_err(m.field("mtp_h", m.E), z[key + "_mtph"]) < 1e-3
    m.close()


def test_model_rejects_positions_past_the_context(gpu, tiny):
    """Calls whose KV rows would fall past n_ctx are refused on the host (status -1) before any
    device work; the model stays usable and later valid calls match a fresh model."""
    path, z = tiny
    n_ctx = 16
    m = pyqwen.Model(path, n_ctx)
    p = z["prompt"]
    m.forward_batch(p[:8], 0)
    assert m.status() == 0 and m.pos == 8
    before = m.field("logits_b", m.V).copy()
    m.forward_batch(p[:8], 12)                       # rows 12..19 > 15
    assert m.status() == -1 and m.pos == 8
    assert np.array_equal(m.field("logits_b", m.V), before)
    m.forward(int(p[0]), n_ctx)
    assert m.status() == -1
    m.L.mtp_forward(m.h, None, int(p[0]), n_ctx, 1)
    assert m.status() == -1
    m.forward_batch(np.array([m.V + 3], np.uint32), 8)   # token id past the vocabulary
    assert m.status() == -1
    m.forward_batch(p[8:16], 8)                      # rows 8..15: the last valid span
    assert m.status() == 0 and m.pos == 16
    got = m.field("logits_b", 8 * m.V).reshape(8, m.V)
    m.close()
    f = pyqwen.Model(path, n_ctx)
    f.forward_batch(p[:8], 0)
    want = f.forward_batch(p[8:16], 8)
    assert np.array_equal(got, want)
    f.close()


def test_model_init_rejects_unsupported_head_ratio(gpu):
    """More than 48 query rows per KV head at the largest batch (attention kernel limit) fails at
    model_init, not at the first verify."""
    spec = host_lib().spec_tiny(5, 0)
    spec.n_head, spec.n_kv_head = 14, 2              # 7 x 8 = 56 > 48
    with pytest.raises(pyqwen.QgpuError):
        pyqwen.Model(spec=spec, n_ctx=64)


# ---------------------------------------------------------------- long context (8192 positions)
def prompt_ids(n, V):
    """the reference harness's prompt: id i = (i * 2654435761 + 12345) mod 2^32 mod V"""
    i = np.arange(n, dtype=np.uint64)
    return (((i * np.uint64(2654435761) + np.uint64(12345)) & np.uint64(0xFFFFFFFF)) % np.uint64(V)).astype(np.uint32)


@pytest.fixture(scope="module")
def accept_long():
    z = load("model_tiny_accept_long.npz")
    td = tempfile.mkdtemp()
    path = os.path.join(td, "accept.gguf")
    host_lib().write_tiny_gguf(path, int(z["seed"]), int(z["variant"]))
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(z["gguf_sha256"])
    yield path, z
    os.remove(path)


@pytest.mark.parametrize("force", [0, 1])
@pytest.mark.parametrize("k", [1, 3, 5, 7])
def test_model_long_context_vs_reference(gpu, accept_long, force, k):
    """An 8176-token prompt in an 8192-position context (attention over the whole KV cache, RoPE tables
    to n_ctx), then speculative decode at k = 1, 3, 5, 7, natural and all-accepted: the prefill
    logits, tokens, j of every cycle, final logits and MTP state against the reference's own run."""
    path, z = accept_long
    n_ctx, n_prompt, n_predict = int(z["n_ctx"]), int(z["n_prompt"]), int(z["n_predict"])
    print(f"\n[long] n_ctx={n_ctx} prompt={n_prompt} k={k} force={force}", flush=True)
    m = pyqwen.Model(path, n_ctx)
    prompt = prompt_ids(n_prompt, m.V)
    key = f"spec_f1_k{k}" if force else f"spec_seq_k{k}"
    m.spec_begin(prompt, k)
    first = m.field("logits", m.V)
    assert rel_err(first, z["prefill_last"]) < 1e-3 and first.argmax() == z["prefill_last"].argmax()
    toks, js, st = m.spec_run(k, 10**6, n_predict, force_accept=force)
    assert m.status() == 0
    assert np.array_equal(toks, z[key]) and np.array_equal(js, z[key + "_j"])
    jl = int(js[-1])
    last = m.field("logits_b", (jl + 1) * m.V).reshape(jl + 1, m.V)[jl]
    assert rel_err(last, z[key + "_last"]) < 1e-3 and last.argmax() == z[key + "_last"].argmax()
    assert rel_err(m.field("mtp_h", m.E), z[key + "_mtph"]) < 1e-3
    if not force:
        assert np.array_equal(toks, z["greedy"][:len(toks)])
    m.close()
