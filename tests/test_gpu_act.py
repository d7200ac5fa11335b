"""GPU parity of the activation transforms fused into the GEMV input preparation
(qgpu_gemv_act_batch): RMSNorm, two-segment RMSNorm (MTP input), SiLU*up and
per-head gated RMSNorm, against the oracle's ops (pinned to the reference)
followed by the oracle's GEMV.  Bars: GEMV outputs within 1e-3 normwise; the
transformed fp32 rows (xout) within 1e-5."""
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


@pytest.mark.parametrize("t", [23, 14])          # IQ4_XS (digit MFMA path), Q6_K (fp32 path via xout)
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
    if kind == "rmsnorm":
        a.kind, a.w = pyqwen.ACT_RMSNORM, wb.f32()
        xin = np.stack([o_rmsnorm(x[b], w) for b in range(B)])
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
    ex = rel_err(xo, xin)
    ref = O.gemv(t, W, ne0, ne1, xin, B)
    eo = rel_err(out, ref)
    print(f"  xout {ex:.2e}  gemv {eo:.2e}", flush=True)
    assert ex < 1e-5 and eo < 1e-3


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
