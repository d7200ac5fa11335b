"""Batched GEMV at the model's real shapes for every matrix-core weight format
(the quant-format sweep: 5120->17408, 17408->5120 and the 5120->248320 lm_head,
B = 1, 2, 4, 8), and on outlier-heavy activations.

Checker: the oracle's gemv_batch / gemv_rows_batch (bit-exact with the
reference's AVX2 kernels).  Bar: 1e-3 normwise relative (max|d| / max|ref|).
Mirrors the reference's test_batch.c:16-20,38-58 (attn_qkv Q5_K, output Q6_K,
eh_proj Q8_0 at full size)."""
import ctypes

import numpy as np
import pytest

import oracle_lib as O
from gpu_util import gpu, rel_err  # noqa: F401
from qwen_pkg import host_lib, pyqwen

pytestmark = pytest.mark.gpu

FORMATS = {"IQ4_XS": 23, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_0": 8}
_mats = {}


def matrix(gpu, t, ne0, ne1):
    """(host bytes, device tensor) of the seeded matrix; the last one stays resident for the next test"""
    key = (t, ne0, ne1)
    if key not in _mats:
        for k in list(_mats):
            _mats.pop(k)[1].close()
        W = host_lib().synth_matrix(t, ne0, ne1, 77, 300 + t, 0.02)
        _mats[key] = (W, gpu.tensor(W, t, ne0, ne1))
    return _mats[key]


def run(gpu, T, x, n, ne1):
    xb, ob = gpu.put(np.ascontiguousarray(x[:n])), gpu.buf(n * ne1 * 4)
    gpu.ok(gpu.L.qgpu_gemv_batch(T.h, xb.f32(), x.shape[1], n, ob.f32(), ne1, 0))
    return ob.download(np.float32).reshape(n, ne1)


@pytest.mark.parametrize("fmt", list(FORMATS))
@pytest.mark.parametrize("shape", [(5120, 17408), (17408, 5120)])
def test_gemv_sweep_shapes_vs_oracle(gpu, fmt, shape):
    ne0, ne1 = shape
    t = FORMATS[fmt]
    print(f"\n[sweep] {fmt} {ne0}->{ne1} B=1,2,4,8", flush=True)
    W, T = matrix(gpu, t, ne0, ne1)
    x = host_lib().synth_normal(8 * ne0, 78, t).reshape(8, ne0)
    ref = O.gemv(t, W, ne0, ne1, x, 8, threads=16)
    for n in (1, 2, 4, 8):
        got = run(gpu, T, x, n, ne1)
        e = rel_err(got, ref[:n])
        print(f"  B={n}: rel err {e:.2e}", flush=True)
        assert e < 1e-3, (fmt, shape, n, e)
        assert np.array_equal(got.argmax(1), ref[:n].argmax(1))


@pytest.mark.parametrize("fmt", list(FORMATS))
def test_gemv_ksplit_17408_vs_oracle(gpu, fmt):
    """The row-parallel 17408->5120 projection (ffn_down) through the K-split kernel: the partial
    planes summed in order equal the oracle GEMV."""
    ne0, ne1 = 17408, 5120
    t = FORMATS[fmt]
    W, T = matrix(gpu, t, ne0, ne1)
    ks = gpu.L.qgpu_gemv_split_ks(T.h)
    print(f"\n[ksplit] {fmt} {ne0}->{ne1} ks={ks}", flush=True)
    assert ks >= 2
    x = host_lib().synth_normal(8 * ne0, 79, t).reshape(8, ne0)
    ref = O.gemv(t, W, ne0, ne1, x, 8, threads=16)
    for n in (1, 2, 4, 8):
        xb, pb = gpu.put(np.ascontiguousarray(x[:n])), gpu.buf(ks * n * ne1 * 4)
        a = pyqwen.Act()
        a.kind, a.x, a.ldx = pyqwen.ACT_COPY, xb.f32(), ne0
        gpu.ok(gpu.L.qgpu_gemv_act_split(T.h, ctypes.byref(a), n, pb.f32(), ne1, ks))
        planes = pb.download(np.float32).reshape(ks, n, ne1)
        e = rel_err(planes.sum(0), ref[:n])
        assert e < 1e-3, (fmt, n, e)


# row ranges of the 248,320-row lm_head checked against the oracle: first and last tiles and
# stretches across the vocabulary (the whole output is computed on the GPU)
LM_ROWS = [(0, 512), (61_440, 61_952), (124_160, 124_672), (186_880, 187_392), (247_808, 248_320)]


@pytest.mark.parametrize("fmt", list(FORMATS))
def test_gemv_lm_head_vs_oracle(gpu, fmt):
    ne0, ne1 = 5120, 248_320
    t = FORMATS[fmt]
    print(f"\n[lm_head] {fmt} {ne0}->{ne1} ({ne1 // 16} tiles) B=1,2,4,8", flush=True)
    W, T = matrix(gpu, t, ne0, ne1)
    x = host_lib().synth_normal(8 * ne0, 80, t).reshape(8, ne0)
    L = O.lib()
    refs = []
    for r0, r1 in LM_ROWS:
        o = np.zeros((8, ne1), np.float32)
        L.or_gemv_rows_batch(t, W.ctypes.data_as(ctypes.c_void_p), ne0, O.fptr(x), ne0, 8, O.fptr(o), ne1, r0, r1)
        refs.append(o[:, r0:r1].copy())
    ref = np.concatenate(refs, axis=1)
    for n in (1, 2, 4, 8):
        got = run(gpu, T, x, n, ne1)
        sel = np.concatenate([got[:, r0:r1] for r0, r1 in LM_ROWS], axis=1)
        e = rel_err(sel, ref[:n])
        print(f"  B={n}: rel err {e:.2e}", flush=True)
        assert e < 1e-3, (fmt, n, e)
        assert np.all(np.isfinite(got))


@pytest.mark.parametrize("fmt", ["IQ4_XS", "Q8_0"])
def test_gemv_lm_head_row_range(gpu, fmt):
    """qgpu_gemv_rows_batch over a range of the 248,320-row lm_head that is still wide enough for the
    LDS-operand kernel (rows [100, 200003): 12,495 tiles, the first and last partly outside the range),
    B = 4 and 8: the rows of the range against the oracle, and every row outside it left as it was."""
    ne0, ne1, r0, r1 = 5120, 248_320, 100, 200_003
    t = FORMATS[fmt]
    W, T = matrix(gpu, t, ne0, ne1)
    x = host_lib().synth_normal(8 * ne0, 81, t).reshape(8, ne0)
    checks = [(r0, r0 + 400), (99_000, 99_512), (r1 - 400, r1)]
    L = O.lib()
    refs = []
    for c0, c1 in checks:
        o = np.zeros((8, ne1), np.float32)
        L.or_gemv_rows_batch(t, W.ctypes.data_as(ctypes.c_void_p), ne0, O.fptr(x), ne0, 8, O.fptr(o), ne1, c0, c1)
        refs.append(o[:, c0:c1].copy())
    for n in (4, 8):
        print(f"\n[lm_head rows] {fmt} [{r0}, {r1}) B={n}", flush=True)
        xb = gpu.put(np.ascontiguousarray(x[:n]))
        fill = np.full((n, ne1), 7.0, np.float32)
        ob = gpu.put(fill)
        gpu.ok(gpu.L.qgpu_gemv_rows_batch(T.h, xb.f32(), ne0, n, ob.f32(), ne1, r0, r1))
        got = ob.download(np.float32).reshape(n, ne1)
        sel = np.concatenate([got[:, c0:c1] for c0, c1 in checks], axis=1)
        ref = np.concatenate([rr[:n] for rr in refs], axis=1)
        e = rel_err(sel, ref)
        print(f"  rel err {e:.2e}", flush=True)
        assert e < 1e-3
        assert np.all(got[:, :r0] == 7.0) and np.all(got[:, r1:] == 7.0)


def outlier_x(n, ne0, seed, spike):
    """N(0,1) rows with one channel per 256-element super-block at `spike` times the rest, and
    super-blocks whose scale alternates over six orders of magnitude"""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, ne0)).astype(np.float32)
    nsb = ne0 // 256
    for t in range(n):
        for sb in range(nsb):
            x[t, sb * 256 + rng.integers(0, 256)] *= spike * (1 if rng.random() < 0.5 else -1)
            x[t, sb * 256:(sb + 1) * 256] *= np.float32(10.0 ** ((sb % 7) - 3))
    return x


@pytest.mark.parametrize("fmt", ["IQ4_XS", "Q6_K", "Q4_K", "Q8_0"])
@pytest.mark.parametrize("spike", [1e3, 1e4])
def test_gemv_outlier_activations(gpu, fmt, spike):
    """Outlier channels (10^3..10^4 x the rest of their super-block) and mixed super-block magnitudes,
    the worst case of the per-(token, super-block) fixed-point activation digits.  Checked against
    the oracle at the 1e-3 bar, and row by row against the bound the digit scheme fixes: x * 2^s is
    rounded to an integer with max_sb * 2^s in [2^21, 2^22), so each x moves by at most 2^-22 max_sb and
    |err_r| <= sum_sb 2^-22 max_sb sum_{i in sb} |W_ri| + fp32 accumulation (<= 1e-6 sum |W_ri x_i|)."""
    t = FORMATS[fmt]
    ne0, ne1 = 5120, 2048
    print(f"\n[outlier] {fmt} spike {spike:g} B=1,2,4,8", flush=True)
    W = host_lib().synth_matrix(t, ne0, ne1, 81, 400 + t, 0.02)
    T = gpu.tensor(W, t, ne0, ne1)
    x = outlier_x(8, ne0, int(spike) + t, spike)
    ref = O.gemv(t, W, ne0, ne1, x, 8, threads=16)
    absW = np.abs(O.dequant_rows(t, W, ne0, ne1)).astype(np.float64)           # [rows][ne0]
    mx = np.abs(x.astype(np.float64)).reshape(8, ne0 // 256, 256).max(2)       # [tok][sb]
    bound = (absW.reshape(ne1, ne0 // 256, 256).sum(2) @ mx.T).T * 2.0 ** -22   # [tok][rows]
    bound += 1e-6 * (np.abs(x.astype(np.float64)) @ absW.T)
    for n in (1, 2, 4, 8):
        got = run(gpu, T, x, n, ne1)
        e = rel_err(got, ref[:n])
        print(f"  B={n}: rel err {e:.2e}", flush=True)
        assert e < 1e-3, (fmt, spike, n, e)
        exact = x[:n].astype(np.float64) @ O.dequant_rows(t, W, ne0, ne1).astype(np.float64).T
        assert np.all(np.abs(got - exact) <= bound[:n]), (fmt, spike, n)
    T.close()


@pytest.mark.parametrize("fmt", ["IQ4_XS", "Q6_K", "Q8_0"])
@pytest.mark.parametrize("shape", [(5120, 17408), (17408, 5120)])
def test_gemv_pair_split_tail(gpu, fmt, shape):
    """Tail balance: a launch a little over a multiple of the compute units (17408 rows: 1024 + 64 tiles,
    5120 rows: 256 + 64 tiles on 256 CUs) runs its last tiles as two half-K blocks whose partial results
    meet in exchange slots.  Every output is written (the buffer starts as NaN), the oracle agrees within
    1e-3 at B = 1, 4, 8, a second call gives the same bits (the slots are left empty), the ACCUM flag adds
    onto the previous contents exactly, and a captured graph of three calls replays to the same bits."""
    ne0, ne1 = shape
    t = FORMATS[fmt]
    ncu = gpu.device_info()[1]
    tiles = (ne1 + 15) // 16
    print(f"\n[pair] {fmt} {ne0}->{ne1}: {tiles} tiles on {ncu} CUs (remainder {tiles % ncu})", flush=True)
    W, T = matrix(gpu, t, ne0, ne1)
    x = host_lib().synth_normal(8 * ne0, 79, t).reshape(8, ne0)
    ref = O.gemv(t, W, ne0, ne1, x, 8, threads=16)
    xb = gpu.put(np.ascontiguousarray(x))
    nan = np.full(8 * ne1, np.nan, np.float32)
    for n in (1, 2, 4, 8):
        ob = gpu.put(nan[:n * ne1])
        gpu.ok(gpu.L.qgpu_gemv_batch(T.h, xb.f32(), ne0, n, ob.f32(), ne1, 0))
        got = ob.download(np.float32).reshape(n, ne1)
        assert not np.isnan(got).any(), (fmt, shape, n)
        e = rel_err(got, ref[:n])
        print(f"  B={n}: rel err {e:.2e}", flush=True)
        assert e < 1e-3, (fmt, shape, n, e)
        gpu.ok(gpu.L.qgpu_gemv_batch(T.h, xb.f32(), ne0, n, ob.f32(), ne1, 0))
        again = ob.download(np.float32).reshape(n, ne1)
        assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), (fmt, shape, n)
        gpu.ok(gpu.L.qgpu_gemv_batch(T.h, xb.f32(), ne0, n, ob.f32(), ne1, 1))      # QGPU_GEMV_ACCUM
        acc = ob.download(np.float32).reshape(n, ne1)
        assert np.array_equal(acc.view(np.uint32), (got + got).view(np.uint32)), (fmt, shape, n)
    n = 4
    ob = gpu.put(nan[:n * ne1])
    gpu.sync()
    gpu.ok(gpu.L.qgpu_graph_begin())
    for _ in range(3):
        gpu.ok(gpu.L.qgpu_gemv_batch(T.h, xb.f32(), ne0, n, ob.f32(), ne1, 0))
    g = ctypes.c_void_p()
    gpu.ok(gpu.L.qgpu_graph_end(ctypes.byref(g)))
    eager = run(gpu, T, x, n, ne1)
    for _ in range(2):
        gpu.ok(gpu.L.qgpu_graph_launch(g))
        gpu.sync()
        assert np.array_equal(ob.download(np.float32).reshape(n, ne1).view(np.uint32), eager.view(np.uint32))
    gpu.ok(gpu.L.qgpu_graph_destroy(g))
