"""GPU parity of the HIP kernels through the C-ABI (libqgpu.so), checked
against the reference's golden vectors (tests/golden, produced from the
compiled reference) and the oracle.

Bars: dequantisation and argmax decisions bit-exact; GEMV outputs
within 1e-3 relative of the reference.  Relative error is normwise per call:
max|got - ref| / max|ref|.  The measured error of the matrix-core IQ4_XS path
is ~1e-7, so the tests also hold it to GEMV_TIGHT to catch partial mistakes.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle_lib as O
from gpu_util import gpu, rel_err  # noqa: F401
from qwen_pkg import host_lib, pyqwen

pytestmark = pytest.mark.gpu

FORMATS = ["F32", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "IQ4_XS"]
GEMV_TOL = 1e-3          # contract
GEMV_TIGHT = 2e-5        # what the kernels actually achieve (fp32 accumulation)


def load(name):
    return np.load(os.path.join(O.GOLDEN, name), allow_pickle=False)


def run_gemv(gpu, T, x, n, flags=0, out_init=None):
    ne0, ne1 = T.ne0, T.ne1
    xb = gpu.put(np.ascontiguousarray(x[:n], np.float32))
    ob = gpu.put(np.zeros((n, ne1), np.float32) if out_init is None else out_init.astype(np.float32))
    gpu.gemv(T, xb, ne0, n, ob, ne1, flags)
    return ob.download(np.float32).reshape(n, ne1)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("shape", ["512x64", "5120x32"])
def test_gemv_vs_reference_golden(gpu, fmt, shape):
    print(f"\n[gemv] {fmt} {shape}", flush=True)
    z = load(f"gemv_{fmt}_{shape}.npz")
    ne0, ne1 = map(int, shape.split("x"))
    T = gpu.tensor(z["W"], int(z["type"]), ne0, ne1)
    for n in range(1, 9):
        got = run_gemv(gpu, T, z["x"], n)
        for t in range(n):
            e = rel_err(got[t], z["out_batch"][t])
            assert e < GEMV_TOL, (fmt, n, t, e)
            assert e < GEMV_TIGHT, (fmt, n, t, e)


@pytest.mark.parametrize("fmt", FORMATS)
def test_tensor_repack_roundtrip(gpu, fmt):
    z = load(f"gemv_{fmt}_5120x32.npz")
    T = gpu.tensor(z["W"], int(z["type"]), 5120, 32)
    assert np.array_equal(gpu.tensor_download(T), z["W"])


@pytest.mark.parametrize("nbytes,n", [(16, 1), (16, 3), (4096, 7), (1 << 20, 2048),
                                      ((47710208 // 16) * 16 + 16 * 999, 2048)])
def test_checksum_is_the_xor_of_the_words(gpu, nbytes, n):
    """qgpu_checksum: the XOR of the n per-block partials is the XOR of the 32-bit words, for
    buffers smaller than one block, within the grid and past it (grid-stride tail)"""
    a = np.random.default_rng(nbytes % 1000).integers(0, 2 ** 32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    src, part = gpu.put(a), gpu.put(np.full(n, 0xDEADBEEF, np.uint32))
    gpu.ok(gpu.L.qgpu_checksum(ctypes.c_void_p(src.ptr), nbytes, part.u32(), n))
    assert np.bitwise_xor.reduce(part.download(np.uint32)) == np.bitwise_xor.reduce(a)
    assert gpu.L.qgpu_checksum(ctypes.c_void_p(src.ptr), 12, part.u32(), n) == -1      # QGPU_E_ARG
    assert gpu.L.qgpu_checksum(ctypes.c_void_p(src.ptr), nbytes, part.u32(), 0) == -1


def test_tensor_checksum_of_unpacked_rows(gpu):
    """a tensor kept in GGUF rows on the device (F32) checksums to the XOR of the uploaded bytes"""
    z = load("gemv_F32_512x64.npz")
    T = gpu.tensor(z["W"], int(z["type"]), 512, 64)
    part = gpu.put(np.zeros(64, np.uint32))
    assert gpu.L.qgpu_tensor_device_bytes(T.h) == z["W"].nbytes
    gpu.ok(gpu.L.qgpu_tensor_checksum(T.h, part.u32(), 64))
    assert np.bitwise_xor.reduce(part.download(np.uint32)) == \
        np.bitwise_xor.reduce(np.frombuffer(z["W"].tobytes(), np.uint32))


@pytest.mark.parametrize("fmt", FORMATS)
def test_dequant_rows_bitexact(gpu, fmt):
    z = load(f"gemv_{fmt}_512x64.npz")
    T = gpu.tensor(z["W"], int(z["type"]), 512, 64)
    rows = np.array([0, 5, 17, 63, 31, 1000000], np.uint32)        # last id out of range -> zeros
    rb = gpu.put(rows)
    ob = gpu.buf(len(rows) * 512 * 4)
    gpu.ok(gpu.L.qgpu_dequant_rows(T.h, rb.u32(), len(rows), ob.f32(), 512))
    got = ob.download(np.float32).reshape(len(rows), 512)
    assert np.array_equal(got[:5], z["deq"][rows[:5]])
    assert np.all(got[5] == 0)


@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_K", "Q5_K", "Q6_K", "IQ4_XS"])
def test_gemv_unit_vector_probe(gpu, fmt):
    """debug_kernels.c:22-28 pattern: x = e_i returns the dequantised column i exactly."""
    z = load(f"gemv_{fmt}_512x64.npz")
    T = gpu.tensor(z["W"], int(z["type"]), 512, 64)
    for batch in ([0, 1, 7, 8], [15, 16, 31, 32], [100, 255, 256, 511]):
        x = np.zeros((4, 512), np.float32)
        for k, i in enumerate(batch):
            x[k, i] = 1.0
        got = run_gemv(gpu, T, x, 4)
        for k, i in enumerate(batch):
            assert np.array_equal(got[k], z["deq"][:, i]), (fmt, i)


def test_gemv_multi_accum_rows(gpu):
    host = host_lib()
    ne0 = 1024
    shapes = [(23, 96), (23, 48), (23, 200), (12, 64)]        # IQ4_XS x3 + Q4_K (two launch groups)
    Ws, Ts = [], []
    for k, (t, rows) in enumerate(shapes):
        W = host.synth_matrix(t, ne0, rows, 77, k, 0.02)
        Ws.append(W)
        Ts.append(gpu.tensor(W, t, ne0, rows))
    x = host.synth_normal(5 * ne0, 9, 1).reshape(5, ne0)
    xb = gpu.put(x)
    outs = [gpu.put(np.zeros((5, r + 3), np.float32)) for _, r in shapes]
    VP = ctypes.c_void_p * 4
    FP = pyqwen.F32P * 4
    LD = ctypes.c_uint64 * 4
    gpu.ok(gpu.L.qgpu_gemv_multi_batch(VP(*[T.h for T in Ts]), 4, xb.f32(), ne0, 5,
                                       FP(*[o.f32() for o in outs]), LD(*[r + 3 for _, r in shapes]), 0))
    for k, (t, rows) in enumerate(shapes):
        got = outs[k].download(np.float32).reshape(5, rows + 3)
        ref = O.gemv(t, Ws[k], ne0, rows, x, 5)
        assert rel_err(got[:, :rows], ref) < GEMV_TIGHT
        assert np.all(got[:, rows:] == 0)
    # accumulate into a residual
    base = np.arange(5 * 96, dtype=np.float32).reshape(5, 96)
    got = run_gemv(gpu, Ts[0], x, 5, pyqwen_accum(), out_init=base)
    assert rel_err(got - base, O.gemv(23, Ws[0], ne0, 96, x, 5)) < 1e-4
    # row range [17, 70)
    ob = gpu.put(np.full((5, 96), -7, np.float32))
    gpu.ok(gpu.L.qgpu_gemv_rows_batch(Ts[0].h, xb.f32(), ne0, 5, ob.f32(), 96, 17, 70))
    got = ob.download(np.float32).reshape(5, 96)
    ref = O.gemv(23, Ws[0], ne0, 96, x, 5)
    assert np.all(got[:, :17] == -7) and np.all(got[:, 70:] == -7)
    assert rel_err(got[:, 17:70], ref[:, 17:70]) < GEMV_TIGHT


@pytest.mark.parametrize("n", [1, 3, 4, 6, 8])
def test_gemv_wide_grids(gpu, n):
    """Wide IQ4_XS grids against the oracle: a single 32768-row matrix (2048 row tiles), a multi-GEMV of
    two 16400-row matrices (1025 tiles each, an odd count per matrix), and an accumulate into the
    outputs."""
    print(f"\n[gemv] wide grids, B={n}", flush=True)
    host = host_lib()
    ne0 = 512
    x = host.synth_normal(8 * ne0, 13, 2).reshape(8, ne0)
    W = host.synth_matrix(23, ne0, 32768, 5, 1, 0.02)
    T = gpu.tensor(W, 23, ne0, 32768)
    got = run_gemv(gpu, T, x, n)
    assert rel_err(got, O.gemv(23, W, ne0, 32768, x, n)) < GEMV_TIGHT
    Ws = [host.synth_matrix(23, ne0, 16400, 6, k, 0.02) for k in range(2)]
    Ts = [gpu.tensor(Wk, 23, ne0, 16400) for Wk in Ws]
    xb = gpu.put(np.ascontiguousarray(x[:n]))
    outs = [gpu.put(np.zeros((n, 16400), np.float32)) for _ in range(2)]
    gpu.ok(gpu.L.qgpu_gemv_multi_batch((ctypes.c_void_p * 2)(*[t.h for t in Ts]), 2, xb.f32(), ne0, n,
                                       (pyqwen.F32P * 2)(*[o.f32() for o in outs]),
                                       (ctypes.c_uint64 * 2)(16400, 16400), 0))
    for k in range(2):
        ref = O.gemv(23, Ws[k], ne0, 16400, x, n)
        assert rel_err(outs[k].download(np.float32).reshape(n, 16400), ref) < GEMV_TIGHT, k
    base = np.arange(n * 32768, dtype=np.float32).reshape(n, 32768) * 1e-3
    got = run_gemv(gpu, T, x, n, pyqwen_accum(), out_init=base)
    assert rel_err(got - base, O.gemv(23, W, ne0, 32768, x, n)) < 1e-4


def pyqwen_accum():
    return 1   # QGPU_GEMV_ACCUM


def test_gemv_config1_shape_vs_oracle(gpu):
    """Config 1: IQ4_XS 17408x5120, d ~ |N(0,0.02)|, x ~ N(0,1), B = 4; plus B = 1 and 8."""
    host = host_lib()
    W = host.synth_matrix(23, 5120, 17408, 1, 0, 0.02)
    x = host.synth_normal(8 * 5120, 1, 1).reshape(8, 5120)
    T = gpu.tensor(W, 23, 5120, 17408)
    ref = O.gemv(23, W, 5120, 17408, x, 8)
    for n in (1, 4, 8):
        got = run_gemv(gpu, T, x, n)
        for t in range(n):
            assert rel_err(got[t], ref[t]) < GEMV_TIGHT, (n, t)


def test_gemv_rejects_bad_args(gpu):
    host = host_lib()
    W = host.synth_matrix(23, 512, 32, 3, 3, 0.02)
    T = gpu.tensor(W, 23, 512, 32)
    xb = gpu.put(np.zeros((9, 512), np.float32))
    ob = gpu.put(np.zeros((9, 32), np.float32))
    assert gpu.L.qgpu_gemv_batch(T.h, xb.f32(), 512, 9, ob.f32(), 32, 0) != 0      # n > 8
    assert gpu.L.qgpu_gemv_batch(T.h, xb.f32(), 256, 2, ob.f32(), 32, 0) != 0      # ldx < ne0
    assert gpu.L.qgpu_gemv_batch(T.h, xb.f32(), 512, 2, ob.f32(), 16, 0) != 0      # ldo < rows
    h = ctypes.c_void_p()
    assert gpu.L.qgpu_tensor_upload(W.ctypes.data_as(ctypes.c_void_p), 23, 500, 32, ctypes.byref(h)) != 0
    assert gpu.L.qgpu_tensor_upload(W.ctypes.data_as(ctypes.c_void_p), 2, 512, 32, ctypes.byref(h)) != 0


# ---------------------------------------------------------------- ops
def test_ops_vs_reference_golden(gpu):
    z = load("ops.npz")
    for n in z["dims"]:
        n = int(n)
        x, w = z[f"x_{n}"], z[f"w_{n}"]
        xb, wb, ob = gpu.put(x), gpu.put(w), gpu.buf(4 * n)
        gpu.ok(gpu.L.qgpu_rmsnorm(ob.f32(), n, xb.f32(), n, wb.f32(), n, 1, 1e-6))
        assert np.allclose(ob.download(np.float32), z[f"rmsnorm_{n}"], rtol=1e-5, atol=1e-6)
        gpu.ok(gpu.L.qgpu_l2norm(ob.f32(), n, xb.f32(), n, n, 1, 1e-6))
        assert np.allclose(ob.download(np.float32), z[f"l2norm_{n}"], rtol=1e-5, atol=1e-7)
        for f in ("silu", "sigmoid", "softplus"):
            yb = gpu.put(x)
            gpu.ok(getattr(gpu.L, f"qgpu_{f}")(yb.f32(), n))
            assert np.allclose(yb.download(np.float32), z[f"{f}_{n}"], rtol=1e-5, atol=1e-6), (f, n)
        yb = gpu.put(x)
        gpu.ok(gpu.L.qgpu_softmax(yb.f32(), n, n, 1))
        assert np.allclose(yb.download(np.float32), z[f"softmax_{n}"], rtol=1e-4, atol=1e-8), n
    xr = z["x_range"]
    for f in ("silu", "sigmoid", "softplus"):
        yb = gpu.put(xr)
        gpu.ok(getattr(gpu.L, f"qgpu_{f}")(yb.f32(), xr.size))
        got = yb.download(np.float32)
        ref = z[f"{f}_range"]
        assert np.allclose(got, ref, rtol=2e-5, atol=1e-30), f


def test_ops_known_answers(gpu):
    """test_ops.c:98-169 known answers on the device ops."""
    def dev(a):
        return gpu.put(np.asarray(a, np.float32))
    o = gpu.buf(16)
    gpu.ok(gpu.L.qgpu_rmsnorm(o.f32(), 4, dev([1, 1, 1, 1]).f32(), 4, dev([2, 2, 2, 2]).f32(), 4, 1, 0.0))
    assert np.allclose(o.download(np.float32), 2.0, rtol=1e-6)
    gpu.ok(gpu.L.qgpu_l2norm(o.f32(), 2, dev([3, 4]).f32(), 2, 2, 1, 1e-5))
    assert np.allclose(o.download(np.float32, 2), [0.6, 0.8], rtol=1e-6)
    s = dev([0, 2, -20, 20])
    gpu.ok(gpu.L.qgpu_silu(s.f32(), 4))
    assert np.allclose(s.download(np.float32), [0, 2 / (1 + np.exp(-2)), -20 * np.exp(-20), 20], rtol=1e-4)
    g = dev([0, 100, -100, 1, -1])
    gpu.ok(gpu.L.qgpu_sigmoid(g.f32(), 5))
    assert np.allclose(g.download(np.float32), [0.5, 1, 0, 1 / (1 + np.e ** -1), 1 / (1 + np.e)], rtol=1e-6,
                       atol=1e-30)
    sp = dev([0, 1, -50, 50, 100, 1000])
    gpu.ok(gpu.L.qgpu_softplus(sp.f32(), 6))
    assert np.allclose(sp.download(np.float32), [np.log(2), np.log1p(np.e), np.exp(-50), 50, 100, 1000], rtol=1e-5)
    sm = dev([1000] * 4)
    gpu.ok(gpu.L.qgpu_softmax(sm.f32(), 4, 4, 1))
    assert np.allclose(sm.download(np.float32), 0.25, rtol=1e-6)


def test_argmax_bitexact_decisions(gpu):
    rng = np.random.default_rng(3)
    V = 248320
    L = rng.standard_normal((8, V)).astype(np.float32)
    L[1, 1000] = L[1, 200000] = 50.0                 # tie: lowest index wins
    L[2, :] = 0.0                                    # all equal -> 0
    L[3, V - 1] = 99.0
    L[4, 0] = 99.0
    L[5] = -np.abs(L[5]) - 1                         # all negative
    lb, ob = gpu.put(L), gpu.buf(8 * 4)
    gpu.ok(gpu.L.qgpu_argmax(lb.f32(), V, V, 8, ob.u32()))
    got = ob.download(np.uint32)
    ref = [O.lib().or_argmax(O.fptr(np.ascontiguousarray(L[r])), V) for r in range(8)]
    assert list(got) == ref
    assert got[1] == 1000 and got[2] == 0 and got[3] == V - 1 and got[4] == 0
    # tiny vocab, fewer elements than partial chunks
    small = np.array([[3, 1, 3], [-1, -1, -2]], np.float32)
    sb, o2 = gpu.put(small), gpu.buf(8)
    gpu.ok(gpu.L.qgpu_argmax(sb.f32(), 3, 3, 2, o2.u32()))
    assert list(o2.download(np.uint32)) == [0, 0]
