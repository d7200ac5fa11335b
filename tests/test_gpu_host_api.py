"""The reference-compatible host-pointer API (include/kernels.h: gemv_batch,
gemv_multi_batch, gemv_rows_batch, gemv, ops) computed on the GPU, against the
golden vectors produced by the compiled reference (tests/golden).  Bars: GEMV
within 1e-3 normwise of the reference's gemv_batch; ops within the reference
test tolerances."""
import ctypes
import os

import numpy as np
import pytest

import oracle_lib as O
from gpu_util import gpu, rel_err  # noqa: F401
from qwen_pkg import host_lib

pytestmark = pytest.mark.gpu
F32P = ctypes.POINTER(ctypes.c_float)


class TI(ctypes.Structure):
    """gguf_tensor_info_t (include/gguf.h)"""
    _fields_ = [("name", ctypes.c_char * 64), ("n_dims", ctypes.c_uint32), ("ne", ctypes.c_uint64 * 4),
                ("type", ctypes.c_int), ("offset", ctypes.c_uint64), ("data", ctypes.c_void_p)]


def lib():
    L = host_lib().L
    L.gemv_batch.argtypes = [ctypes.c_void_p, ctypes.POINTER(TI), F32P, ctypes.c_uint64, ctypes.c_int, F32P,
                             ctypes.c_uint64]
    L.gemv.argtypes = [ctypes.c_void_p, ctypes.POINTER(TI), F32P, F32P]
    L.gemv_rows_batch.argtypes = [ctypes.POINTER(TI), F32P, ctypes.c_uint64, ctypes.c_int, F32P, ctypes.c_uint64,
                                  ctypes.c_uint64, ctypes.c_uint64]
    L.gemv_multi_batch.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.POINTER(TI)), F32P, ctypes.c_uint64,
                                   ctypes.c_int, ctypes.POINTER(F32P), ctypes.POINTER(ctypes.c_uint64), ctypes.c_int]
    L.rmsnorm.argtypes = [F32P, F32P, F32P, ctypes.c_uint64, ctypes.c_float]
    L.l2norm.argtypes = [F32P, F32P, ctypes.c_uint64, ctypes.c_float]
    for f in ("silu_inplace", "sigmoid_inplace", "softplus_inplace", "softmax_inplace"):
        getattr(L, f).argtypes = [F32P, ctypes.c_uint64]
    L.kernels_release_weights.argtypes = []
    return L


def ti(W, t, ne0, ne1, name=b"w"):
    d = TI(name=name, n_dims=2, type=t, offset=0, data=W.ctypes.data_as(ctypes.c_void_p))
    d.ne[0], d.ne[1], d.ne[2], d.ne[3] = ne0, ne1, 1, 1
    return d


def fp(a):
    return a.ctypes.data_as(F32P)


@pytest.mark.parametrize("fmt", ["IQ4_XS", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "F32"])
def test_host_gemv_batch_vs_reference(gpu, fmt):
    L = lib()
    z = np.load(os.path.join(O.GOLDEN, f"gemv_{fmt}_5120x32.npz"), allow_pickle=False)
    W, x = z["W"], np.ascontiguousarray(z["x"])
    t, (n, ne0), ne1 = int(z["type"]), x.shape, z["out_batch"].shape[1]
    d = ti(W, t, ne0, ne1)
    out = np.zeros((n, ne1), np.float32)
    L.gemv_batch(None, ctypes.byref(d), fp(x), ne0, n, fp(out), ne1)
    assert rel_err(out, z["out_batch"]) < 1e-3
    one = np.zeros(ne1, np.float32)
    L.gemv(None, ctypes.byref(d), fp(x[0]), fp(one))
    assert rel_err(one, z["out_single"][0]) < 1e-3
    rows = np.zeros((n, ne1), np.float32)
    L.gemv_rows_batch(ctypes.byref(d), fp(x), ne0, n, fp(rows), ne1, 5, 21)
    assert rel_err(rows[:, 5:21], z["out_batch"][:, 5:21]) < 1e-3
    assert not rows[:, :5].any() and not rows[:, 21:].any()
    # multi: the same matrix twice with different output strides
    o1, o2 = np.zeros((n, ne1), np.float32), np.zeros((n, ne1 + 7), np.float32)
    ptrs = (ctypes.POINTER(TI) * 2)(ctypes.pointer(d), ctypes.pointer(d))
    outs = (F32P * 2)(fp(o1), fp(o2))
    lds = (ctypes.c_uint64 * 2)(ne1, ne1 + 7)
    L.gemv_multi_batch(None, ptrs, fp(x), ne0, n, outs, lds, 2)
    assert rel_err(o1, z["out_batch"]) < 1e-3 and rel_err(o2[:, :ne1], z["out_batch"]) < 1e-3
    L.kernels_release_weights()


def test_host_ops_vs_reference(gpu):
    L = lib()
    z = np.load(os.path.join(O.GOLDEN, "ops.npz"), allow_pickle=False)
    for n in z["dims"]:
        n = int(n)
        x, w = np.ascontiguousarray(z[f"x_{n}"]), np.ascontiguousarray(z[f"w_{n}"])
        out = np.zeros(n, np.float32)
        L.rmsnorm(fp(out), fp(x), fp(w), n, 1e-6)
        assert np.allclose(out, z[f"rmsnorm_{n}"], rtol=1e-5, atol=1e-6)
        L.l2norm(fp(out), fp(x), n, 1e-6)
        assert np.allclose(out, z[f"l2norm_{n}"], rtol=1e-5, atol=1e-7)
        for f in ("silu", "sigmoid", "softplus", "softmax"):
            y = x.copy()
            getattr(L, f + "_inplace")(fp(y), n)
            assert np.allclose(y, z[f"{f}_{n}"], rtol=1e-5, atol=1e-6), (f, n)
