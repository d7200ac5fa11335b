"""qgpu_gemv_batch_noalloc (the allocation-free gemv_batch, static device
scratch) against qgpu_gemv_batch through the C-ABI: bit-identical outputs on two
calls in a row, the second with a smaller input (fewer tokens, fewer columns and
rows), then a third whose 272 tiles run their last 16 as half-K pairs on 256
compute units (the exchange slots in the scratch), for every weight format;
arguments past the scratch's limits rejected."""
import ctypes

import numpy as np
import pytest

from gpu_util import gpu  # noqa: F401
from qwen_pkg import host_lib

pytestmark = pytest.mark.gpu

FORMATS = {"IQ4_XS": 23, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_0": 8, "F32": 0}
_hip = None


def device_sync():
    """the entry point ran on the default stream: wait for the whole device"""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
    assert _hip.hipDeviceSynchronize() == 0


def run_pair(gpu, T, x, n, ne0, ne1):
    xb = gpu.put(np.ascontiguousarray(x[:n]))
    ob_lib, ob_na = gpu.buf(n * ne1 * 4), gpu.buf(n * ne1 * 4)
    gpu.ok(gpu.L.qgpu_gemv_batch(T.h, xb.f32(), ne0, n, ob_lib.f32(), ne1, 0))
    gpu.sync()
    gpu.ok(gpu.L.qgpu_gemv_batch_noalloc(T.h, xb.f32(), ne0, n, ob_na.f32(), ne1, 0, None))
    device_sync()
    return ob_lib.download(np.float32).reshape(n, ne1), ob_na.download(np.float32).reshape(n, ne1)


@pytest.mark.parametrize("fmt", list(FORMATS))
def test_noalloc_gemv_matches_gemv_batch(gpu, fmt):
    t = FORMATS[fmt]
    host = host_lib()
    print(f"\n[noalloc] {fmt}: 5120x1040 B=8, then 1024x272 B=3, then 5120x4352 B=4 (pair-split tail)", flush=True)
    for (ne0, ne1, n, seed) in ((5120, 1040, 8, 31), (1024, 272, 3, 32), (5120, 4352, 4, 33)):
        W = host.synth_matrix(t, ne0, ne1, seed, 200 + t, 0.02 if t else 1.0)
        T = gpu.tensor(W, t, ne0, ne1)
        x = host.synth_normal(8 * ne0, seed, 9).reshape(8, ne0)
        a, b = run_pair(gpu, T, x, n, ne0, ne1)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (fmt, ne0, ne1, n)
        assert np.abs(a).max() > 0
        T.close()


def test_noalloc_gemv_rejects_sizes_past_the_scratch(gpu):
    host = host_lib()
    ne0 = 65536 + 256                                      # one super-block past the digit planes
    W = host.synth_matrix(23, ne0, 16, 5, 5, 0.02)
    T = gpu.tensor(W, 23, ne0, 16)
    xb, ob = gpu.buf(ne0 * 4), gpu.buf(16 * 4)
    assert gpu.L.qgpu_gemv_batch_noalloc(T.h, xb.f32(), ne0, 1, ob.f32(), 16, 0, None) == -4  # QGPU_E_RANGE
    T.close()
    W = host.synth_matrix(23, 512, 16, 5, 6, 0.02)
    T = gpu.tensor(W, 23, 512, 16)
    xb, ob = gpu.buf(9 * 512 * 4), gpu.buf(9 * 16 * 4)
    assert gpu.L.qgpu_gemv_batch_noalloc(T.h, xb.f32(), 512, 9, ob.f32(), 16, 0, None) == -1  # QGPU_E_ARG: batch above 8
    T.close()
