"""ctypes bindings of the package's two native libraries.

  lib/libqgpu.so  -- the C-ABI HIP layer (include/qgpu.h), device pointers
  lib/libqwen.so  -- the C11 host library (include/gguf.h, quant.h, kernels.h,
                     model.h, qwen_synth.h) built on top of libqgpu

Both are built in-tree by build.py.  Nothing here falls back to a CPU
implementation: if a library is missing the loader raises.
"""
import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG, "lib")

F32P = ctypes.POINTER(ctypes.c_float)
U32P = ctypes.POINTER(ctypes.c_uint32)

GGML = {"F32": 0, "F16": 1, "Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_XS": 23}
BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 23: (256, 136)}


def row_bytes(t, ne0):
    be, bs = BLOCK[t]
    return ne0 // be * bs


def fptr(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(F32P)


class SynthSpec(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_uint32) for n in (
        "n_embd n_ff n_layer n_head n_kv_head head_dim n_k_heads n_v_heads state vocab "
        "rope_dim full_attn_interval context_len").split()]
        + [("rope_theta", ctypes.c_float), ("eps", ctypes.c_float)]
        + [(n, ctypes.c_int32) for n in "type_default type_embd type_output type_qkv type_eh_proj".split()]
        + [("gain_output", ctypes.c_float), ("seed", ctypes.c_uint64)])


class SynthTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("n_dims", ctypes.c_uint32), ("ne", ctypes.c_uint64 * 2),
                ("type", ctypes.c_int32), ("nbytes", ctypes.c_uint64), ("mu", ctypes.c_float),
                ("sigma", ctypes.c_float), ("neg_abs", ctypes.c_int32)]


def _load(name):
    path = os.path.join(LIB_DIR, name)
    if not os.path.exists(path):
        raise OSError(f"{path} is missing: run `python {os.path.join(PKG, 'build.py')}` "
                      "(or __graft_entry__.build()) first")
    return ctypes.CDLL(path)


class HostLib:
    """Host-side C11 library: generator, GGUF, scalar dequant."""

    def __init__(self):
        self.L = L = _load("libqwen.so")
        L.qwen_synth_matrix.argtypes = [ctypes.c_int32, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                        ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p, ctypes.c_int]
        L.qwen_synth_normal.argtypes = [F32P, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                        ctypes.c_float, ctypes.c_float]
        L.qwen_synth_write_gguf.argtypes = [ctypes.POINTER(SynthSpec), ctypes.c_char_p]
        L.qwen_synth_spec_tiny.argtypes = [ctypes.POINTER(SynthSpec), ctypes.c_uint64, ctypes.c_int]
        L.qwen_synth_spec_27b.argtypes = [ctypes.POINTER(SynthSpec), ctypes.c_uint64]
        L.qwen_synth_count.argtypes = [ctypes.POINTER(SynthSpec)]
        L.qwen_synth_count.restype = ctypes.c_uint32
        L.qwen_synth_describe.argtypes = [ctypes.POINTER(SynthSpec), ctypes.c_uint32, ctypes.POINTER(SynthTensor)]
        L.qwen_synth_fill.argtypes = [ctypes.POINTER(SynthSpec), ctypes.c_uint32, ctypes.c_void_p]
        L.qwen_f32_to_f16.argtypes = [ctypes.c_float]
        L.qwen_f32_to_f16.restype = ctypes.c_uint16
        L.dequant_row.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, F32P]
        L.fp16_to_f32.argtypes = [ctypes.c_uint16]
        L.fp16_to_f32.restype = ctypes.c_float

    def synth_matrix(self, t, ne0, ne1, seed, tid, sigma, threads=0):
        out = np.empty(row_bytes(t, ne0) * ne1, np.uint8)
        rc = self.L.qwen_synth_matrix(t, ne0, ne1, seed, tid, sigma, out.ctypes.data_as(ctypes.c_void_p), threads)
        if rc:
            raise ValueError("qwen_synth_matrix failed")
        return out

    def synth_normal(self, n, seed, tid, mu=0.0, sigma=1.0):
        out = np.empty(n, np.float32)
        self.L.qwen_synth_normal(fptr(out), n, seed, tid, mu, sigma)
        return out

    def spec_tiny(self, seed, mixed=0):
        s = SynthSpec()
        self.L.qwen_synth_spec_tiny(ctypes.byref(s), seed, mixed)
        return s

    def spec_27b(self, seed):
        s = SynthSpec()
        self.L.qwen_synth_spec_27b(ctypes.byref(s), seed)
        return s

    def write_gguf(self, spec, path):
        if self.L.qwen_synth_write_gguf(ctypes.byref(spec), path.encode()):
            raise OSError(f"writing {path} failed")

    def write_tiny_gguf(self, path, seed, mixed=0):
        self.write_gguf(self.spec_tiny(seed, mixed), path)

    def tensors(self, spec):
        n = self.L.qwen_synth_count(ctypes.byref(spec))
        out = []
        for i in range(n):
            t = SynthTensor()
            self.L.qwen_synth_describe(ctypes.byref(spec), i, ctypes.byref(t))
            out.append(t)
        return out

    def fill(self, spec, i, nbytes):
        buf = np.empty(nbytes, np.uint8)
        self.L.qwen_synth_fill(ctypes.byref(spec), i, buf.ctypes.data_as(ctypes.c_void_p))
        return buf

    def dequant_row(self, t, data, ne0):
        out = np.empty(ne0, np.float32)
        if self.L.dequant_row(t, data.ctypes.data_as(ctypes.c_void_p), ne0, fptr(out)):
            raise ValueError("unsupported type")
        return out


_host = None


def host_lib():
    global _host
    if _host is None:
        _host = HostLib()
    return _host


# ---------------------------------------------------------------------- GPU layer
class QgpuError(RuntimeError):
    pass


class DevBuf:
    """A device allocation owned by Python (freed on close/GC)."""

    def __init__(self, gpu, nbytes):
        self.gpu = gpu
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        gpu.ok(gpu.L.qgpu_malloc(ctypes.byref(p), max(1, self.nbytes)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, gpu, a):
        a = np.ascontiguousarray(a)
        b = cls(gpu, a.nbytes)
        gpu.ok(gpu.L.qgpu_memcpy_h2d(ctypes.c_void_p(b.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes))
        return b

    def upload(self, a, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        self.gpu.ok(self.gpu.L.qgpu_memcpy_h2d(ctypes.c_void_p(self.ptr + offset), a.ctypes.data_as(ctypes.c_void_p),
                                               a.nbytes))

    def download(self, dtype, count=None, offset=0):
        dt = np.dtype(dtype)
        count = (self.nbytes - offset) // dt.itemsize if count is None else count
        out = np.empty(count, dt)
        self.gpu.ok(self.gpu.L.qgpu_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr + offset),
                                               out.nbytes))
        return out

    def f32(self, offset_elems=0):
        return ctypes.cast(ctypes.c_void_p(self.ptr + 4 * offset_elems), F32P)

    def u32(self, offset_elems=0):
        return ctypes.cast(ctypes.c_void_p(self.ptr + 4 * offset_elems), U32P)

    def close(self):
        if self.ptr:
            self.gpu.L.qgpu_free(ctypes.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Tensor:
    def __init__(self, gpu, handle, t, ne0, ne1):
        self.gpu, self.h, self.type, self.ne0, self.ne1 = gpu, handle, t, ne0, ne1

    def close(self):
        if self.h:
            self.gpu.L.qgpu_tensor_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GpuLib:
    """libqgpu.so: the HIP C-ABI (include/qgpu.h)."""

    def __init__(self, device=0):
        self.L = L = _load("libqgpu.so")
        vp, u64, i32, f32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
        sigs = {
            "qgpu_init": [i32], "qgpu_sync": [], "qgpu_device_info": [ctypes.c_char_p, i32, ctypes.POINTER(i32),
                                                                     ctypes.POINTER(u64)],
            "qgpu_malloc": [ctypes.POINTER(vp), ctypes.c_size_t], "qgpu_free": [vp],
            "qgpu_memcpy_h2d": [vp, vp, ctypes.c_size_t], "qgpu_memcpy_d2h": [vp, vp, ctypes.c_size_t],
            "qgpu_memcpy_d2d": [vp, vp, ctypes.c_size_t], "qgpu_memset": [vp, i32, ctypes.c_size_t],
            "qgpu_event_create": [ctypes.POINTER(vp)], "qgpu_event_destroy": [vp], "qgpu_event_record": [vp],
            "qgpu_event_elapsed_ms": [vp, vp, ctypes.POINTER(f32)],
            "qgpu_graph_begin": [], "qgpu_graph_end": [ctypes.POINTER(vp)], "qgpu_graph_launch": [vp],
            "qgpu_graph_destroy": [vp],
            "qgpu_tensor_upload": [vp, i32, u64, u64, ctypes.POINTER(vp)],
            "qgpu_tensor_from_device": [vp, i32, u64, u64, ctypes.POINTER(vp)],
            "qgpu_tensor_free": [vp], "qgpu_tensor_download": [vp, vp],
            "qgpu_gemv_batch": [vp, F32P, u64, i32, F32P, u64, i32],
            "qgpu_gemv_multi_batch": [ctypes.POINTER(vp), i32, F32P, u64, i32, ctypes.POINTER(F32P),
                                      ctypes.POINTER(u64), i32],
            "qgpu_gemv_rows_batch": [vp, F32P, u64, i32, F32P, u64, u64, u64],
            "qgpu_dequant_rows": [vp, U32P, i32, F32P, u64],
            "qgpu_rmsnorm": [F32P, u64, F32P, u64, F32P, u64, i32, f32],
            "qgpu_l2norm": [F32P, u64, F32P, u64, u64, i32, f32],
            "qgpu_silu": [F32P, u64], "qgpu_sigmoid": [F32P, u64], "qgpu_softplus": [F32P, u64],
            "qgpu_softmax": [F32P, u64, u64, i32],
            "qgpu_silu_mul": [F32P, u64, F32P, u64, u64, i32],
            "qgpu_add": [F32P, u64, F32P, u64, u64, i32],
            "qgpu_argmax": [F32P, u64, ctypes.c_uint32, i32, U32P],
            "qgpu_gemv_prepare": [F32P, u64, i32, u64], "qgpu_gemv_prepared": [vp, i32, F32P, u64, i32],
            "qgpu_copy": [vp, vp, ctypes.c_size_t],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = i32
        L.qgpu_strerror.argtypes = [i32]
        L.qgpu_strerror.restype = ctypes.c_char_p
        L.qgpu_tensor_bytes.argtypes = [vp]
        L.qgpu_tensor_bytes.restype = u64
        self.ok(L.qgpu_init(device))

    def ok(self, rc):
        if rc != 0:
            raise QgpuError(f"qgpu error {rc}: {self.L.qgpu_strerror(rc).decode()}")
        return rc

    def device_info(self):
        name = ctypes.create_string_buffer(256)
        ncu, hbm = ctypes.c_int(), ctypes.c_uint64()
        self.ok(self.L.qgpu_device_info(name, 256, ctypes.byref(ncu), ctypes.byref(hbm)))
        return name.value.decode(), ncu.value, hbm.value

    def sync(self):
        self.ok(self.L.qgpu_sync())

    def buf(self, nbytes):
        return DevBuf(self, nbytes)

    def put(self, a):
        return DevBuf.from_array(self, a)

    def tensor(self, host_bytes, t, ne0, ne1):
        h = ctypes.c_void_p()
        self.ok(self.L.qgpu_tensor_upload(host_bytes.ctypes.data_as(ctypes.c_void_p), t, ne0, ne1, ctypes.byref(h)))
        return Tensor(self, h, t, ne0, ne1)

    def tensor_download(self, T):
        out = np.empty(row_bytes(T.type, T.ne0) * T.ne1, np.uint8)
        self.ok(self.L.qgpu_tensor_download(T.h, out.ctypes.data_as(ctypes.c_void_p)))
        return out

    def gemv(self, T, xbuf, ldx, n, obuf, ldo, flags=0):
        self.ok(self.L.qgpu_gemv_batch(T.h, xbuf.f32(), ldx, n, obuf.f32(), ldo, flags))

    def event(self):
        e = ctypes.c_void_p()
        self.ok(self.L.qgpu_event_create(ctypes.byref(e)))
        return e

    def record(self, e):
        self.ok(self.L.qgpu_event_record(e))

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        self.ok(self.L.qgpu_event_elapsed_ms(a, b, ctypes.byref(ms)))
        return ms.value


_gpu = None


def gpu_lib():
    global _gpu
    if _gpu is None:
        _gpu = GpuLib()
    return _gpu
