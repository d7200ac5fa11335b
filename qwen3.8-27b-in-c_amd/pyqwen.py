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


class Act(ctypes.Structure):
    """qgpu_act (include/qgpu.h): activation transform fused into the GEMV input preparation."""
    _fields_ = [("kind", ctypes.c_int), ("x", F32P), ("ldx", ctypes.c_uint64), ("y", F32P), ("ldy", ctypes.c_uint64),
                ("w", F32P), ("w2", F32P), ("seg", ctypes.c_uint64), ("eps", ctypes.c_float), ("xout", F32P),
                ("ldxo", ctypes.c_uint64), ("part", F32P), ("ldp", ctypes.c_uint64), ("n_part", ctypes.c_int),
                ("xnew", F32P), ("ldxn", ctypes.c_uint64), ("embd", ctypes.c_void_p),
                ("tok", ctypes.POINTER(ctypes.c_uint32))]


ACT_COPY, ACT_RMSNORM, ACT_SILU_MUL, ACT_GATED_NORM = 0, 1, 2, 3


class SynthSpec(ctypes.Structure):
    _fields_ = ([(n, ctypes.c_uint32) for n in (
        "n_embd n_ff n_layer n_head n_kv_head head_dim n_k_heads n_v_heads state vocab "
        "rope_dim full_attn_interval context_len").split()]
        + [("rope_theta", ctypes.c_float), ("eps", ctypes.c_float)]
        + [(n, ctypes.c_int32) for n in "type_default type_embd type_output type_qkv type_eh_proj".split()]
        + [("gain_output", ctypes.c_float), ("seed", ctypes.c_uint64)]
        + [("gain_embd", ctypes.c_float), ("gain_resid", ctypes.c_float), ("mtp_diag", ctypes.c_int32),
           ("norm_sigma", ctypes.c_float), ("tie_shift", ctypes.c_int32), ("tokenizer", ctypes.c_int32),
           ("tie_output", ctypes.c_int32)])


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

    def spec_27b_mix(self, seed):
        """the 27B hybrid with the real checkpoint's format mix (reference test_batch.c:16-20,
        test_kernels.c:120-126): token_embd Q4_K, attn_qkv Q5_K, output Q6_K, nextn.eh_proj Q8_0,
        every other 2-D weight IQ4_XS"""
        s = self.spec_27b(seed)
        s.type_embd, s.type_qkv, s.type_output, s.type_eh_proj = 12, 13, 14, 8
        return s

    def write_gguf(self, spec, path):
        if self.L.qwen_synth_write_gguf(ctypes.byref(spec), path.encode()):
            raise OSError(f"writing {path} failed")

    def write_tiny_gguf(self, path, seed, mixed=0, tokenizer=0):
        spec = self.spec_tiny(seed, mixed)
        spec.tokenizer = tokenizer
        self.write_gguf(spec, path)

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

    # Typed pointers into the buffer.  Each pointer holds a reference to the
    # buffer, so `gpu.put(a).f32()` passed straight to a call keeps the device
    # memory alive until the call returns (qgpu_free then waits for the device).
    def _ptr(self, offset_elems, typ):
        assert self.ptr, "buffer already freed"
        p = ctypes.cast(ctypes.c_void_p(self.ptr + 4 * offset_elems), typ)
        p._owner = self
        return p

    def f32(self, offset_elems=0):
        return self._ptr(offset_elems, F32P)

    def u32(self, offset_elems=0):
        return self._ptr(offset_elems, U32P)

    def u64(self, offset_elems=0):
        return self._ptr(offset_elems, ctypes.POINTER(ctypes.c_uint64))

    def i32(self, offset_elems=0):
        return self._ptr(offset_elems, ctypes.POINTER(ctypes.c_int))

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
            "qgpu_gemv_batch_noalloc": [vp, F32P, u64, i32, F32P, u64, i32, vp],
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
            "qgpu_sample": [F32P, ctypes.c_uint32, U32P, ctypes.c_uint32, f32, f32, ctypes.c_uint32, f32,
                            ctypes.c_uint32, ctypes.POINTER(u64), U32P],
            "qgpu_gemv_prepare": [F32P, u64, i32, u64], "qgpu_gemv_prepared": [vp, i32, F32P, u64, i32],
            "qgpu_copy": [vp, vp, ctypes.c_size_t],
            "qgpu_checksum": [vp, ctypes.c_size_t, U32P, i32], "qgpu_tensor_checksum": [vp, U32P, i32],
            "qgpu_gdn_conv": [F32P, u64, i32, i32, F32P, F32P, u64, i32, ctypes.POINTER(i32), F32P, u64],
            "qgpu_gdn_recurrence": [F32P, u64, F32P, F32P, u64, F32P, F32P, F32P, u64, i32, ctypes.POINTER(i32),
                                    i32, i32, i32, i32, f32, F32P, u64],
            "qgpu_rmsnorm_gated": [F32P, F32P, F32P, F32P, i32, i32, u64, f32],
            "qgpu_gdn_fused": [F32P, u64, i32, i32, F32P, F32P, u64, F32P, F32P, u64, F32P, F32P, F32P, u64, i32,
                               ctypes.POINTER(i32), i32, i32, i32, f32, F32P, u64],
            "qgpu_gdn_fused_planes": [F32P, u64, i32, i32, F32P, F32P, u64, F32P, F32P, u64, i32, u64, F32P, F32P,
                                      F32P, u64, i32, ctypes.POINTER(i32), i32, i32, i32, f32, F32P, u64],
            "qgpu_gdn_fused_factor": [F32P, u64, i32, i32, F32P, F32P, u64, F32P, F32P, u64, i32, u64, F32P, F32P,
                                      F32P, u64, i32, ctypes.POINTER(i32), i32, i32, i32, f32, F32P, u64, F32P, u64,
                                      ctypes.POINTER(i32), i32],
            "qgpu_gdn_materialize": [F32P, u64, i32, ctypes.POINTER(i32), i32, i32, i32, F32P, u64,
                                     ctypes.POINTER(i32)],
            "qgpu_attn_prep": [F32P, u64, F32P, F32P, u64, F32P, F32P, F32P, F32P, F32P, F32P, i32,
                               ctypes.POINTER(i32), i32, i32, i32, i32, f32],
            "qgpu_attn_decode": [F32P, u64, F32P, F32P, ctypes.POINTER(i32), i32, i32, i32, i32, i32, F32P, u64],
            "qgpu_attn_fused": [F32P, u64, F32P, F32P, u64, F32P, F32P, F32P, F32P, F32P, F32P, i32,
                                ctypes.POINTER(i32), i32, i32, i32, i32, i32, f32, F32P, u64],
            "qgpu_attn_fused_act": [F32P, u64, F32P, F32P, u64, F32P, F32P, F32P, F32P, F32P, F32P, i32,
                                    ctypes.POINTER(i32), i32, i32, i32, i32, i32, f32, F32P, u64],
            "qgpu_attn_fused_act_live": [F32P, u64, F32P, F32P, u64, F32P, F32P, F32P, F32P, F32P, F32P, i32,
                                         ctypes.POINTER(i32), i32, i32, i32, i32, i32, f32, F32P, u64, i32],
            "qgpu_attn_split_bound": [i32, i32, i32, i32],
            "qgpu_attn_reserve": [i32, i32],
            "qgpu_set_i32": [ctypes.POINTER(i32), i32],
            "qgpu_gemv_act_batch": [ctypes.POINTER(vp), i32, ctypes.POINTER(Act), i32, ctypes.POINTER(F32P),
                                    ctypes.POINTER(u64), i32],
            "qgpu_gemv_act_batch_ks": [ctypes.POINTER(vp), i32, ctypes.POINTER(Act), i32, ctypes.POINTER(F32P),
                                       ctypes.POINTER(u64), ctypes.POINTER(i32)],
            "qgpu_act_prepare": [ctypes.POINTER(Act), i32, u64],
            "qgpu_gemv_act_split": [vp, ctypes.POINTER(Act), i32, F32P, u64, i32],
            "qgpu_gemv_split_ks": [vp],
            "qgpu_gemv_prepared_split": [vp, i32, F32P, u64, i32],
            "qgpu_add_partials": [F32P, u64, F32P, u64, F32P, u64, i32, u64, i32],
            "qgpu_spec_accept": [U32P, U32P, i32, i32, ctypes.POINTER(i32), ctypes.POINTER(i32), i32, U32P],
            "qgpu_spec_accept_at": [U32P, U32P, i32, i32, i32, i32, ctypes.POINTER(i32), ctypes.POINTER(i32), i32,
                                    U32P],
            "qgpu_spec_accept_anchor": [U32P, U32P, i32, i32, i32, i32, ctypes.POINTER(i32), ctypes.POINTER(i32),
                                        i32, U32P, F32P, u64, i32, F32P, U32P, U32P],
            "qgpu_host_malloc": [ctypes.POINTER(vp), ctypes.c_size_t], "qgpu_host_free": [vp],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = i32
        L.qgpu_strerror.argtypes = [i32]
        L.qgpu_strerror.restype = ctypes.c_char_p
        L.qgpu_tensor_bytes.argtypes = [vp]
        L.qgpu_tensor_bytes.restype = u64
        L.qgpu_tensor_device_bytes.argtypes = [vp]
        L.qgpu_tensor_device_bytes.restype = u64
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


# ---------------------------------------------------------------------- model (include/model.h)
class GenStats(ctypes.Structure):
    _fields_ = [("n_cycles", ctypes.c_uint64), ("n_accepted", ctypes.c_uint64), ("n_drafts", ctypes.c_uint64),
                ("t_prefill_s", ctypes.c_double), ("t_decode_s", ctypes.c_double)]


def _model_lib():
    L = host_lib().L
    if getattr(L, "_model_sigs", False):
        return L
    vp, u32, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int
    L.qwen_model_alloc.restype = vp
    L.qwen_model_dealloc.argtypes = [vp]
    L.model_init.argtypes = [vp, ctypes.c_char_p, u32]
    L.model_init_synth.argtypes = [vp, ctypes.POINTER(SynthSpec), u32]
    L.model_free.argtypes = [vp]
    L.model_forward.argtypes = [vp, vp, u32, u32]
    L.model_forward_batch.argtypes = [vp, vp, U32P, u32, u32, i32]
    L.model_rollback_to.argtypes = [vp, u32]
    L.model_reset.argtypes = [vp]
    L.mtp_forward.argtypes = [vp, vp, u32, u32, i32]
    L.mtp_forward_batch.argtypes = [vp, vp, U32P, u32, u32, i32]
    L.qwen_model_field.argtypes = [vp, ctypes.c_char_p]
    L.qwen_model_field.restype = F32P
    L.qwen_model_get.argtypes = [vp, ctypes.c_char_p]
    L.qwen_model_get.restype = u32
    L.qwen_model_set_pos.argtypes = [vp, u32]
    L.qwen_model_set_host_sync.argtypes = [vp, i32]
    L.qwen_model_set_graphs.argtypes = [vp, i32]
    L.qwen_model_set_profile.argtypes = [vp, i32]
    L.model_generate_spec.argtypes = [vp, U32P, u32, u32, u32, u32, i32, U32P, U32P, ctypes.POINTER(GenStats)]
    L.model_generate_spec.restype = u32
    L.model_spec_begin.argtypes = [vp, U32P, u32, u32]
    L.model_spec_run.argtypes = [vp, u32, u32, i32, u32, u32, U32P, U32P, ctypes.POINTER(GenStats)]
    L.model_spec_run.restype = u32
    L.model_generate_greedy.argtypes = [vp, U32P, u32, u32, u32, U32P, ctypes.POINTER(GenStats)]
    L.model_generate_greedy.restype = u32
    L.model_generate_sample.argtypes = [vp, U32P, u32, u32, ctypes.c_float, ctypes.c_float, u32, ctypes.c_float,
                                        ctypes.c_uint64, u32, U32P, ctypes.POINTER(GenStats)]
    L.model_generate_sample.restype = u32
    L.model_time_steps.argtypes = [vp, u32, i32, F32P, F32P, F32P]
    L.qwen_model_status.argtypes = [vp]
    L.qwen_model_status.restype = i32
    L._model_sigs = True
    return L


def uptr(a):
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(U32P)


class Model:
    """The GPU model through the reference-compatible C API (include/model.h)."""

    def __init__(self, path=None, n_ctx=256, spec=None):
        gpu_lib()                                  # HIP layer must load (fails loudly otherwise)
        self.L = _model_lib()
        self.h = self.L.qwen_model_alloc()
        rc = self.L.model_init_synth(self.h, ctypes.byref(spec), n_ctx) if spec is not None else \
            self.L.model_init(self.h, path.encode(), n_ctx)
        if rc:
            self.L.qwen_model_dealloc(self.h)
            self.h = None
            raise QgpuError(f"model_init failed ({path or 'synthetic'})")
        self.V = self.L.qwen_model_get(self.h, b"vocab")
        self.E = self.L.qwen_model_get(self.h, b"n_embd")

    def set_profile(self, on):
        self.L.qwen_model_set_profile(self.h, 1 if on else 0)

    def prof_counters(self):
        """the reference's section counters (seconds) and model_forward call count"""
        out = {k: ctypes.c_double.in_dll(self.L, f"qwen_prof_{k}").value for k in ("embed", "gdn", "attn", "head")}
        out["calls"] = ctypes.c_uint64.in_dll(self.L, "qwen_prof_calls").value
        return out

    def status(self):
        """0 = last call done, -1 = rejected on the host, -2 = device error (include/model.h)"""
        return self.L.qwen_model_status(self.h)

    def set_graphs(self, on):
        """replay captured launch sequences (HIP graphs) of the forward / MTP bodies (default off)"""
        self.L.qwen_model_set_graphs(self.h, 1 if on else 0)

    def close(self):
        if self.h:
            self.L.model_free(self.h)
            self.L.qwen_model_dealloc(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def field(self, name, n):
        return np.ctypeslib.as_array(self.L.qwen_model_field(self.h, name.encode()), shape=(n,)).copy()

    @property
    def pos(self):
        return self.L.qwen_model_get(self.h, b"pos")

    @pos.setter
    def pos(self, p):
        self.L.qwen_model_set_pos(self.h, p)

    def forward(self, tok, pos):
        self.L.model_forward(self.h, None, tok, pos)
        return self.field("logits", self.V)

    def forward_batch(self, toks, pos, ckpt=1):
        t = np.ascontiguousarray(toks, np.uint32)
        self.L.model_forward_batch(self.h, None, uptr(t), pos, len(t), ckpt)
        return self.field("logits_b", len(t) * self.V).reshape(len(t), self.V)

    def h_save(self, B):
        return self.field("h_save", B * self.E).reshape(B, self.E)

    def reset(self):
        self.L.model_reset(self.h)

    def rollback_to(self, b):
        self.L.model_rollback_to(self.h, b)

    def mtp_forward(self, tok, pos, want_logits=1):
        self.L.mtp_forward(self.h, None, tok, pos, want_logits)
        return self.field("logits", self.V) if want_logits else None

    def mtp_forward_batch(self, toks, pos, want_logits=0):
        t = np.ascontiguousarray(toks, np.uint32)
        self.L.mtp_forward_batch(self.h, None, uptr(t), pos, len(t), want_logits)

    def generate_spec(self, prompt, n_predict, k, eos=0xFFFFFFFF, force_accept=False):
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_predict + 16, np.uint32)
        js = np.zeros(n_predict + 16, np.uint32)
        st = GenStats()
        n = self.L.model_generate_spec(self.h, uptr(p), len(p), n_predict, k, eos, int(force_accept), uptr(out),
                                       uptr(js), ctypes.byref(st))
        return out[:n], js[:st.n_cycles], st

    def spec_begin(self, prompt, k):
        p = np.ascontiguousarray(prompt, np.uint32)
        if self.L.model_spec_begin(self.h, uptr(p), len(p), k):
            raise QgpuError("model_spec_begin failed")

    def spec_run(self, k, max_cycles, max_tokens=None, force_accept=0, eos=0xFFFFFFFF):
        """continue the speculative loop: returns (tokens, accepted index per cycle, stats)"""
        max_tokens = max_cycles * (k + 1) if max_tokens is None else max_tokens
        out = np.zeros(max_tokens + 16, np.uint32)
        js = np.zeros(max_cycles + 16, np.uint32)
        st = GenStats()
        n = self.L.model_spec_run(self.h, k, eos, int(force_accept), max_cycles, max_tokens, uptr(out), uptr(js),
                                  ctypes.byref(st))
        return out[:n], js[:st.n_cycles], st

    def generate_greedy(self, prompt, n_predict, eos=0xFFFFFFFF):
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_predict, np.uint32)
        st = GenStats()
        n = self.L.model_generate_greedy(self.h, uptr(p), len(p), n_predict, eos, uptr(out), ctypes.byref(st))
        return out[:n], st

    def generate_sample(self, prompt, n_predict, temp, top_p, top_k, repeat_penalty, seed, eos=0xFFFFFFFF):
        """Prefill, then the sampled decode of main.c:232-248 with the sampler on the device."""
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_predict, np.uint32)
        st = GenStats()
        n = self.L.model_generate_sample(self.h, uptr(p), len(p), n_predict, temp, top_p, top_k, repeat_penalty,
                                         seed, eos, uptr(out), ctypes.byref(st))
        return out[:n], st

    def time_steps(self, B, reps):
        v, d, dr = ctypes.c_float(), ctypes.c_float(), ctypes.c_float()
        if self.L.model_time_steps(self.h, B, reps, ctypes.byref(v), ctypes.byref(d), ctypes.byref(dr)):
            raise QgpuError("model_time_steps failed")
        return v.value, d.value, dr.value
