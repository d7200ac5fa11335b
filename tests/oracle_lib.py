"""ctypes handle on the oracle (oracle/liboracle.so): the CPU restatement of the
reference used as the checker.  Test infrastructure only."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libqwenref.so")
GOLDEN = os.path.join(ROOT, "tests", "golden")

F32P = ctypes.POINTER(ctypes.c_float)
U32P = ctypes.POINTER(ctypes.c_uint32)


def fptr(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(F32P)


def uptr(a):
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(U32P)


class SpecStats(ctypes.Structure):
    _fields_ = [("n_cycles", ctypes.c_uint64), ("n_accepted", ctypes.c_uint64), ("n_drafts", ctypes.c_uint64)]


class Sampler(ctypes.Structure):
    """or_sampler_t (the layout of the reference's sampler_t, sampler.h:7-14)."""
    _fields_ = [("temp", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("repeat_penalty", ctypes.c_float), ("repeat_last_n", ctypes.c_uint32), ("rng_state", ctypes.c_uint64)]


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(ORACLE_SO):
        import subprocess
        subprocess.check_call(["make", "-C", os.path.join(ROOT, "oracle"), "-s"])
    L = ctypes.CDLL(ORACLE_SO)
    vp, u64, i32, f32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
    L.or_fp16_to_f32.argtypes = [ctypes.c_uint16]
    L.or_fp16_to_f32.restype = f32
    L.or_row_bytes.argtypes = [i32, u64]
    L.or_row_bytes.restype = ctypes.c_size_t
    L.or_dequant_row.argtypes = [i32, vp, u64, F32P]
    L.or_gemv_rows_batch.argtypes = [i32, vp, u64, F32P, u64, i32, F32P, u64, u64, u64]
    L.or_gemv_batch.argtypes = [i32, vp, u64, u64, F32P, u64, i32, F32P, u64, i32]
    L.or_rmsnorm.argtypes = [F32P, F32P, F32P, u64, f32]
    L.or_l2norm.argtypes = [F32P, F32P, u64, f32]
    for f in ("or_silu_inplace", "or_sigmoid_inplace", "or_softplus_inplace", "or_softmax_inplace"):
        getattr(L, f).argtypes = [F32P, u64]
    L.or_exp8_lane.argtypes = [f32]
    L.or_exp8_lane.restype = f32
    L.or_argmax.argtypes = [F32P, ctypes.c_uint32]
    L.or_argmax.restype = ctypes.c_uint32
    L.or_gdn_block.argtypes = [i32, i32, i32, i32, i32, i32, f32, F32P, F32P, F32P, F32P, F32P, F32P,
                               F32P, F32P, F32P, F32P, F32P]
    L.or_model_open.argtypes = [ctypes.c_char_p, ctypes.c_uint32, ctypes.c_uint32]
    L.or_model_open.restype = vp
    L.or_model_close.argtypes = [vp]
    for f in ("or_model_logits", "or_model_logits_b", "or_model_h_save", "or_model_mtp_h", "or_model_x"):
        getattr(L, f).argtypes = [vp]
        getattr(L, f).restype = F32P
    for f in ("or_model_ssm_state", "or_model_conv_state"):
        getattr(L, f).argtypes = [vp, i32]
        getattr(L, f).restype = F32P
    L.or_model_vocab.argtypes = [vp]
    L.or_model_vocab.restype = ctypes.c_uint32
    L.or_model_n_embd.argtypes = [vp]
    L.or_model_pos.argtypes = [vp]
    L.or_model_pos.restype = ctypes.c_uint32
    L.or_model_set_pos.argtypes = [vp, ctypes.c_uint32]
    L.or_model_set_threads.argtypes = [vp, i32]
    L.or_model_forward.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32]
    L.or_model_forward_batch.argtypes = [vp, U32P, ctypes.c_uint32, ctypes.c_uint32, i32]
    L.or_model_rollback_to.argtypes = [vp, ctypes.c_uint32]
    L.or_mtp_forward.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32, i32]
    L.or_mtp_forward_batch.argtypes = [vp, U32P, ctypes.c_uint32, ctypes.c_uint32, i32]
    L.or_generate_spec.argtypes = [vp, U32P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                   ctypes.c_uint32, U32P, ctypes.POINTER(SpecStats), U32P]
    L.or_generate_spec.restype = ctypes.c_uint32
    L.or_generate_spec_ex.argtypes = [vp, U32P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.c_uint32, i32, U32P, ctypes.POINTER(SpecStats), U32P]
    L.or_generate_spec_ex.restype = ctypes.c_uint32
    L.or_generate_greedy.argtypes = [vp, U32P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, U32P]
    L.or_generate_greedy.restype = ctypes.c_uint32
    SP = ctypes.POINTER(Sampler)
    L.or_sampler_init.argtypes = [SP, f32, f32, ctypes.c_uint32, f32, u64]
    L.or_sampler_sample.argtypes = [SP, F32P, ctypes.c_uint32, U32P, ctypes.c_size_t]
    L.or_sampler_sample.restype = ctypes.c_uint32
    L.or_generate_sample.argtypes = [vp, U32P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, SP, U32P]
    L.or_generate_sample.restype = ctypes.c_uint32
    _lib = L
    return L


def sampler(temp, top_p, top_k, repeat_penalty, seed):
    s = Sampler()
    lib().or_sampler_init(ctypes.byref(s), temp, top_p, top_k, repeat_penalty, seed)
    return s


def sample(s, logits, tokens):
    """one sampler_sample call; `logits` (float32) receives the repeat penalty in place"""
    t = np.ascontiguousarray(tokens, np.uint32)
    return lib().or_sampler_sample(ctypes.byref(s), fptr(logits), len(logits), uptr(t) if len(t) else None, len(t))


def gemv(t, W, ne0, ne1, x, n, threads=8):
    """oracle batched GEMV: x [n][ne0] -> out [n][ne1]"""
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros((n, ne1), np.float32)
    lib().or_gemv_batch(t, W.ctypes.data_as(ctypes.c_void_p), ne0, ne1, fptr(x), ne0, n, fptr(out), ne1, threads)
    return out


def dequant_rows(t, W, ne0, ne1):
    L = lib()
    rb = L.or_row_bytes(t, ne0)
    out = np.zeros((ne1, ne0), np.float32)
    for r in range(ne1):
        L.or_dequant_row(t, ctypes.c_void_p(W.ctypes.data + r * rb), ne0, fptr(out[r]))
    return out


class Model:
    def __init__(self, path, n_ctx, k_max=2, threads=4):
        self.L = lib()
        self.h = self.L.or_model_open(path.encode(), n_ctx, k_max)
        if not self.h:
            raise OSError(f"oracle could not open {path}")
        self.L.or_model_set_threads(self.h, threads)
        self.V = self.L.or_model_vocab(self.h)
        self.E = self.L.or_model_n_embd(self.h)

    def close(self):
        if self.h:
            self.L.or_model_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def arr(self, getter, n):
        return np.ctypeslib.as_array(getter(self.h), shape=(n,)).copy()

    def forward(self, tok, pos):
        self.L.or_model_forward(self.h, tok, pos)
        return self.arr(self.L.or_model_logits, self.V)

    def forward_batch(self, toks, pos, ckpt):
        t = np.ascontiguousarray(toks, np.uint32)
        self.L.or_model_forward_batch(self.h, uptr(t), pos, len(t), ckpt)
        return self.arr(self.L.or_model_logits_b, len(t) * self.V).reshape(len(t), self.V)

    def generate_sample(self, prompt, n_predict, s, eos=0xFFFFFFFF):
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_predict, np.uint32)
        n = self.L.or_generate_sample(self.h, uptr(p), len(p), n_predict, eos, ctypes.byref(s), uptr(out))
        return out[:n]

    def h_save(self, B):
        return self.arr(self.L.or_model_h_save, B * self.E).reshape(B, self.E)

    def generate_spec(self, prompt, n_predict, k, eos=0xFFFFFFFF, force_accept=False):
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_predict + 16, np.uint32)
        js = np.zeros(n_predict + 16, np.uint32)
        st = SpecStats()
        n = self.L.or_generate_spec_ex(self.h, uptr(p), len(p), n_predict, k, eos, int(force_accept), uptr(out),
                                       ctypes.byref(st), uptr(js))
        return out[:n], js[:st.n_cycles], st

    def generate_greedy(self, prompt, n_predict, eos=0xFFFFFFFF):
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(n_predict, np.uint32)
        n = self.L.or_generate_greedy(self.h, uptr(p), len(p), n_predict, eos, uptr(out))
        return out[:n]
