"""The C-ABI libraries load on a machine without a GPU and export every
function and variable that include/*.h declares (no compute calls)."""
import ctypes
import os
import re
import subprocess

import pytest

from qwen_pkg import PKG_DIR as PKG

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
LIBS = [os.path.join(PKG, "lib", n) for n in ("libqgpu.so", "libqwen.so")]

DECL = re.compile(r"^(?!\s*(?:typedef|#|return|/\*|\*))\s*(?:extern\s+)?(?:const\s+)?"
                  r"(?:unsigned\s+|signed\s+|struct\s+)?[A-Za-z_][A-Za-z_0-9]*\s*\**\s+\**\s*"
                  r"([A-Za-z_][A-Za-z_0-9]*)\s*\(", re.M)
EXTERN_VAR = re.compile(r"^\s*extern\s+(?!\"C\")[A-Za-z_0-9 ]+?\s+([A-Za-z_][A-Za-z_0-9]*(?:\s*,\s*[A-Za-z_][A-Za-z_0-9]*)*)\s*;",
                        re.M)


def declared():
    names = {}
    for fn in sorted(os.listdir(INC)):
        if not fn.endswith(".h"):
            continue
        src = open(os.path.join(INC, fn)).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        for m in DECL.finditer(src):
            names[m.group(1)] = fn
        for m in EXTERN_VAR.finditer(src):
            for v in m.group(1).split(","):
                names[v.strip()] = fn
    return names


def exported():
    out = set()
    for so in LIBS:
        txt = subprocess.check_output(["nm", "-D", "--defined-only", so], text=True)
        out |= {ln.split()[-1] for ln in txt.splitlines() if ln.strip()}
    return out


def test_libraries_load_without_gpu():
    for so in LIBS:
        assert os.path.exists(so), f"{so} not built (run __graft_entry__.build())"
        ctypes.CDLL(so)


def test_every_declared_symbol_is_exported():
    names = declared()
    assert len(names) > 80 and "qgpu_gemv_batch" in names and "model_forward_batch" in names \
        and "qwen_prof_calls" in names
    missing = sorted(f"{n} ({h})" for n, h in names.items() if n not in exported())
    assert not missing, missing


@pytest.mark.parametrize("name", ["qgpu_strerror"])
def test_error_strings_without_gpu(name):
    L = ctypes.CDLL(LIBS[0])
    f = getattr(L, name)
    f.restype = ctypes.c_char_p
    f.argtypes = [ctypes.c_int]
    assert f(0) and f(-1) and f(-12345)


def test_gguf_open_rejects_truncated_tensor_data(tmp_path):
    """A GGUF whose last tensor runs past the end of the file is refused by gguf_open (not read
    past the mapping later)."""
    from qwen_pkg import host_lib
    host = host_lib()
    path = str(tmp_path / "t.gguf")
    host.write_tiny_gguf(path, 1, 0)
    L = host.L

    class Ctx(ctypes.Structure):
        _fields_ = [("pad", ctypes.c_uint8 * 65536)]
    L.gguf_open.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
    L.gguf_close.argtypes = [ctypes.c_void_p]
    ctx = Ctx()
    assert L.gguf_open(ctypes.byref(ctx), path.encode()) == 0
    L.gguf_close(ctypes.byref(ctx))
    data = open(path, "rb").read()
    bad = str(tmp_path / "cut.gguf")
    open(bad, "wb").write(data[:-1000])
    assert L.gguf_open(ctypes.byref(ctx), bad.encode()) == -1


def test_attn_cache_fits_at_the_offset_boundary():
    """The attention kernels address a KV head's rows at 32-bit buffer offsets: a cache of
    n_ctx x n_kv x 1 KiB (head_dim 256, fp32) must stay within 2^31 - 1 bytes.  The check is
    arithmetic only, so it runs here without a GPU, at the first rejected sizes."""
    L = ctypes.CDLL(LIBS[0])
    f = L.qgpu_attn_cache_fits
    f.argtypes = [ctypes.c_int, ctypes.c_int]
    for ctx, kv, ok in [(524287, 4, 1), (524288, 4, 0), (2097151, 1, 1), (2097152, 1, 0), (262143, 8, 1),
                        (262144, 8, 0), (1, 1, 1), (0, 4, 0), (8, 0, 0), (-1, 4, 0)]:
        assert f(ctx, kv) == ok, (ctx, kv)


def run_child(code, tmp_path):
    """runs a Python snippet in a fresh process (the kernels API keeps its status per process);
    returns its stdout, stderr"""
    import sys
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120,
                       cwd=os.path.join(ROOT, "tests"))
    assert p.returncode == 0, p.stdout + p.stderr
    return p.stdout, p.stderr


def test_kernels_api_rejects_write_zeros(tmp_path):
    """kernels.h: a failing call writes zeros to its outputs.  A batch above 8 and rows past the
    matrix are refused before any device work and zero the in-range part of out; the row ops
    (here without a device, so their staging fails) zero out too.  kernels_status() reports it."""
    code = r'''
import ctypes, numpy as np
from qwen_pkg import PKG_DIR
L = ctypes.CDLL(PKG_DIR + "/lib/libqwen.so")
class TI(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("n_dims", ctypes.c_uint32), ("ne", ctypes.c_uint64 * 4),
                ("type", ctypes.c_int), ("offset", ctypes.c_uint64), ("data", ctypes.c_void_p)]
ne0, ne1 = 256, 16
raw = np.zeros(ne1 * ne0 * 4, np.uint8)
W = TI(b"w", 2, (ctypes.c_uint64 * 4)(ne0, ne1, 1, 1), 0, 0, raw.ctypes.data)
L.gemv_rows_batch.argtypes = [ctypes.POINTER(TI), ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p,
                              ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64]
x = np.ones((9, ne0), np.float32)
out = np.full((9, ne1), 7.0, np.float32)
L.gemv_rows_batch(ctypes.byref(W), x.ctypes.data, ne0, 9, out.ctypes.data, ne1, 2, 10)
assert L.kernels_status() != 0
assert (out[:8, 2:10] == 0).all() and (out[:8, :2] == 7).all() and (out[:8, 10:] == 7).all() and (out[8] == 7).all()
out[:] = 7.0
L.gemv_rows_batch(ctypes.byref(W), x.ctypes.data, ne0, 3, out.ctypes.data, ne1, 12, 20)   # rows 16..19 past the matrix
assert (out[:3, 12:16] == 0).all() and (out[:3, :12] == 7).all() and (out[3:] == 7).all()
L.rmsnorm.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_float]
o = np.full(64, 5.0, np.float32)
L.rmsnorm(o.ctypes.data, x.ctypes.data, x.ctypes.data, 64, 1e-6)
assert (o == 0).all()
L.silu_inplace.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
v = np.full(32, 3.0, np.float32)
L.silu_inplace(v.ctypes.data, 32)
assert (v == 0).all()
print("ok")
'''
    out, _ = run_child(code, tmp_path)
    assert out.strip().endswith("ok")


def test_model_init_rejects_kv_cache_beyond_attention_offsets(tmp_path):
    """An n_ctx whose KV cache the attention kernels cannot address (n_ctx x n_kv x 1 KiB above
    2^31 - 1 bytes) is refused by model_init with a message, before any device work."""
    from qwen_pkg import host_lib
    path = str(tmp_path / "t.gguf")
    host = host_lib()
    host.write_tiny_gguf(path, 1, 0)
    n_kv = int(host.spec_tiny(1, 0).n_kv_head)
    n_ctx = (2 ** 31) // (n_kv * 1024)               # the first size past the limit
    code = f'''
import ctypes
from qwen_pkg import PKG_DIR
L = ctypes.CDLL(PKG_DIR + "/lib/libqwen.so")
L.model_init.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_uint32]
m = ctypes.create_string_buffer(1 << 16)
print("rc", L.model_init(m, {path!r}.encode(), {n_ctx}))
'''
    out, err = run_child(code, tmp_path)
    assert "rc -1" in out and "KV cache" in err, (out, err)
