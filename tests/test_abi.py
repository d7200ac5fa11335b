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
