"""The reference's own full-size programs, run on the GPU through libqwen.so
(compiled unchanged from the reference's src/ against include/, oracle's
Makefile, into oracle/_ref/dropin/), on a 27B GGUF file written on the box:
the seeded random-init 27B hybrid with the real checkpoint's format mix
(token_embd Q4_K, attn_qkv Q5_K, output Q6_K, nextn.eh_proj Q8_0, the rest
IQ4_XS; reference test_kernels.c:120-126) and the generator's byte-level BPE
vocabulary (248,320 ids), so the programs that tokenize text run too.
  * test_forward (test_forward.c:16-50): one decode step of id 151644; the
    logit range and the greedy token printed are the reference engine's for
    the same file (tests/golden/dropin_27b.npz, from oracle/_ref/test_forward_cpu);
  * test_forward_batch (test_forward_batch.c:17-77), B = 3, 4, 8: batched
    logits against B sequential steps, its own pass condition (exit 0, no argmax
    difference) and max_rel within 1e-3;
  * debug_rollback (debug_rollback.c:10-57): batch, model_rollback_to(1),
    batch against the sequential model, at 27B state size;
  * debug_spec2 (debug_spec2.c:41-94): four two-draft speculative cycles with
    rollback and MTP re-anchor against a sequential model: no divergence, and
    every cycle (position, candidates, j) as the reference engine prints it;
  * test_kernels (test_kernels.c:102-127): every format of the file at its
    real shape against the reference's scalar dot product (max_rel < 1e-4);
  * test_quant (test_quant.c:62-84): ten rows dequantised from the file (every
    format) and their statistics, printed exactly as the reference engine
    prints them for the same file.  (Both exit 1 on this file: the program's
    plausibility rule |mean| < 0.5 does not hold for the generator's ssm_a.)"""
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

import oracle_lib as O
from gpu_util import gpu  # noqa: F401
from qwen_pkg import host_lib

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "dropin")
FIX = os.path.join(O.GOLDEN, "dropin_27b.npz")


def file_digest(path, span=32 << 20):
    """sha256 of the file's first and last 32 MiB and its size (header, metadata and vocabulary
    lie at the start), as tests/golden/make_golden.py computes it"""
    import hashlib
    h = hashlib.sha256()
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        h.update(f.read(span))
        f.seek(max(0, size - span))
        h.update(f.read(span))
    h.update(str(size).encode())
    return h.hexdigest()


def run(prog, *args, timeout=240):
    exe = os.path.join(BIN, prog)
    if not os.path.exists(exe):
        pytest.skip(f"{exe} not built (reference checkout absent at build time)")
    print(f"\n[dropin-27b] {prog} {' '.join(os.path.basename(str(a)) for a in args)}", flush=True)
    p = subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=timeout)
    return p.returncode, p.stdout + p.stderr


@pytest.fixture(scope="module")
def m27_file():
    if not os.path.exists(FIX):
        pytest.skip("dropin_27b.npz fixture absent")
    z = np.load(FIX, allow_pickle=False)
    host = host_lib()
    spec = host.spec_27b_mix(int(z["seed"]))
    spec.tokenizer = 1
    need = sum(t.nbytes for t in host.tensors(spec)) + (256 << 20)
    import shutil
    dirs = [d for d in ("/dev/shm", tempfile.gettempdir()) if os.path.isdir(d) and shutil.disk_usage(d).free > need]
    if not dirs:
        pytest.skip("no room for the 27B file")
    td = tempfile.mkdtemp(dir=dirs[0])
    path = os.path.join(td, "m27_mix_tok.gguf")
    print(f"\n[dropin-27b] writing {path} ({need / 1e9:.1f} GB)", flush=True)
    host.write_gguf(spec, path)
    assert file_digest(path) == str(z["digest"])
    yield path, z
    os.remove(path)
    os.rmdir(td)


def stats(out):
    m = re.search(r"Logits stats: min = (\S+), max = (\S+), greedy token = (\d+) \(logit = (\S+)\)", out)
    assert m, out[-2000:]
    return float(m.group(1)), float(m.group(2)), int(m.group(3)), float(m.group(4))


def test_reference_test_forward_27b(gpu, m27_file):
    path, z = m27_file
    rc, out = run("test_forward", path)
    assert rc == 0 and "completed successfully" in out, out[-2000:]
    got, ref = stats(out), stats(str(z["test_forward"]))
    print(f"  gpu {got}  reference engine {ref}", flush=True)
    assert got[2] == ref[2]                                  # greedy token
    scale = max(abs(ref[0]), abs(ref[1]))
    for a, b in ((got[0], ref[0]), (got[1], ref[1]), (got[3], ref[3])):
        assert abs(a - b) <= 1e-3 * scale, (got, ref)


@pytest.mark.parametrize("B", [3, 4, 8])
def test_reference_test_forward_batch_27b(gpu, m27_file, B):
    path, _ = m27_file
    rc, out = run("test_forward_batch", path, B)
    m = re.search(r"max_abs=(\S+) \(token \d+\)\s+max_rel=(\S+)\s+argmax_diff=(\d+)/(\d+)", out)
    assert rc == 0 and m, out[-3000:]
    print(f"  B={B}: max_abs {m.group(1)}, max_rel {m.group(2)}, argmax differences {m.group(3)}", flush=True)
    assert int(m.group(3)) == 0 and int(m.group(4)) == B
    assert float(m.group(2)) < 1e-3
    assert out.count(" OK ") == B


def test_reference_debug_rollback_27b(gpu, m27_file):
    path, _ = m27_file
    rc, out = run("debug_rollback", path)
    lines = [ln for ln in out.splitlines() if ln.startswith("batch2[")]
    assert rc == 0 and len(lines) == 2, out[-2000:]
    for ln in lines:
        print("  " + ln, flush=True)
        d = float(re.search(r"maxdiff=(\S+)", ln).group(1))
        assert ln.rstrip().endswith("OK") and d < 1e-2, ln


def cycles(out):
    return [ln.rstrip() for ln in out.splitlines() if ln.startswith("ref cand0") or ln.startswith("  cycle")]


def test_reference_debug_spec2_27b(gpu, m27_file):
    """two-draft speculative cycles with rollback and re-anchor at full size: the program's own
    check against a sequential model (no DIVERGENCE line) and the reference engine's cycles"""
    path, z = m27_file
    rc, out = run("debug_spec2", path)
    assert rc == 0 and "DIVERGENCE" not in out, out[-3000:]
    got, ref = cycles(out), cycles(str(z["debug_spec2"]))
    for ln in got:
        print("  " + ln, flush=True)
    assert len(got) == 8 and got == ref


def test_reference_test_kernels_27b(gpu, m27_file):
    """every format of the file at its real shape (IQ4_XS attn_q and ffn_down, Q5_K attn_qkv,
    Q4_K token_embd, Q6_K output, Q8_0 eh_proj, F32 conv1d) against the reference's scalar dot
    product; then its GEMV sweep over one decode step's weights with one thread count"""
    path, _ = m27_file
    rc, out = run("test_kernels", path, 1)
    rows = [ln for ln in out.splitlines() if "max_rel=" in ln]
    for ln in rows:
        print("  " + ln, flush=True)
    assert rc == 0 and len(rows) == 7 and all(ln.rstrip().endswith("OK") for ln in rows), out[-3000:]
    fmts = {ln.split()[1] for ln in rows}
    assert {"IQ4_XS", "Q5_K", "Q4_K", "Q6_K", "Q8_0", "F32"} <= fmts, fmts


def test_reference_test_quant_27b(gpu, m27_file):
    path, z = m27_file
    rc, out = run("test_quant", path)
    ref = str(z["test_quant"])
    rows = [ln for ln in out.splitlines() if " ligne " in ln]
    print("  " + "\n  ".join(rows), flush=True)
    assert len(rows) == 10 and "NON FINI" not in out, out[-3000:]
    assert out.splitlines() == ref.splitlines(), out[-3000:]
