"""The reference's own test programs, run on the GPU through libqwen.so: each
was compiled unchanged from the reference's src/ against include/ (oracle's
Makefile, into oracle/_ref/dropin/), so what it checks is this library behind
the reference's API.  The programs a small model can drive run here; the ones
that need the full vocabulary or tensor names of the 27B file (test_forward,
test_forward_batch, test_quant, test_kernels) and the tokenizer tools only
build (tests/test_dropin_build.py).
  * test_ops: the reference's known-answer and dimension checks of rmsnorm,
    l2norm, silu, sigmoid, softplus and softmax (kernels.h on host buffers);
  * test_batch: gemv_batch(n) bit-identical to n single-token gemv calls, on
    the mixed-format tiny model (IQ4_XS, Q5_K, Q4_K, Q6_K, F32 tensors);
  * test_model: model_init and the state report on both tiny models."""
import hashlib
import os
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


def run(prog, *args, timeout=120):
    exe = os.path.join(BIN, prog)
    if not os.path.exists(exe):
        pytest.skip(f"{exe} not built (reference checkout absent at build time)")
    print(f"\n[dropin] {prog} {' '.join(os.path.basename(a) for a in args)}", flush=True)
    p = subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout)
    return p.returncode, p.stdout + p.stderr


@pytest.fixture(scope="module")
def tiny_files():
    td = tempfile.mkdtemp()
    out = {}
    for name in ("tiny", "tiny_mixed"):
        z = np.load(os.path.join(O.GOLDEN, f"model_{name}.npz"), allow_pickle=False)
        path = os.path.join(td, f"{name}.gguf")
        host_lib().write_tiny_gguf(path, int(z["seed"]), int(z["mixed"]))
        assert hashlib.sha256(open(path, "rb").read()).hexdigest() == str(z["gguf_sha256"])
        out[name] = path
    yield out
    for p in out.values():
        os.remove(p)


def test_reference_test_ops_on_gpu(gpu):
    rc, out = run("test_ops")
    assert rc == 0 and "ALL D1 TESTS PASSED" in out, out[-2000:]


def test_reference_test_batch_on_gpu(gpu, tiny_files):
    rc, out = run("test_batch", tiny_files["tiny_mixed"])
    assert rc == 0 and "OK: batch == single-token everywhere" in out, out[-3000:]
    identical = [ln for ln in out.splitlines() if "identical" in ln]
    # 5 tensors of the tiny model (the 27B-only MTP name is absent) x n = 1..8
    assert len(identical) == 5 * 8, out[-3000:]


@pytest.mark.parametrize("name", ["tiny", "tiny_mixed"])
def test_reference_test_model_on_gpu(gpu, tiny_files, name):
    rc, out = run("test_model", tiny_files[name], "256")
    assert rc == 0 and out.rstrip().endswith("OK"), out[-2000:]
