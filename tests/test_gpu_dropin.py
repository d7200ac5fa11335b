"""The reference's own test programs, run on the GPU through libqwen.so: each
was compiled unchanged from the reference's src/ against include/ (oracle's
Makefile, into oracle/_ref/dropin/), so what it checks is this library behind
the reference's API.  The programs a small model can drive run here; the ones
that need the 27B file's vocabulary size or tensor names (test_forward,
test_forward_batch, test_quant, test_kernels, debug_rollback, debug_spec2) run
on a full-size file in tests/test_gpu_dropin_27b.py; every program builds in
tests/test_dropin_build.py.
  * test_ops: the reference's known-answer and dimension checks of rmsnorm,
    l2norm, silu, sigmoid, softplus and softmax (kernels.h on host buffers);
  * test_batch: gemv_batch(n) bit-identical to n single-token gemv calls, on
    the mixed-format tiny model (IQ4_XS, Q5_K, Q4_K, Q6_K, F32 tensors);
  * test_model: model_init and the state report on both tiny models;
  * qwen (main.c, the reference CLI): prompt text in, generated text out, on a
    tiny model whose GGUF carries a byte-level BPE vocabulary, against the same
    CLI compiled on the reference engine (oracle/_ref/qwen_cpu): greedy
    speculative decoding (--spec 1/2, --temp 0), greedy decoding through the
    reference sampler (--temp 0, repetition penalty 1.1) with --profile."""
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


# ---------------------------------------------------------------- the reference CLI
PROMPT = "the other tall tree, in the north"


@pytest.fixture(scope="module")
def tok_files():
    """tiny models with a vocabulary: the draft-accepting one (synth variant 2) and the
    mixed-format one (variant 1)"""
    td = tempfile.mkdtemp()
    out = {}
    for name, seed, variant in (("accept", 1234, 2), ("mixed", 1, 1)):
        path = os.path.join(td, f"{name}_tok.gguf")
        host_lib().write_tiny_gguf(path, seed, variant, tokenizer=1)
        out[name] = path
    yield out
    for p in out.values():
        os.remove(p)


def cli(exe, gguf, args, env=None):
    if not os.path.exists(exe):
        pytest.skip(f"{exe} not built (reference checkout absent at build time)")
    cmd = [exe, "-m", gguf, "-p", PROMPT, "-c", "256", "-t", "4", *args]
    print(f"\n[cli] {os.path.relpath(exe, ROOT)} {' '.join(args)} on {os.path.basename(gguf)}", flush=True)
    p = subprocess.run(cmd, capture_output=True, timeout=120, env=env)
    # single-byte tokens print bytes that are not UTF-8 on their own: keep them as they are
    out, err = (b.decode("utf-8", "surrogateescape") for b in (p.stdout, p.stderr))
    assert p.returncode == 0, out[-2000:] + err[-2000:]
    return out, err


def generation(stdout):
    """the generated text: what main.c prints after "Generation: " up to its closing rule"""
    head, _, rest = stdout.partition("Generation: ")
    assert rest, stdout[-2000:]
    return rest.split("\n================================================", 1)[0]


@pytest.mark.parametrize("name,spec", [("accept", 2), ("accept", 1), ("mixed", 2)])
def test_reference_cli_speculative_on_gpu(gpu, tok_files, name, spec):
    """greedy speculative decoding from the command line: the same text and the same
    draft statistics (cycles, accepted drafts, acceptance depths) as the reference"""
    args = ["-n", "48", "--temp", "0", "--spec", str(spec)]
    ref_out, ref_err = cli(os.path.join(ROOT, "oracle", "_ref", "qwen_cpu"), tok_files[name], args)
    out, err = cli(os.path.join(BIN, "qwen"), tok_files[name], args)
    prompt_line = [ln for ln in ref_out.splitlines() if ln.startswith("Prompt (")]
    assert prompt_line and prompt_line == [ln for ln in out.splitlines() if ln.startswith("Prompt (")]
    assert generation(out) == generation(ref_out)
    assert "Generation         : 48 tokens" in out
    stats = [ln for ln in ref_err.splitlines() if ln.startswith("[spec]")]
    assert len(stats) == 1 and stats == [ln for ln in err.splitlines() if ln.startswith("[spec]")], err[-2000:]
    if name == "accept":
        accepted = int(stats[0].split()[3].split("/")[0])
        assert accepted > 0, stats          # the rollback-free branch ran, not only j = 0


def test_reference_cli_sampler_greedy_with_profile_on_gpu(gpu, tok_files):
    """--temp 0 without drafts: model_forward one token at a time, the reference
    sampler (repetition penalty) on this library's logits, and the --profile line
    filled by the section counters (QWEN_PROFILE in the environment)"""
    args = ["-n", "32", "--temp", "0", "--profile"]
    ref_out, _ = cli(os.path.join(ROOT, "oracle", "_ref", "qwen_cpu"), tok_files["mixed"], args)
    env = dict(os.environ, QWEN_PROFILE="1")
    out, _ = cli(os.path.join(BIN, "qwen"), tok_files["mixed"], args, env=env)
    assert generation(out) == generation(ref_out)
    prof = [ln for ln in out.splitlines() if ln.startswith("Profile (")]
    ref_prof = [ln for ln in ref_out.splitlines() if ln.startswith("Profile (")]
    assert len(prof) == 1 and len(ref_prof) == 1, out[-2000:]
    # the same number of model_forward calls, every section timed
    assert prof[0].split(")")[0] == ref_prof[0].split(")")[0]
    for sec in ("embed", "GDN", "attn", "head"):
        assert f"{sec} " in prof[0]
