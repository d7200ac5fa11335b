"""Source compatibility of the drop-in boundary: every program of the
reference's src/ (its driver main.c, the test_* programs and the debug_* /
bench_* tools), unmodified, compiles against include/ and links against
libqwen.so in place of gguf.c quant.c kernels.c threadpool.c model.c (the
reference's tokenizer.c and sampler.c are linked as they are).  The model_* /
gemv_* / dequant calls then resolve to this library.  CPU-only (compile and
link); skipped where the reference checkout is absent.  tests/test_gpu_dropin.py
runs the programs a small model can drive on the GPU."""
import os
import shutil
import subprocess

import pytest

from qwen_pkg import PKG_DIR

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
# every program of the reference's src/ that has a main() (main.c is the driver)
PROGRAMS = ["main", "test_tokenizer", "test_forward", "test_model", "test_kernels", "test_ops", "test_quant",
            "test_batch", "test_forward_batch", "debug_kernels", "debug_rollback", "debug_spec", "debug_spec2",
            "debug_tokenizer", "bench_cache"]
# the reference symbols each program must take from libqwen.so (a sample per program)
USES = {
    "main": ["model_init", "model_forward_batch", "mtp_forward", "model_rollback_to", "model_sample_greedy"],
    "test_ops": ["rmsnorm", "l2norm", "silu_inplace", "softplus_inplace", "softmax_inplace"],
    "test_batch": ["gemv", "gemv_batch", "gguf_find_tensor"],
    "test_kernels": ["gemv_rows", "dequant_row", "quant_row_ptr"],
    "test_forward_batch": ["model_forward", "model_forward_batch"],
    "test_quant": ["gguf_open", "dequant_row"],
    "debug_spec2": ["mtp_forward", "model_rollback_to"],
}

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(REF, "src", "main.c")) or not shutil.which("gcc"),
                                reason="reference checkout or gcc absent")


def compile_program(name, out_dir):
    lib = os.path.join(PKG_DIR, "lib")
    exe = os.path.join(out_dir, name)
    srcs = [os.path.join(REF, "src", f"{name}.c"), os.path.join(REF, "src", "tokenizer.c"),
            os.path.join(REF, "src", "sampler.c")]
    p = subprocess.run(["gcc", "-O2", "-std=c11", f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(REF, 'include')}",
                        *srcs, "-o", exe, f"-L{lib}", "-lqwen", f"-Wl,-rpath,{lib}", "-lm", "-lpthread"],
                       capture_output=True, text=True)
    assert p.returncode == 0, f"{name} does not build against include/ + libqwen.so:\n{p.stderr[-3000:]}"
    return exe


def test_every_reference_program_is_listed():
    """the list covers every source file of the reference's src/ that defines main()"""
    with_main = sorted(f[:-2] for f in os.listdir(os.path.join(REF, "src"))
                       if f.endswith(".c") and "int main(" in open(os.path.join(REF, "src", f), errors="replace").read())
    assert with_main == sorted(PROGRAMS)


@pytest.mark.parametrize("name", PROGRAMS)
def test_reference_program_builds_against_libqwen(tmp_path, name):
    exe = compile_program(name, str(tmp_path))
    undefined = subprocess.run(["nm", "-u", exe], check=True, capture_output=True, text=True).stdout
    for sym in USES.get(name, []):
        assert sym in undefined, sym          # resolved from libqwen.so at run time
    # no reference engine symbol is defined inside the program itself
    defined = subprocess.run(["nm", "--defined-only", exe], check=True, capture_output=True, text=True).stdout
    for sym in ("model_init", "gemv_batch", "gguf_open", "dequant_row"):
        assert f" T {sym}\n" not in defined, sym


def test_reference_tokenizer_test_runs_on_libqwen(tmp_path):
    """The reference's test_tokenizer, linked with libqwen.so (its gguf_open and the
    mapped file it leaves in gguf_context_t feed the reference tokenizer), prints the
    same encodings as the same program on the reference engine, for a GGUF that
    carries a byte-level BPE vocabulary; every prompt decodes back to itself."""
    from qwen_pkg import host_lib
    ref_exe = os.path.join(ROOT, "oracle", "_ref", "test_tokenizer_cpu")
    if not os.path.exists(ref_exe):
        pytest.skip("oracle/_ref/test_tokenizer_cpu not built")
    exe = compile_program("test_tokenizer", str(tmp_path))
    gguf = str(tmp_path / "tok.gguf")
    host_lib().write_tiny_gguf(gguf, 1234, 2, tokenizer=1)
    ours = subprocess.run([exe, gguf], capture_output=True, text=True, timeout=60)
    ref = subprocess.run([ref_exe, gguf], capture_output=True, text=True, timeout=60)
    assert ours.returncode == 0 and ref.returncode == 0, ours.stderr + ref.stderr
    assert ours.stdout == ref.stdout
    assert "vocab_size = 1024, n_merges = 12" in ours.stdout
    prompts = [ln.split('"', 1)[1].rsplit('"', 1)[0] for ln in ours.stdout.splitlines() if ln.startswith("Prompt [")]
    decoded = [ln.split('"', 1)[1].rsplit('"', 1)[0] for ln in ours.stdout.splitlines() if ln.startswith("Decoded:")]
    assert len(prompts) == 5 and decoded == prompts
