"""Source compatibility of the drop-in boundary: the reference's own driver
(src/main.c with its tokenizer and sampler, unmodified) compiles against
include/ and links against libqwen.so, whose model_* / gemv_* functions then
run on the GPU.  CPU-only (compile and link); skipped where the reference
checkout is absent."""
import os
import shutil
import subprocess

import pytest

from qwen_pkg import PKG_DIR

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"


@pytest.mark.skipif(not os.path.exists(os.path.join(REF, "src", "main.c")) or not shutil.which("gcc"),
                    reason="reference checkout or gcc absent")
def test_reference_driver_links_against_libqwen(tmp_path):
    lib = os.path.join(PKG_DIR, "lib")
    objs = []
    for src in ("main.c", "tokenizer.c", "sampler.c"):
        o = str(tmp_path / (src + ".o"))
        subprocess.run(["gcc", "-O2", "-std=c11", f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(REF, 'include')}",
                        "-c", os.path.join(REF, "src", src), "-o", o], check=True, capture_output=True)
        objs.append(o)
    exe = str(tmp_path / "qwen_gpu")
    subprocess.run(["gcc", *objs, f"-L{lib}", "-lqwen", f"-Wl,-rpath,{lib}", "-lm", "-lpthread", "-o", exe],
                   check=True, capture_output=True)
    undefined = subprocess.run(["nm", "-u", exe], check=True, capture_output=True, text=True).stdout
    for sym in ("model_init", "model_forward_batch", "mtp_forward", "model_rollback_to", "model_sample_greedy"):
        assert sym in undefined, sym          # resolved from libqwen.so at run time
