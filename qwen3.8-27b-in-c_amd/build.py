"""Builds the package's native libraries in-tree:

  lib/libqgpu.so  <- csrc/*.hip, csrc/*.cpp   (hipcc --offload-arch=gfx950)
  lib/libqwen.so  <- host/*.c                 (gcc -std=c11, links libqgpu)

    python build.py [--jobs N]

Compiles every time it is called (objects in _build/, one hipcc per file in
parallel).  hipcc cross-compiles gfx950 code objects without a GPU present.
"""
import argparse
import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INC = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "lib")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", f"-I{INC}", f"-I{os.path.join(PKG, 'csrc')}",
             # packed-FP32 VALU ops stay off: scalar/float2 code only
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             # matrix-core results in VGPRs (no v_accvgpr_read per result)
             "-mllvm", "-amdgpu-mfma-vgpr-form",
             "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]
CC_FLAGS = ["-O2", "-std=c11", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter", f"-I{INC}"]


def run(cmd):
    p = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (p.stdout + p.stderr).splitlines()
                    if "is not a recognized feature for this target" not in line)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(jobs=8, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    hip_srcs = sorted(glob.glob(os.path.join(PKG, "csrc", "*.hip")) + glob.glob(os.path.join(PKG, "csrc", "*.cpp")))
    objs = []

    def compile_one(src):
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        out = run([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
        if verbose and out.strip():
            print(out)
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, hip_srcs))
    qgpu = os.path.join(LIB, "libqgpu.so")
    tmp = qgpu + ".tmp"
    run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, qgpu)

    host_srcs = sorted(glob.glob(os.path.join(PKG, "host", "*.c")))
    qwen = os.path.join(LIB, "libqwen.so")
    tmp = qwen + ".tmp"
    run(["gcc", *CC_FLAGS, "-shared", *host_srcs, "-o", tmp, f"-L{LIB}", "-lqgpu",
         "-Wl,-rpath,$ORIGIN", "-lm", "-lpthread"])
    os.replace(tmp, qwen)
    return qgpu, qwen


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        sys.exit(f"hipcc not found at {HIPCC}")
    for p in build(a.jobs, a.verbose):
        print("built", p)


if __name__ == "__main__":
    main()
