"""Build libgfl_moe.so (gfx950 HIP kernels + C-ABI host layer) in place with hipcc.

    python glm-flash-lite_amd/build.py          # compile everything, link glm-flash-lite_amd/libgfl_moe.so

Every HIP translation unit is compiled with -ffp-contract=off (the rounding points of the expert arithmetic are
explicit) and with packed-FP32 instruction selection disabled.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgfl_moe.so")
ARCH = os.environ.get("GFL_ARCH", "gfx950")

SOURCES = ["k_moe.hip", "k_split.hip", "k_prefill.hip", "gfl_api.cpp"]

CFLAGS = ["--offload-arch=" + ARCH, "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          # MFMA results straight into VGPRs: the transposing MFMA of the GEMV feeds VALU FMAs, and the AGPR form
          # costs four v_accvgpr_read per tile
          "-mllvm", "-amdgpu-mfma-vgpr-form",
          "-Wno-unused-result", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def _compile(src):
    out = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    cmd = [hipcc()] + CFLAGS + lang + ["-c", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("compile failed: %s\n%s\n%s" % (" ".join(cmd), r.stdout, r.stderr))
    return out


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed: %s\n%s" % (r.stdout, r.stderr))
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
