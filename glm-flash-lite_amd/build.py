"""Build libgfl_moe.so (gfx950 HIP kernels + C-ABI host layer) in place with hipcc.

    python glm-flash-lite_amd/build.py          # compile everything, link glm-flash-lite_amd/libgfl_moe.so, then build
                                                # the torch extension _torch_ext/gfl_torch_ext.so against it

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
    # the soname lets the torch extension (linked with -lgfl_moe) bind to this library once it is loaded
    cmd = [hipcc(), "--offload-arch=" + ARCH, "-shared", "-fPIC", "-Wl,-soname,libgfl_moe.so", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed: %s\n%s" % (r.stdout, r.stderr))
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


EXT_NAME = "gfl_torch_ext"
EXT_DIR = os.path.join(HERE, "_torch_ext")


def build_torch_ext(verbose=False):
    """The PyTorch-ROCm extension (csrc/torch_ext.cpp: the reference's tier_* / ft_split / ft_combine names), built
    in place with torch.utils.cpp_extension into _torch_ext/gfl_torch_ext.so, linked against libgfl_moe.so."""
    import ctypes
    import torch.utils.cpp_extension as ce
    os.makedirs(EXT_DIR, exist_ok=True)
    ctypes.CDLL(LIB)   # load() imports the module it built: its libgfl_moe.so dependency resolves to this by soname
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    torch_lib = os.path.join(os.path.dirname(ce.__file__), "..", "lib")
    # a host-only C++ translation unit: HIP runtime and c10_hip headers/libraries named directly (no device code, no
    # source translation step)
    ce.load(name=EXT_NAME, sources=[os.path.join(CSRC, "torch_ext.cpp")], build_directory=EXT_DIR,
            extra_include_paths=[os.path.join(ROOT, "include"), os.path.join(rocm, "include")],
            extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1"],
            extra_ldflags=["-L" + HERE, "-lgfl_moe", "-L" + os.path.abspath(torch_lib), "-lc10_hip",
                           "-L" + os.path.join(rocm, "lib"), "-lamdhip64"],
            with_cuda=False, verbose=verbose)
    so = os.path.join(EXT_DIR, EXT_NAME + ".so")
    if verbose:
        print("built", so)
    return so


if __name__ == "__main__":
    build(verbose=True)
    if "--no-torch-ext" not in sys.argv:
        build_torch_ext(verbose=False)
        print("built", os.path.join(EXT_DIR, EXT_NAME + ".so"))
    sys.exit(0)
