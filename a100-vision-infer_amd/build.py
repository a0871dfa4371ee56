"""Build the fp8lin HIP library for gfx950 in-tree.

    python a100-vision-infer_amd/build.py          # -> a100-vision-infer_amd/lib/libfp8lin.so
    python a100-vision-infer_amd/build.py --aten   # also lib/avi_aten.so (LibTorch shim)

Each source is compiled with hipcc in parallel, then linked into one shared
library exporting the C ABI of include/fp8lin.h.  Packed FP32 instructions are
disabled for the device code (-target-feature -packed-fp32-ops); hipcc's host
pass warns that it does not know that feature, which is expected.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libfp8lin.so")
SOURCES = ["api.cpp", "gemv.hip", "small_m.hip", "gemm.hip", "skinny.hip", "elementwise.hip", "epilogue.hip",
           "chain.hip"]
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the fp8lin library needs ROCm's hipcc")
    return path


def _filter(text):
    # Drop the expected host-pass warning about the device-only feature flag.
    lines = [l for l in text.splitlines() if "packed-fp32-ops" not in l]
    return "\n".join(lines)


def _compile(src, verbose):
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc()] + COMMON + ["-x", "hip", "-c", os.path.join(CSRC, src), "-o", out]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    msg = _filter(r.stdout + r.stderr)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{msg}")
    if msg.strip() and verbose:
        print(msg, flush=True)
    return out


def build(verbose=False, jobs=None):
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + _filter(r.stdout + r.stderr))
    os.replace(tmp, LIB)
    return LIB


ATEN_SRC = os.path.join(HERE, "aten", "avi_ops.cpp")
ATEN_LIB = os.path.join(LIBDIR, "avi_aten.so")


def build_aten(verbose=False):
    """The reference's avi:: operators on ROCm LibTorch over the C ABI
    (aten/avi_ops.cpp), as a Python extension module.  Its fp8lin_* symbols
    resolve against libfp8lin.so, which fp8lin.aten loads first (global)."""
    import ctypes

    import torch
    from torch.utils import cpp_extension

    if not os.path.exists(LIB):
        raise RuntimeError("build the fp8lin library first")
    ctypes.CDLL(LIB, mode=ctypes.RTLD_GLOBAL)
    bdir = os.path.join(OBJ, "aten")
    shutil.rmtree(bdir, ignore_errors=True)
    os.makedirs(bdir)
    tlib = os.path.join(os.path.dirname(torch.__file__), "lib")
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cpp_extension.load(
        name="avi_aten", sources=[ATEN_SRC], build_directory=bdir, with_cuda=False, verbose=verbose,
        extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-I{rocm}/include"],
        extra_ldflags=[f"-L{rocm}/lib", "-lamdhip64", f"-L{tlib}", "-lc10_hip"])
    tmp = ATEN_LIB + ".tmp"
    shutil.copyfile(os.path.join(bdir, "avi_aten.so"), tmp)
    os.replace(tmp, ATEN_LIB)
    return ATEN_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    if "--aten" in sys.argv:
        print(build_aten(verbose="-v" in sys.argv))
