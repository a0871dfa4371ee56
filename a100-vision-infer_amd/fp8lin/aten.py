"""Loader for the compiled LibTorch shim (a100-vision-infer_amd/aten/avi_ops.cpp):
the reference's avi:: linear-path operators with their C++ signatures, over
the same C ABI.  The module's fp8lin_* symbols resolve against
libfp8lin.so, loaded here with global visibility first."""
import ctypes
import importlib.util
import os

from ._lib import LIB_PATH

ATEN_PATH = os.path.join(os.path.dirname(LIB_PATH), "avi_aten.so")
_mod = None


def load():
    global _mod
    if _mod is None:
        if not os.path.exists(ATEN_PATH):
            raise RuntimeError(f"{ATEN_PATH} is not built: run a100-vision-infer_amd/build.py --aten")
        import torch  # noqa: F401  (LibTorch must be loaded before the extension)
        ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL).fp8lin_init()  # the current device, outside any capture
        spec = importlib.util.spec_from_file_location("avi_aten", ATEN_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _mod = mod
    return _mod
