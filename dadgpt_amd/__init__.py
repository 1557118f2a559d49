"""MI355X-native (gfx950) fused causal attention for DadGPT.

The work happens in ``lib/libdadgpt_attn.so`` (hand-written HIP kernels behind the C ABI of
``include/dadgpt/gpu_attention.h``) and ``lib/libdadgpt_gen.so`` (hipBLASLt GEMMs, the
materialized attention path and batched GPT-2 generation); ``attention`` and ``gpt2`` are their
Python mirrors over ctypes.

Import this package before ``torch``. Both use the HIP runtime, and both use a hipBLASLt:
PyTorch's ROCm wheel bundles its own (older) hipBLASLt and rocRoller, under the same sonames as
the ROCm installation's. At import this package loads, in order:

1. PyTorch's ``libamdhip64`` (when PyTorch is installed), so the process has one HIP runtime,
   the one PyTorch needs;
2. the two libraries, which bind to that runtime;
3. the ROCm installation's hipBLASLt, privately (``dadgpt_blas_open``), while its rocRoller
   dependency can still resolve to the ROCm installation's own.

``import torch`` then loads PyTorch's own hipBLASLt and rocRoller beside it (PyTorch asks for
them under other file names) and binds to those. If torch was imported first, step 3 cannot
bind the right rocRoller, and hipBLASLt handle creation fails with a message that says so.
"""
import ctypes
import importlib.util
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_DIR = os.path.join(HERE, "lib")

# Why step 3 did not happen ("" if it did, or if the libraries are not built yet).
load_error = ""


def _load_native_stack() -> None:
    global load_error
    if "torch" not in sys.modules:
        spec = importlib.util.find_spec("torch")
        if spec is not None and spec.submodule_search_locations:
            hip = os.path.join(list(spec.submodule_search_locations)[0], "lib", "libamdhip64.so")
            if os.path.exists(hip):
                ctypes.CDLL(hip, mode=ctypes.RTLD_GLOBAL)
    gen = os.path.join(_LIB_DIR, "libdadgpt_gen.so")
    if not os.path.exists(gen):
        return  # not built: every call raises LibraryNotBuilt later
    lib = ctypes.CDLL(gen)
    lib.dadgpt_blas_open.restype = ctypes.c_int
    lib.dadgpt_gen_last_error.restype = ctypes.c_char_p
    if lib.dadgpt_blas_open() != 0:
        load_error = lib.dadgpt_gen_last_error().decode()


_load_native_stack()

from . import attention  # noqa: E402,F401

__all__ = ["attention", "load_error"]
