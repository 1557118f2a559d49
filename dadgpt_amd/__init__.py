"""MI355X-native (gfx950) fused causal attention for DadGPT.

The work happens in ``lib/libdadgpt_attn.so`` (hand-written HIP kernels behind the C ABI of
``include/dadgpt/gpu_attention.h``); ``attention`` is its Python mirror over ctypes.
"""
from . import attention  # noqa: F401

__all__ = ["attention"]
