"""Python mirror of the attention wrappers, over the C ABI of ``libdadgpt_attn.so``.

Function names, argument order and meaning follow the reference's launch wrappers
(``cuda/gpu_ops.cuh:112-122``): raw device buffers in ``[BH, S, d_head]`` layout, ``lse`` and
``delta`` ``[BH, S]``, outputs overwritten; errors raise (``RuntimeError`` as the reference's
``CUDA_CHECK`` throws ``std::runtime_error``, ``cuda/gpu_ops.cuh:10-17``). Here the buffers
are torch tensors: torch provides device memory and the stream, the library does the work.

The product path has no fallback: if the HIP library is missing or fails to load, every
call raises ``LibraryNotBuilt``.
"""
from __future__ import annotations

import ctypes
import math
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libdadgpt_attn.so")

# Symbols declared in include/dadgpt/gpu_attention.h (C linkage) and
# include/dadgpt/gpu_ops_attention.hpp (C++ linkage, reference names).
C_SYMBOLS = (
    "dadgpt_last_error",
    "dadgpt_status_string",
    "dadgpt_version",
    "dadgpt_flash_attention_supported",
    "dadgpt_flash_attention_forward",
    "dadgpt_flash_attention_backward",
    "dadgpt_flash_attention_forward_async",
    "dadgpt_flash_attention_backward_async",
    "dadgpt_flash_attention_forward_bf16",
    "dadgpt_flash_attention_backward_bf16",
    "dadgpt_flash_attention_backward_bf16_phase",
    "dadgpt_flash_attention_forward_bf16_dropout",
    "dadgpt_flash_attention_backward_bf16_dropout",
    "dadgpt_flash_attention_forward_dropout",
    "dadgpt_flash_attention_backward_dropout",
    "dadgpt_flash_attention_forward_bf16_strided",
    "dadgpt_flash_attention_backward_bf16_strided",
    "dadgpt_flash_attention_forward_bf16_tokens",
    "dadgpt_flash_attention_backward_bf16_tokens",
    "dadgpt_decode_workspace_bytes",
    "dadgpt_decode_attention_bf16",
    "dadgpt_decode_attention_bf16_noalloc",
    "dadgpt_decode_attention_f32",
    "dadgpt_softmax",
    "dadgpt_softmax_backward",
    "dadgpt_causal_mask",
    "dadgpt_causal_mask_zero",
    "dadgpt_scale",
    "dadgpt_split_heads",
    "dadgpt_merge_heads",
    "dadgpt_attention_probs",
    "dadgpt_attention_probs_backward",
    "dadgpt_attention_dropout",
    "dadgpt_attention_probs_backward_dropout",
    "dadgpt_decode_probs",
    "dadgpt_use_fused_attention",
)
CXX_SYMBOLS = (
    "_Z29gpu_flash_attention_supportedi",
    "_Z27gpu_flash_attention_forwardPfS_PKfS1_S1_iiif",
    "_Z28gpu_flash_attention_backwardPfS_S_S_PKfS1_S1_S1_S1_S1_iiif",
    "_Z11gpu_softmaxPfPKfii",
    "_Z20gpu_softmax_backwardPfPKfS1_ii",
    "_Z15gpu_causal_maskPfii",
    "_Z20gpu_causal_mask_zeroPfii",
    "_Z9gpu_scalePfif",
    "_Z15gpu_split_headsPfPKfiiii",
    "_Z15gpu_merge_headsPfPKfiiii",
    "_Z19use_fused_attention13AttentionImpliib",
)

STATUS = {0: "ok", 1: "invalid argument", 2: "unsupported", 3: "hip error", 4: "workspace"}


class HeadStrides(ctypes.Structure):
    """dadgpt_head_strides: element strides of a [B, H, S, d_head] view (batch, head, row)."""
    _fields_ = [("batch", ctypes.c_int64), ("head", ctypes.c_int64), ("row", ctypes.c_int64)]


class LibraryNotBuilt(RuntimeError):
    pass


class AttentionError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message or STATUS.get(status, f"status {status}"))
        self.status = status


_lib = None


def lib():
    """The loaded HIP library. torch is imported first so the library binds to the same HIP
    runtime (libamdhip64.so.7) torch already loaded."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryNotBuilt(f"{LIB_PATH} is not built; run __graft_entry__.build() or "
                              f"`make -C dadgpt_amd/csrc`")
    try:
        L = ctypes.CDLL(LIB_PATH)
    except OSError as e:  # pragma: no cover - depends on the machine
        raise LibraryNotBuilt(f"cannot load {LIB_PATH}: {e}") from e
    vp, i, f, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    L.dadgpt_last_error.restype = ctypes.c_char_p
    L.dadgpt_last_error.argtypes = []
    L.dadgpt_status_string.restype = ctypes.c_char_p
    L.dadgpt_status_string.argtypes = [i]
    L.dadgpt_version.restype = ctypes.c_char_p
    L.dadgpt_version.argtypes = []
    L.dadgpt_flash_attention_supported.argtypes = [i]
    L.dadgpt_flash_attention_forward.argtypes = [vp] * 5 + [i, i, i, f]
    L.dadgpt_flash_attention_backward.argtypes = [vp] * 10 + [i, i, i, f]
    L.dadgpt_flash_attention_forward_async.argtypes = [vp] * 5 + [i, i, i, f, vp]
    L.dadgpt_flash_attention_backward_async.argtypes = [vp] * 10 + [i, i, i, f, vp]
    L.dadgpt_flash_attention_forward_bf16.argtypes = [vp] * 5 + [i, i, i, f, vp]
    L.dadgpt_flash_attention_backward_bf16.argtypes = [vp] * 10 + [i, i, i, f, vp]
    L.dadgpt_flash_attention_backward_bf16_phase.argtypes = [i] + [vp] * 10 + [i, i, i, f, vp]
    u64 = ctypes.c_uint64
    L.dadgpt_flash_attention_forward_bf16_dropout.argtypes = [vp] * 5 + [i, i, i, f, f, u64, vp]
    L.dadgpt_flash_attention_backward_bf16_dropout.argtypes = [vp] * 10 + [i, i, i, f, f, u64,
                                                                          vp]
    L.dadgpt_flash_attention_forward_dropout.argtypes = [vp] * 5 + [i, i, i, f, f, u64, vp]
    L.dadgpt_flash_attention_backward_dropout.argtypes = [vp] * 10 + [i, i, i, f, f, u64, vp]
    i64, hs = ctypes.c_int64, ctypes.POINTER(HeadStrides)
    L.dadgpt_flash_attention_forward_bf16_strided.argtypes = [vp] * 5 + [i, i, i, i, f, hs, vp]
    L.dadgpt_flash_attention_backward_bf16_strided.argtypes = [vp] * 10 + [i, i, i, i, f, hs,
                                                                          vp]
    L.dadgpt_flash_attention_forward_bf16_tokens.argtypes = [vp, i64, vp, vp, vp, vp, i64, i, i,
                                                             i, i, f, vp]
    L.dadgpt_flash_attention_backward_bf16_tokens.argtypes = [vp, vp, vp, i64, vp, vp, vp, i64,
                                                              vp, vp, vp, vp, i64, i, i, i, i, f,
                                                              vp]
    L.dadgpt_decode_workspace_bytes.restype = sz
    L.dadgpt_decode_workspace_bytes.argtypes = [i, i, i, i]
    L.dadgpt_decode_attention_bf16.argtypes = [vp] * 5 + [i, i, i, i, f, vp, sz, vp]
    L.dadgpt_decode_attention_f32.argtypes = [vp] * 5 + [i, i, i, i, f, vp, sz, vp]
    L.dadgpt_decode_attention_bf16_noalloc.argtypes = [vp] * 5 + [i, i, i, i, f, vp]
    L.dadgpt_softmax.argtypes = [vp, vp, i, i, vp]
    L.dadgpt_softmax_backward.argtypes = [vp, vp, vp, i, i, vp]
    L.dadgpt_causal_mask.argtypes = [vp, i, i, vp]
    L.dadgpt_causal_mask_zero.argtypes = [vp, i, i, vp]
    L.dadgpt_scale.argtypes = [vp, i64, f, vp]
    L.dadgpt_split_heads.argtypes = [vp, vp, i, i, i, i, vp]
    L.dadgpt_merge_heads.argtypes = [vp, vp, i, i, i, i, vp]
    L.dadgpt_attention_probs.argtypes = [vp, i, i, f, vp]
    L.dadgpt_attention_probs_backward.argtypes = [vp, vp, vp, i, i, f, vp]
    L.dadgpt_attention_dropout.argtypes = [vp, vp, i, i, f, u64, vp]
    L.dadgpt_attention_probs_backward_dropout.argtypes = [vp, vp, vp, i, i, f, f, u64, vp]
    L.dadgpt_decode_probs.argtypes = [vp, vp, i, i, i, f, vp]
    L.dadgpt_use_fused_attention.argtypes = [i, i, i, i]
    _lib = L
    return L


def last_error() -> str:
    return lib().dadgpt_last_error().decode()


def _check(status: int) -> None:
    if status != 0:
        raise AttentionError(status, last_error())


def _ptr(t) -> int | None:
    """Device address of a tensor (None for None: the C side reports the null pointer)."""
    if t is None:
        return None
    return t.data_ptr()


def _stream_ptr(stream) -> int | None:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream or None


def _require(t, name, dtype, numel, device=None):
    if t is None:
        return
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < numel:
        raise ValueError(f"{name} has {t.numel()} elements, needs {numel}")


# --------------------------------------------------------------- reference-named wrappers

def flash_attention_supported(d_head: int) -> bool:
    """gpu_flash_attention_supported (cuda/gpu_ops.cuh:115)."""
    return bool(lib().dadgpt_flash_attention_supported(int(d_head)))


def flash_attention_forward(out, lse, q, k, v, BH: int, S: int, d_head: int, scale: float,
                            stream=None) -> None:
    """gpu_flash_attention_forward (cuda/gpu_ops.cuh:116-117). fp32 buffers, overwritten."""
    n = BH * S * d_head
    for t, nm in ((out, "out"), (q, "q"), (k, "k"), (v, "v")):
        _require(t, nm, torch.float32, n)
    _require(lse, "lse", torch.float32, BH * S)
    _check(lib().dadgpt_flash_attention_forward_async(
        _ptr(out), _ptr(lse), _ptr(q), _ptr(k), _ptr(v), BH, S, d_head, scale,
        _stream_ptr(stream)))


def flash_attention_backward(dq, dk, dv, delta, dout, out, lse, q, k, v, BH: int, S: int,
                             d_head: int, scale: float, stream=None) -> None:
    """gpu_flash_attention_backward (cuda/gpu_ops.cuh:119-122). Writes dq, dk, dv and the
    delta scratch."""
    n = BH * S * d_head
    for t, nm in ((dq, "dq"), (dk, "dk"), (dv, "dv"), (dout, "dout"), (out, "out"),
                  (q, "q"), (k, "k"), (v, "v")):
        _require(t, nm, torch.float32, n)
    _require(delta, "delta", torch.float32, BH * S)
    _require(lse, "lse", torch.float32, BH * S)
    _check(lib().dadgpt_flash_attention_backward_async(
        _ptr(dq), _ptr(dk), _ptr(dv), _ptr(delta), _ptr(dout), _ptr(out), _ptr(lse), _ptr(q),
        _ptr(k), _ptr(v), BH, S, d_head, scale, _stream_ptr(stream)))


def flash_attention_forward_bf16(out, lse, q, k, v, BH: int, S: int, d_head: int,
                                 scale: float, stream=None) -> None:
    n = BH * S * d_head
    for t, nm in ((out, "out"), (q, "q"), (k, "k"), (v, "v")):
        _require(t, nm, torch.bfloat16, n)
    _require(lse, "lse", torch.float32, BH * S)
    _check(lib().dadgpt_flash_attention_forward_bf16(
        _ptr(out), _ptr(lse), _ptr(q), _ptr(k), _ptr(v), BH, S, d_head, scale,
        _stream_ptr(stream)))


def flash_attention_backward_bf16(dq, dk, dv, delta, dout, out, lse, q, k, v, BH: int, S: int,
                                  d_head: int, scale: float, stream=None) -> None:
    n = BH * S * d_head
    for t, nm in ((dq, "dq"), (dk, "dk"), (dv, "dv"), (dout, "dout"), (out, "out"),
                  (q, "q"), (k, "k"), (v, "v")):
        _require(t, nm, torch.bfloat16, n)
    _require(delta, "delta", torch.float32, BH * S)
    _require(lse, "lse", torch.float32, BH * S)
    _check(lib().dadgpt_flash_attention_backward_bf16(
        _ptr(dq), _ptr(dk), _ptr(dv), _ptr(delta), _ptr(dout), _ptr(out), _ptr(lse), _ptr(q),
        _ptr(k), _ptr(v), BH, S, d_head, scale, _stream_ptr(stream)))


def flash_attention_forward_dropout(out, lse, q, k, v, BH: int, S: int, d_head: int,
                                    scale: float, dropout_p: float, seed: int,
                                    stream=None) -> None:
    """fp32 forward with attention-probability dropout (the reference's precision)."""
    n = BH * S * d_head
    for t, nm in ((out, "out"), (q, "q"), (k, "k"), (v, "v")):
        _require(t, nm, torch.float32, n)
    _require(lse, "lse", torch.float32, BH * S)
    _check(lib().dadgpt_flash_attention_forward_dropout(
        _ptr(out), _ptr(lse), _ptr(q), _ptr(k), _ptr(v), BH, S, d_head, scale, dropout_p,
        seed & 0xFFFFFFFFFFFFFFFF, _stream_ptr(stream)))


def flash_attention_backward_dropout(dq, dk, dv, delta, dout, out, lse, q, k, v, BH: int,
                                     S: int, d_head: int, scale: float, dropout_p: float,
                                     seed: int, stream=None) -> None:
    """fp32 backward of flash_attention_forward_dropout with the same (dropout_p, seed)."""
    n = BH * S * d_head
    for t, nm in ((dq, "dq"), (dk, "dk"), (dv, "dv"), (dout, "dout"), (out, "out"),
                  (q, "q"), (k, "k"), (v, "v")):
        _require(t, nm, torch.float32, n)
    _require(delta, "delta", torch.float32, BH * S)
    _require(lse, "lse", torch.float32, BH * S)
    _check(lib().dadgpt_flash_attention_backward_dropout(
        _ptr(dq), _ptr(dk), _ptr(dv), _ptr(delta), _ptr(dout), _ptr(out), _ptr(lse), _ptr(q),
        _ptr(k), _ptr(v), BH, S, d_head, scale, dropout_p, seed & 0xFFFFFFFFFFFFFFFF,
        _stream_ptr(stream)))


def flash_attention_forward_bf16_dropout(out, lse, q, k, v, BH: int, S: int, d_head: int,
                                         scale: float, dropout_p: float, seed: int,
                                         stream=None) -> None:
    """bf16 forward with attention-probability dropout (the reference's materialized path
    with dropout, src/model.cpp:406-416, fused); the mask is a function of (seed, position)."""
    n = BH * S * d_head
    for t, nm in ((out, "out"), (q, "q"), (k, "k"), (v, "v")):
        _require(t, nm, torch.bfloat16, n)
    _require(lse, "lse", torch.float32, BH * S)
    _check(lib().dadgpt_flash_attention_forward_bf16_dropout(
        _ptr(out), _ptr(lse), _ptr(q), _ptr(k), _ptr(v), BH, S, d_head, scale, dropout_p,
        seed & 0xFFFFFFFFFFFFFFFF, _stream_ptr(stream)))


def flash_attention_backward_bf16_dropout(dq, dk, dv, delta, dout, out, lse, q, k, v, BH: int,
                                          S: int, d_head: int, scale: float, dropout_p: float,
                                          seed: int, stream=None) -> None:
    """The backward of flash_attention_forward_bf16_dropout with the same (dropout_p, seed)."""
    n = BH * S * d_head
    for t, nm in ((dq, "dq"), (dk, "dk"), (dv, "dv"), (dout, "dout"), (out, "out"),
                  (q, "q"), (k, "k"), (v, "v")):
        _require(t, nm, torch.bfloat16, n)
    _require(delta, "delta", torch.float32, BH * S)
    _require(lse, "lse", torch.float32, BH * S)
    _check(lib().dadgpt_flash_attention_backward_bf16_dropout(
        _ptr(dq), _ptr(dk), _ptr(dv), _ptr(delta), _ptr(dout), _ptr(out), _ptr(lse), _ptr(q),
        _ptr(k), _ptr(v), BH, S, d_head, scale, dropout_p, seed & 0xFFFFFFFFFFFFFFFF,
        _stream_ptr(stream)))


def flash_attention_backward_bf16_phase(phase: int, dq, dk, dv, delta, dout, out, lse, q, k, v,
                                        BH: int, S: int, d_head: int, scale: float,
                                        stream=None) -> None:
    """One kernel of the bf16 backward (0 delta, 1 dq, 2 dk/dv), for per-kernel timing."""
    _check(lib().dadgpt_flash_attention_backward_bf16_phase(
        int(phase), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(delta), _ptr(dout), _ptr(out), _ptr(lse),
        _ptr(q), _ptr(k), _ptr(v), BH, S, d_head, scale, _stream_ptr(stream)))


# ------------------------------------------------ strided layouts (no split/merge passes)

def _head_view(t, name, shape=None):
    """A bf16 device view [B, H, S, d_head] whose rows are contiguous -> its strides."""
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be a bfloat16 device tensor")
    if t.dim() != 4 or t.stride(3) != 1:
        raise ValueError(f"{name} must be a [B, H, S, d_head] view with contiguous rows")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    return HeadStrides(t.stride(0), t.stride(1), t.stride(2))


def flash_attention_forward_bf16_strided(out, lse, q, k, v, scale: float, stream=None) -> None:
    """Forward over [B, H, S, d_head] views of any row placement (e.g. heads sliced out of
    the token-major projection output, or a KV cache's first S rows); lse [B*H, S] fp32.
    Replaces split_heads + flash forward + merge_heads (src/model.cpp:384-392,423-424)."""
    B, H, S, D = q.shape
    st = (HeadStrides * 4)(*[_head_view(t, nm, (B, H, S, D))
                             for t, nm in ((q, "q"), (k, "k"), (v, "v"), (out, "out"))])
    _require(lse, "lse", torch.float32, B * H * S)
    _check(lib().dadgpt_flash_attention_forward_bf16_strided(
        _ptr(out), _ptr(lse), _ptr(q), _ptr(k), _ptr(v), B, H, S, D, scale, st,
        _stream_ptr(stream)))


def flash_attention_backward_bf16_strided(dq, dk, dv, delta, dout, out, lse, q, k, v,
                                          scale: float, stream=None) -> None:
    """Backward over [B, H, S, d_head] views (see flash_attention_forward_bf16_strided);
    replaces split_heads + flash backward + 3 merge_heads (src/model.cpp:564-576,619-624)."""
    B, H, S, D = q.shape
    views = ((q, "q"), (k, "k"), (v, "v"), (out, "out"), (dout, "dout"), (dq, "dq"),
             (dk, "dk"), (dv, "dv"))
    st = (HeadStrides * 8)(*[_head_view(t, nm, (B, H, S, D)) for t, nm in views])
    _require(delta, "delta", torch.float32, B * H * S)
    _require(lse, "lse", torch.float32, B * H * S)
    _check(lib().dadgpt_flash_attention_backward_bf16_strided(
        _ptr(dq), _ptr(dk), _ptr(dv), _ptr(delta), _ptr(dout), _ptr(out), _ptr(lse), _ptr(q),
        _ptr(k), _ptr(v), B, H, S, D, scale, st, _stream_ptr(stream)))


def flash_attention_forward_bf16_tokens(out, ld_out: int, lse, q, k, v, ld_qkv: int, B: int,
                                        H: int, S: int, d_head: int, scale: float,
                                        stream=None) -> None:
    """Token-major forward: rows b*S + s of q, k, v (pitch ld_qkv) and out (pitch ld_out)
    hold the H heads side by side. q, k, v may be slices of one fused [B*S, 3*H*d_head]
    projection output (ld_qkv = 3*H*d_head). Raw device buffers, as the C ABI."""
    _check(lib().dadgpt_flash_attention_forward_bf16_tokens(
        _ptr(out), ld_out, _ptr(lse), _ptr(q), _ptr(k), _ptr(v), ld_qkv, B, H, S, d_head, scale,
        _stream_ptr(stream)))


def flash_attention_backward_bf16_tokens(dq, dk, dv, ld_dqkv: int, delta, dout, out,
                                         ld_out: int, lse, q, k, v, ld_qkv: int, B: int, H: int,
                                         S: int, d_head: int, scale: float,
                                         stream=None) -> None:
    """Token-major backward (see flash_attention_forward_bf16_tokens); dq, dk, dv rows
    ld_dqkv apart (3*H*d_head: the gradient of a fused QKV projection output)."""
    _check(lib().dadgpt_flash_attention_backward_bf16_tokens(
        _ptr(dq), _ptr(dk), _ptr(dv), ld_dqkv, _ptr(delta), _ptr(dout), _ptr(out), ld_out,
        _ptr(lse), _ptr(q), _ptr(k), _ptr(v), ld_qkv, B, H, S, d_head, scale,
        _stream_ptr(stream)))


def decode_workspace_bytes(n_seq: int, n_heads: int, max_len: int, d_head: int) -> int:
    return int(lib().dadgpt_decode_workspace_bytes(n_seq, n_heads, max_len, d_head))


def decode_workspace(n_seq, n_heads, max_len, d_head, device="cuda"):
    """The workspace decode_attention needs for this cache shape, or None when it needs
    none (max_len fits one workgroup chunk). It is zero-filled, as the library requires
    before first use (its arrival counters start at zero; every call leaves them there)."""
    nbytes = decode_workspace_bytes(n_seq, n_heads, max_len, d_head)
    if nbytes == 0:
        return None
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def decode_attention(out, q, k_cache, v_cache, lens, n_seq, n_heads, max_len, d_head, scale,
                     workspace, stream=None) -> None:
    """Ragged KV-cache decode (the per-head composition of src/model.cpp:758-790 as one
    launch). bf16 or fp32 by the tensors' dtype; lens is a device int32 tensor."""
    dt = q.dtype
    if dt not in (torch.bfloat16, torch.float32):
        raise TypeError("decode_attention: q must be bfloat16 or float32")
    _require(q, "q", dt, n_seq * n_heads * d_head)
    _require(out, "out", dt, n_seq * n_heads * d_head)
    _require(k_cache, "k_cache", dt, n_seq * n_heads * max_len * d_head)
    _require(v_cache, "v_cache", dt, n_seq * n_heads * max_len * d_head)
    _require(lens, "lens", torch.int32, n_seq)
    if workspace is not None and (not workspace.is_cuda or not workspace.is_contiguous()):
        raise ValueError("workspace must be a contiguous device tensor")
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    fn = (lib().dadgpt_decode_attention_bf16 if dt == torch.bfloat16
          else lib().dadgpt_decode_attention_f32)
    _check(fn(_ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(lens), n_seq, n_heads,
              max_len, d_head, scale, _ptr(workspace), ws_bytes, _stream_ptr(stream)))


# --------------------------------------------------------------- allocating conveniences

# Scratch each device holds for decode_attention_noalloc (the header's
# DADGPT_DECODE_NOALLOC_SCRATCH_BYTES).
DECODE_NOALLOC_SCRATCH_BYTES = 4 << 20


def decode_attention_noalloc(out, q, k_cache, v_cache, lens, n_seq, n_heads, max_len, d_head,
                             scale, stream=None) -> None:
    """bf16 decode without a workspace argument: the library's fixed per-device scratch
    (DECODE_NOALLOC_SCRATCH_BYTES) holds the split-cache partials, so the call allocates
    nothing. Calls that overlap in time on one device race on that scratch."""
    dt = torch.bfloat16
    _require(q, "q", dt, n_seq * n_heads * d_head)
    _require(out, "out", dt, n_seq * n_heads * d_head)
    _require(k_cache, "k_cache", dt, n_seq * n_heads * max_len * d_head)
    _require(v_cache, "v_cache", dt, n_seq * n_heads * max_len * d_head)
    _require(lens, "lens", torch.int32, n_seq)
    _check(lib().dadgpt_decode_attention_bf16_noalloc(
        _ptr(out), _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(lens), n_seq, n_heads, max_len,
        d_head, scale, _stream_ptr(stream)))


# ---------------------------------------------------------------- materialized attention

# The reference's AttentionImpl (src/model.hpp:80).
ATTENTION_IMPL = {"auto": 0, "fused": 1, "materialized": 2}


def use_fused_attention(impl: str, d_head: int, ctx_len: int, attn_dropout: bool) -> bool:
    """use_fused_attention (src/model.cpp:183-197): dropout or an unsupported d_head take the
    materialized path; 'fused' / 'materialized' force theirs; 'auto' is fused from ctx 512."""
    return bool(lib().dadgpt_use_fused_attention(ATTENTION_IMPL[impl], d_head, ctx_len,
                                                 int(bool(attn_dropout))))


def _rows(t, name, numel):
    _require(t, name, torch.float32, numel)


def softmax(out, x, rows: int, cols: int, stream=None) -> None:
    """gpu_softmax (cuda/gpu_ops.cu:147-199): row softmax of x [rows, cols] into out."""
    _rows(out, "out", rows * cols)
    _rows(x, "in", rows * cols)
    _check(lib().dadgpt_softmax(_ptr(out), _ptr(x), rows, cols, _stream_ptr(stream)))


def softmax_backward(din, dout, out, rows: int, cols: int, stream=None) -> None:
    """gpu_softmax_backward (cuda/gpu_ops.cu:542-569): din += out (dout - rowsum(dout out))."""
    for t, n in ((din, "din"), (dout, "dout"), (out, "out")):
        _rows(t, n, rows * cols)
    _check(lib().dadgpt_softmax_backward(_ptr(din), _ptr(dout), _ptr(out), rows, cols,
                                         _stream_ptr(stream)))


def causal_mask(scores, n_blocks: int, S: int, zero: bool = False, stream=None) -> None:
    """gpu_causal_mask (-1e9) or gpu_causal_mask_zero (0) above each block's diagonal
    (cuda/gpu_ops.cu:476-511)."""
    _rows(scores, "scores", n_blocks * S * S)
    fn = lib().dadgpt_causal_mask_zero if zero else lib().dadgpt_causal_mask
    _check(fn(_ptr(scores), n_blocks, S, _stream_ptr(stream)))


def scale_(x, scale: float, stream=None) -> None:
    """gpu_scale (cuda/gpu_ops.cu:513-525): x *= scale in place."""
    _rows(x, "data", x.numel())
    _check(lib().dadgpt_scale(_ptr(x), x.numel(), scale, _stream_ptr(stream)))


def split_heads(out, inp, batch_size: int, seq_len: int, n_heads: int, d_head: int,
                stream=None) -> None:
    """gpu_split_heads (cuda/gpu_ops.cu:426-446): fp32 [B*S, H*dh] -> [B*H, S, dh]."""
    n = batch_size * seq_len * n_heads * d_head
    _rows(out, "out", n)
    _rows(inp, "in", n)
    _check(lib().dadgpt_split_heads(_ptr(out), _ptr(inp), batch_size, seq_len, n_heads, d_head,
                                    _stream_ptr(stream)))


def merge_heads(out, inp, batch_size: int, seq_len: int, n_heads: int, d_head: int,
                stream=None) -> None:
    """gpu_merge_heads (cuda/gpu_ops.cu:448-474): fp32 [B*H, S, dh] -> [B*S, H*dh]."""
    n = batch_size * seq_len * n_heads * d_head
    _rows(out, "out", n)
    _rows(inp, "in", n)
    _check(lib().dadgpt_merge_heads(_ptr(out), _ptr(inp), batch_size, seq_len, n_heads, d_head,
                                    _stream_ptr(stream)))


def attention_probs(probs, BH: int, S: int, scale: float, stream=None) -> None:
    """Scores [BH,S,S] -> probabilities in place (x scale, causal -1e9, row softmax)."""
    _rows(probs, "probs", BH * S * S)
    _check(lib().dadgpt_attention_probs(_ptr(probs), BH, S, scale, _stream_ptr(stream)))


def attention_probs_backward(dscores, dprobs, probs, BH: int, S: int, scale: float,
                             stream=None) -> None:
    """d(scores) from d(probs) and probs (softmax backward, causal zero, x scale)."""
    for t, n in ((dscores, "dscores"), (dprobs, "dprobs"), (probs, "probs")):
        _rows(t, n, BH * S * S)
    _check(lib().dadgpt_attention_probs_backward(_ptr(dscores), _ptr(dprobs), _ptr(probs), BH, S,
                                                 scale, _stream_ptr(stream)))


def attention_dropout(dropped, probs, BH: int, S: int, dropout_p: float, seed: int,
                      stream=None) -> None:
    """dropped = probs * keep / (1 - dropout_p) over [BH,S,S] (src/model.cpp:406-416), with the
    flash _dropout entry points' mask; dropped may be probs."""
    _rows(dropped, "dropped", BH * S * S)
    _rows(probs, "probs", BH * S * S)
    _check(lib().dadgpt_attention_dropout(_ptr(dropped), _ptr(probs), BH, S, dropout_p, seed,
                                          _stream_ptr(stream)))


def attention_probs_backward_dropout(dscores, dprobs, probs, BH: int, S: int, scale: float,
                                     dropout_p: float, seed: int, stream=None) -> None:
    """attention_probs_backward after the dropout backward (src/model.cpp:594-607): dprobs (of
    the dropped probabilities) times keep / (1 - dropout_p), softmax backward against probs."""
    for t, n in ((dscores, "dscores"), (dprobs, "dprobs"), (probs, "probs")):
        _rows(t, n, BH * S * S)
    _check(lib().dadgpt_attention_probs_backward_dropout(
        _ptr(dscores), _ptr(dprobs), _ptr(probs), BH, S, scale, dropout_p, seed,
        _stream_ptr(stream)))


def decode_probs(probs, lens, n_seq: int, n_heads: int, max_len: int, scale: float,
                 stream=None) -> None:
    """Decode scores [n_seq*H, max_len] -> probabilities over each sequence's first lens keys."""
    _rows(probs, "probs", n_seq * n_heads * max_len)
    _require(lens, "lens", torch.int32, n_seq)
    _check(lib().dadgpt_decode_probs(_ptr(probs), _ptr(lens), n_seq, n_heads, max_len, scale,
                                     _stream_ptr(stream)))


def default_scale(d_head: int) -> float:
    """1/sqrt(d_head), as src/model.cpp:389 computes it (in fp32)."""
    return float(torch.tensor(1.0 / math.sqrt(d_head), dtype=torch.float32))


def attention_forward(q, k, v, scale=None):
    """Allocating forward: q, k, v [BH, S, D] (fp32 or bf16) -> (out, lse)."""
    BH, S, D = q.shape
    scale = default_scale(D) if scale is None else scale
    out = torch.empty_like(q)
    lse = torch.empty((BH, S), dtype=torch.float32, device=q.device)
    if q.dtype == torch.bfloat16:
        flash_attention_forward_bf16(out, lse, q, k, v, BH, S, D, scale)
    else:
        flash_attention_forward(out, lse, q, k, v, BH, S, D, scale)
    return out, lse


def attention_backward(dout, out, lse, q, k, v, scale=None):
    """Allocating backward -> (dq, dk, dv, delta)."""
    BH, S, D = q.shape
    scale = default_scale(D) if scale is None else scale
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty((BH, S), dtype=torch.float32, device=q.device)
    if q.dtype == torch.bfloat16:
        flash_attention_backward_bf16(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, D,
                                      scale)
    else:
        flash_attention_backward(dq, dk, dv, delta, dout, out, lse, q, k, v, BH, S, D, scale)
    return dq, dk, dv, delta
