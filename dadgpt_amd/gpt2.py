"""Python mirror of libdadgpt_gen: bf16 hipBLASLt projections and batched GPT-2 generation.

The C ABI is declared in include/dadgpt/gpt2_generate.h and include/dadgpt/gpu_matmul.h.
It replaces the reference's generation stack (src/generate.cpp:94-139 generate_tokens with
greedy sample_token, src/model.cpp:659-851 KV cache, cached forward and prefill) and its
cuBLAS projection wrappers (cuda/gpu_ops.cu:94-112). Like the attention wrappers, every call
raises on failure and there is no fallback: a missing library raises ``LibraryNotBuilt``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

from . import attention as _attn

GEN_PATH = os.path.join(_attn.HERE, "lib", "libdadgpt_gen.so")

# The reference's named architectures (src/model.cpp:221-234); vocab as GPT-2's tokenizer.
PRESETS = {
    "tiny": dict(d_model=128, n_layers=2, n_heads=4, d_ff=512, ctx_len=64, vocab_size=512),
    "small": dict(d_model=512, n_layers=8, n_heads=8, d_ff=2048, ctx_len=128, vocab_size=512),
    "gpt2-124m": dict(d_model=768, n_layers=12, n_heads=12, d_ff=3072, ctx_len=1024,
                      vocab_size=50257),
}

GEN_SYMBOLS = (
    "dadgpt_gen_last_error",
    "dadgpt_blas_open",
    "dadgpt_blas_create",
    "dadgpt_blas_destroy",
    "dadgpt_blas_library_version",
    "dadgpt_blas_stack_versions",
    "dadgpt_blas_stack_supported",
    "dadgpt_set_matmul_precision",
    "dadgpt_get_matmul_precision",
    "dadgpt_matmul_bf16",
    "dadgpt_matmul_transposed_b_bf16",
    "dadgpt_matmul_f32",
    "dadgpt_matmul_f32_strided_batched",
    "dadgpt_attention_materialized_forward",
    "dadgpt_attention_materialized_backward",
    "dadgpt_attention_materialized_forward_dropout",
    "dadgpt_attention_materialized_backward_dropout",
    "dadgpt_gpt2_param_count",
    "dadgpt_gpt2_init_params",
    "dadgpt_gpt2_create",
    "dadgpt_gpt2_destroy",
    "dadgpt_gpt2_set_graphs",
    "dadgpt_gpt2_generate",
    "dadgpt_gpt2_truncate_prompt",
    "dadgpt_gpt2_generate_tokens",
)


class Config(ctypes.Structure):
    _fields_ = [(k, ctypes.c_int) for k in
                ("d_model", "n_layers", "n_heads", "d_ff", "ctx_len", "vocab_size")]

    @classmethod
    def of(cls, cfg) -> "Config":
        if isinstance(cfg, Config):
            return cfg
        if isinstance(cfg, str):
            cfg = PRESETS[cfg]
        return cls(**cfg)

    def as_dict(self) -> dict:
        return {k: getattr(self, k) for k, _ in self._fields_}


class Timing(ctypes.Structure):
    _fields_ = [("prefill_ms", ctypes.c_float), ("decode_ms", ctypes.c_float),
                ("decode_attn_ms", ctypes.c_float), ("decode_steps", ctypes.c_int)]


_gen = None


def gen_lib():
    """The loaded generation library (after the attention library it links against)."""
    global _gen
    if _gen is not None:
        return _gen
    _attn.lib()
    if not os.path.exists(GEN_PATH):
        raise _attn.LibraryNotBuilt(f"{GEN_PATH} is not built; run __graft_entry__.build()")
    try:
        L = ctypes.CDLL(GEN_PATH)
    except OSError as e:  # pragma: no cover - depends on the machine
        raise _attn.LibraryNotBuilt(f"cannot load {GEN_PATH}: {e}") from e
    vp, i, f, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    cfgp = ctypes.POINTER(Config)
    L.dadgpt_gen_last_error.restype = ctypes.c_char_p
    L.dadgpt_gen_last_error.argtypes = []
    L.dadgpt_blas_open.argtypes = []
    L.dadgpt_blas_create.argtypes = [ctypes.POINTER(vp)]
    L.dadgpt_blas_destroy.argtypes = [vp]
    L.dadgpt_blas_destroy.restype = None
    L.dadgpt_matmul_bf16.argtypes = [vp, vp, vp, vp, i, i, i, vp]
    L.dadgpt_matmul_transposed_b_bf16.argtypes = [vp, vp, vp, vp, i, i, i, vp]
    ll = ctypes.c_longlong
    L.dadgpt_blas_library_version.argtypes = [vp]
    L.dadgpt_blas_stack_versions.argtypes = [ctypes.POINTER(i), ctypes.POINTER(i)]
    L.dadgpt_blas_stack_supported.argtypes = [i, i]
    L.dadgpt_set_matmul_precision.argtypes = [i]
    L.dadgpt_get_matmul_precision.argtypes = []
    L.dadgpt_matmul_f32.argtypes = [vp, vp, vp, vp, i, i, i, i, f, vp]
    L.dadgpt_matmul_f32_strided_batched.argtypes = [vp, vp, vp, vp, i, i, i, i, f, ll, ll, ll, i,
                                                    vp]
    L.dadgpt_attention_materialized_forward.argtypes = [vp] * 6 + [i, i, i, f, vp]
    L.dadgpt_attention_materialized_backward.argtypes = [vp] * 10 + [i, i, i, f, vp]
    u64 = ctypes.c_uint64
    L.dadgpt_attention_materialized_forward_dropout.argtypes = [vp] * 7 + [i, i, i, f, f, u64,
                                                                           vp]
    L.dadgpt_attention_materialized_backward_dropout.argtypes = [vp] * 10 + [i, i, i, f, f, u64,
                                                                             vp]
    L.dadgpt_gpt2_param_count.argtypes = [cfgp]
    L.dadgpt_gpt2_param_count.restype = sz
    L.dadgpt_gpt2_init_params.argtypes = [vp, cfgp, ctypes.c_uint64, vp]
    L.dadgpt_gpt2_create.argtypes = [cfgp, vp, i, i, ctypes.POINTER(vp)]
    L.dadgpt_gpt2_destroy.argtypes = [vp]
    L.dadgpt_gpt2_destroy.restype = None
    L.dadgpt_gpt2_set_graphs.argtypes = [vp, i]
    L.dadgpt_gpt2_generate.argtypes = [vp, vp, vp, i, i, i, vp, vp, vp, ctypes.POINTER(Timing)]
    L.dadgpt_gpt2_truncate_prompt.argtypes = [vp, i, i, i, vp, vp]
    L.dadgpt_gpt2_generate_tokens.argtypes = [vp, vp, vp, i, i, i, vp, vp, i, vp]
    for name in GEN_SYMBOLS:
        if name not in ("dadgpt_gen_last_error", "dadgpt_blas_destroy", "dadgpt_gpt2_destroy",
                        "dadgpt_gpt2_param_count"):
            getattr(L, name).restype = i
    _gen = L
    return L


def last_error() -> str:
    return gen_lib().dadgpt_gen_last_error().decode()


def _check(status: int) -> None:
    if status != 0:
        raise _attn.AttentionError(status, last_error())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


# ------------------------------------------------------------------------------ GEMMs

def _version_str(v: int, major: int, minor: int) -> str:
    return "unknown" if v < 0 else f"{v // major}.{v // minor % (major // minor)}.{v % minor}"


def blas_stack_versions() -> dict:
    """The process's HIP runtime and hipBLASLt versions (as numbers and dotted), and whether
    dadgpt_blas_create accepts the pair (a combination the GPU tests cover)."""
    rt, lt = ctypes.c_int(), ctypes.c_int()
    _check(gen_lib().dadgpt_blas_stack_versions(ctypes.byref(rt), ctypes.byref(lt)))
    return {"hip_runtime": rt.value, "hipblaslt": lt.value,
            "hip_runtime_str": _version_str(rt.value, 10_000_000, 100_000),
            "hipblaslt_str": _version_str(lt.value, 100_000, 100),
            "supported": bool(gen_lib().dadgpt_blas_stack_supported(rt.value, lt.value))}


def blas_stack_supported(hip_runtime: int, hipblaslt: int) -> bool:
    return bool(gen_lib().dadgpt_blas_stack_supported(hip_runtime, hipblaslt))

# The reference's MatmulPrecision (cuda/gpu_ops.cuh:43), process-wide.
PRECISIONS = {"fp32": 0, "tf32": 1, "bf16": 2}


def set_matmul_precision(name: str) -> None:
    """gpu_set_matmul_precision (cuda/gpu_ops.cu:63-67) for the fp32 GEMMs below: 'fp32',
    'tf32' (runs as fp32 on gfx950) or 'bf16' (inputs rounded to bf16 inside the GEMM)."""
    _check(gen_lib().dadgpt_set_matmul_precision(PRECISIONS[name]))


def get_matmul_precision() -> str:
    v = gen_lib().dadgpt_get_matmul_precision()
    return {k: n for n, k in PRECISIONS.items()}[v]


class Blas:
    """An opaque hipBLASLt handle (the reference's cublasHandle_t, src/model.cpp:236)."""

    def __init__(self):
        self._h = ctypes.c_void_p()
        # bound now: at interpreter exit __del__ may run after this module's globals are gone
        self._destroy = gen_lib().dadgpt_blas_destroy
        _check(gen_lib().dadgpt_blas_create(ctypes.byref(self._h)))

    def close(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = ctypes.c_void_p()

    __del__ = close

    def _mm(self, fn, a, b, M, K, N):
        for t, nm in ((a, "a"), (b, "b")):
            if t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{nm} must be a contiguous bfloat16 device tensor")
        out = torch.empty(M, N, dtype=torch.float32, device=a.device)
        _check(fn(self._h, out.data_ptr(), a.data_ptr(), b.data_ptr(), M, K, N, _stream()))
        return out

    def matmul(self, a, b):
        """gpu_matmul (cuda/gpu_ops.cu:94-98): a [M,K] @ b [K,N] -> fp32 [M,N]."""
        (M, K), (K2, N) = a.shape, b.shape
        if K != K2:
            raise ValueError("inner dimensions differ")
        return self._mm(gen_lib().dadgpt_matmul_bf16, a, b, M, K, N)

    def matmul_transposed_b(self, a, b):
        """gpu_matmul_transposed_b (cuda/gpu_ops.cu:108-112): a [M,K] @ b[N,K]^T -> [M,N]."""
        (M, K), (N, K2) = a.shape, b.shape
        if K != K2:
            raise ValueError("inner dimensions differ")
        return self._mm(gen_lib().dadgpt_matmul_transposed_b_bf16, a, b, M, K, N)

    def library_version(self) -> int:
        """The hipBLASLt version behind the handle (major*100000 + minor*100 + patch)."""
        return int(gen_lib().dadgpt_blas_library_version(self._h))

    @staticmethod
    def _f32(t, name):
        if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 device tensor")

    def matmul_f32(self, out, a, b, M: int, K: int, N: int, op: str = "N",
                   beta: float = 0.0) -> None:
        """fp32 GEMM into out [M,N]: op 'N' gpu_matmul (a [M,K], b [K,N]), 'A'
        gpu_matmul_transposed_a (a [K,M]; beta 1 accumulates), 'B' gpu_matmul_transposed_b
        (b [N,K]) (cuda/gpu_ops.cu:94-112), at the process-wide precision."""
        for t, nm in ((out, "out"), (a, "a"), (b, "b")):
            self._f32(t, nm)
        _check(gen_lib().dadgpt_matmul_f32(self._h, out.data_ptr(), a.data_ptr(), b.data_ptr(),
                                           M, K, N, ord(op), beta, _stream()))

    def matmul_f32_batched(self, out, a, b, M: int, K: int, N: int, op: str, beta: float,
                           stride_a: int, stride_b: int, stride_out: int, count: int) -> None:
        """Strided-batched fp32 GEMM: op 'B' beta 0 gpu_matmul_strided_batched_bt, 'N' beta 0
        gpu_matmul_strided_batched, 'A' beta 1 gpu_matmul_strided_batched_at
        (cuda/gpu_ops.cu:117-141)."""
        for t, nm in ((out, "out"), (a, "a"), (b, "b")):
            self._f32(t, nm)
        _check(gen_lib().dadgpt_matmul_f32_strided_batched(
            self._h, out.data_ptr(), a.data_ptr(), b.data_ptr(), M, K, N, ord(op), beta,
            stride_a, stride_b, stride_out, count, _stream()))

    def attention_materialized_forward(self, out, probs, q, k, v, BH: int, S: int, d_head: int,
                                       scale: float) -> None:
        """The reference's materialized attention forward (src/model.cpp:395-420): probs
        [BH,S,S] receives softmax(mask(q k^T * scale)), out = probs v."""
        for t, nm in ((out, "out"), (probs, "probs"), (q, "q"), (k, "k"), (v, "v")):
            self._f32(t, nm)
        _check(gen_lib().dadgpt_attention_materialized_forward(
            self._h, out.data_ptr(), probs.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
            BH, S, d_head, scale, _stream()))

    def attention_materialized_backward(self, dq, dk, dv, dscores, dout, probs, q, k, v, BH: int,
                                        S: int, d_head: int, scale: float) -> None:
        """Its backward (src/model.cpp:575-616): dq, dk, dv overwritten; dscores [BH,S,S]
        scratch."""
        ts = (dq, dk, dv, dscores, dout, probs, q, k, v)
        for t, nm in zip(ts, ("dq", "dk", "dv", "dscores", "dout", "probs", "q", "k", "v")):
            self._f32(t, nm)
        _check(gen_lib().dadgpt_attention_materialized_backward(
            self._h, *[t.data_ptr() for t in ts], BH, S, d_head, scale, _stream()))

    def attention_materialized_forward_dropout(self, out, probs, dropped, q, k, v, BH: int,
                                               S: int, d_head: int, scale: float,
                                               dropout_p: float, seed: int) -> None:
        """The forward with attention dropout (src/model.cpp:395-420): probs [BH,S,S] receives
        the probabilities, dropped [BH,S,S] probs * keep / (1 - dropout_p), out = dropped v."""
        ts = (out, probs, dropped, q, k, v)
        for t, nm in zip(ts, ("out", "probs", "dropped", "q", "k", "v")):
            self._f32(t, nm)
        _check(gen_lib().dadgpt_attention_materialized_forward_dropout(
            self._h, *[t.data_ptr() for t in ts], BH, S, d_head, scale, dropout_p, seed,
            _stream()))

    def attention_materialized_backward_dropout(self, dq, dk, dv, dscores, dout, probs, q, k, v,
                                                BH: int, S: int, d_head: int, scale: float,
                                                dropout_p: float, seed: int) -> None:
        """Its backward (src/model.cpp:575-616 with :594-599): same seed and dropout_p as the
        forward; dscores [BH,S,S] scratch."""
        ts = (dq, dk, dv, dscores, dout, probs, q, k, v)
        for t, nm in zip(ts, ("dq", "dk", "dv", "dscores", "dout", "probs", "q", "k", "v")):
            self._f32(t, nm)
        _check(gen_lib().dadgpt_attention_materialized_backward_dropout(
            self._h, *[t.data_ptr() for t in ts], BH, S, d_head, scale, dropout_p, seed,
            _stream()))


# ------------------------------------------------------------------------ the model

def param_count(cfg) -> int:
    c = Config.of(cfg)
    return int(gen_lib().dadgpt_gpt2_param_count(ctypes.byref(c)))


def init_params(cfg, seed: int, device="cuda") -> torch.Tensor:
    """A device bf16 parameter arena with the reference's GPT-2 initialisation
    (src/model.cpp:121-166), from a seeded counter-based stream."""
    c = Config.of(cfg)
    n = param_count(c)
    if n == 0:
        raise ValueError(f"invalid config {c.as_dict()}")
    params = torch.empty(n, dtype=torch.bfloat16, device=device)
    _check(gen_lib().dadgpt_gpt2_init_params(params.data_ptr(), ctypes.byref(c), seed,
                                             _stream()))
    return params


def truncate_prompt(prompt, max_len: int, ctx_len: int) -> list:
    """generate_tokens' prompt truncation (src/generate.cpp:97-110), as the library applies
    it: with eff = min(max_len, ctx_len), a prompt of at least eff tokens (and more than one)
    keeps its first token and its last max(eff - 2, 0) tokens."""
    p = np.ascontiguousarray(np.asarray(prompt, np.int32))
    out = np.zeros(max(len(p), 1), np.int32)
    n = ctypes.c_int32()
    _check(gen_lib().dadgpt_gpt2_truncate_prompt(p.ctypes.data, len(p), max_len, ctx_len,
                                                 out.ctypes.data, ctypes.byref(n)))
    return [int(t) for t in out[:n.value]]


# Attention of a model (include/dadgpt/gpt2_generate.h DADGPT_GPT2_ATTN_*), and the flag for
# fp32 projections (DADGPT_GPT2_FP32_PROJECTIONS).
ATTENTION = {"bf16": 0, "fp32": 1, "fp32_materialized": 2}
FP32_PROJECTIONS = 0x100


class GPT2:
    """Batched greedy generation over a bf16 parameter arena (kept referenced here).

    attention: 'bf16' (flash prefill and decode kernels over bf16 caches), 'fp32' (the fp32
    flash kernels over fp32 caches) or 'fp32_materialized' (the reference's materialized path
    on fp32 GEMMs, over fp32 caches); everything else is identical.
    projections: 'bf16' (bf16 GEMM inputs, the default) or 'fp32' (with fp32 attention: the
    reference's fp32 precision end to end)."""

    def __init__(self, cfg, params: torch.Tensor, max_batch: int, attention: str = "bf16",
                 projections: str = "bf16"):
        self.cfg = Config.of(cfg)
        if params.dtype != torch.bfloat16 or not params.is_cuda:
            raise ValueError("params must be a bfloat16 device tensor")
        if params.numel() != param_count(self.cfg):
            raise ValueError("params has the wrong size for this config")
        self.params = params
        self.max_batch = max_batch
        self._m = ctypes.c_void_p()
        self._destroy = gen_lib().dadgpt_gpt2_destroy  # bound now, as in Blas
        torch.cuda.synchronize()  # the arena may still be being written on torch's stream
        _check(gen_lib().dadgpt_gpt2_create(ctypes.byref(self.cfg), params.data_ptr(), max_batch,
                                            ATTENTION[attention] |
                                            (FP32_PROJECTIONS if projections == "fp32" else 0),
                                            ctypes.byref(self._m)))
        self.attention, self.projections = attention, projections

    def close(self):
        if getattr(self, "_m", None):
            self._destroy(self._m)
            self._m = ctypes.c_void_p()

    __del__ = close

    def set_graphs(self, enable: bool) -> None:
        """Replay a captured decode step (default) or launch every step eagerly."""
        _check(gen_lib().dadgpt_gpt2_set_graphs(self._m, int(enable)))

    def generate(self, prompts, new_tokens: int, logits: bool = False, timing: bool = False):
        """prompts: list of 1-D int sequences. Returns a dict with tokens [n, new_tokens]
        int32, margins [n, new_tokens] float32, and optionally logits
        [new_tokens, n, vocab] float32 and timing (ms)."""
        n = len(prompts)
        lens = np.array([len(p) for p in prompts], np.int32)
        stride = int(lens.max())
        pad = np.zeros((n, stride), np.int32)
        for b, p in enumerate(prompts):
            pad[b, :len(p)] = np.asarray(p, np.int32)
        toks = np.zeros((n, new_tokens), np.int32)
        margins = np.zeros((n, new_tokens), np.float32)
        lg = np.zeros((new_tokens, n, self.cfg.vocab_size), np.float32) if logits else None
        tm = Timing()
        torch.cuda.synchronize()
        _check(gen_lib().dadgpt_gpt2_generate(
            self._m, pad.ctypes.data, lens.ctypes.data, n, stride, new_tokens, toks.ctypes.data,
            margins.ctypes.data, None if lg is None else lg.ctypes.data,
            ctypes.byref(tm) if timing else None))
        out = {"tokens": toks, "margins": margins}
        if lg is not None:
            out["logits"] = lg
        if timing:
            out["timing"] = {"prefill_ms": tm.prefill_ms, "decode_ms": tm.decode_ms,
                             "decode_attn_ms": tm.decode_attn_ms,
                             "decode_steps": tm.decode_steps}
        return out

    def generate_tokens(self, prompts, max_len: int, stop_tokens=None):
        """generate_tokens (src/generate.cpp:94-139) with greedy sampling for a batch: each
        row's prompt is truncated as truncate_prompt does, then greedy picks are appended until
        the row holds min(max_len, ctx_len) tokens or picks its stop token (kept as its last
        token). stop_tokens: one per row (-1 for none), or None. Returns one list per row:
        the truncated prompt followed by the picks."""
        n = len(prompts)
        lens = np.array([len(p) for p in prompts], np.int32)
        stride = int(lens.max())
        pad = np.zeros((n, stride), np.int32)
        for b, p in enumerate(prompts):
            pad[b, :len(p)] = np.asarray(p, np.int32)
        stops = None
        if stop_tokens is not None:
            stops = np.ascontiguousarray(np.asarray(stop_tokens, np.int32))
            if stops.shape != (n,):
                raise ValueError("stop_tokens needs one entry per prompt")
        out_stride = max(min(max_len, self.cfg.ctx_len), 1)
        out = np.zeros((n, out_stride), np.int32)
        out_lens = np.zeros(n, np.int32)
        torch.cuda.synchronize()
        _check(gen_lib().dadgpt_gpt2_generate_tokens(
            self._m, pad.ctypes.data, lens.ctypes.data, n, stride, max_len,
            None if stops is None else stops.ctypes.data, out.ctypes.data, out_stride,
            out_lens.ctypes.data))
        return [[int(t) for t in out[b, :out_lens[b]]] for b in range(n)]
