"""CPU oracle for the fused causal attention path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this package, and only as the checker or the timed CPU baseline. The product path
(``dadgpt_amd``) never imports it.

Two libraries, both built by ``oracle/Makefile``:

* ``liboracle_attn.so`` — ``attn_oracle.c``, a plain-C restatement of the reference's CPU
  operators composed in the op order of its materialized attention (``src/model.cpp:396-419``,
  ``:585-615``, decode ``:765-790``).
* ``_ref/libref_attn.so`` — the reference's own ``src/tensor_ops.cpp`` and
  ``src/backward.cpp`` compiled from ``/root/reference`` plus ``ref_glue.cpp``. Present only
  where ``/root/reference`` was available at build time (and on GPU boxes the tree was sent to).

Numpy in, numpy out; float32 arrays for the f32 functions, float64 for the f64 twins.

``gpt2_oracle`` (numpy) restates the GPT-2 forward of the generation path; ``ref_gpt2_forward``
composes the reference's own CPU operators (``src/tensor_ops.cpp``, from ``_ref``) in
``model_forward``'s order to pin it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_attn.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_attn.so")

_lib = None
_ref = None

_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_ip = ctypes.POINTER(ctypes.c_int)


def build(with_ref: bool | None = None) -> None:
    """Compile the oracle (and the reference build when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if with_ref is None:
        with_ref = os.path.isdir("/root/reference/src")
    if with_ref:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _f(a):
    return a.ctypes.data_as(_fp)


def _d(a):
    return a.ctypes.data_as(_dp)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(with_ref=False)
        L = ctypes.CDLL(LIB_PATH)
        i, f, d = ctypes.c_int, ctypes.c_float, ctypes.c_double
        L.oracle_attn_fwd_f32.argtypes = [_fp, _fp, _fp, _fp, _fp, i, i, i, f]
        L.oracle_attn_fwd_f32_range.argtypes = [_fp, _fp, _fp, _fp, _fp, i, i, i, i, f]
        L.oracle_attn_bwd_f32.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, i, i, i, f]
        L.oracle_attn_bwd_f32_range.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _fp, i, i, i, i, f]
        L.oracle_attn_delta_f32.argtypes = [_fp, _fp, _fp, ctypes.c_long, i]
        L.oracle_attn_delta_f32.restype = None
        L.oracle_decode_f32.argtypes = [_fp, _fp, _fp, _fp, _ip, i, i, i, i, f]
        L.oracle_attn_fwd_f64.argtypes = [_dp, _dp, _dp, _dp, _dp, i, i, i, d]
        L.oracle_attn_bwd_f64.argtypes = [_dp, _dp, _dp, _dp, _dp, _dp, _dp, i, i, i, d]
        L.oracle_attn_fwd_f32_mt.argtypes = [_fp, _fp, _fp, _fp, _fp, i, i, i, f, i]
        L.oracle_attn_bwd_f32_mt.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _fp, i, i, i, f, i]
        u32p, u8p, u64 = (ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint8),
                          ctypes.c_uint64)
        L.oracle_philox4x32_10.argtypes = [u32p, u32p, u32p]
        L.oracle_philox4x32_10.restype = None
        L.oracle_dropout_threshold.argtypes = [f]
        L.oracle_dropout_threshold.restype = ctypes.c_uint32
        L.oracle_dropout_mask.argtypes = [u8p, i, i, u64, f]
        L.oracle_dropout_mask.restype = None
        L.oracle_attn_fwd_dropout_f32.argtypes = [_fp, _fp, _fp, _fp, _fp, i, i, i, f, f, u64]
        L.oracle_attn_bwd_dropout_f32.argtypes = ([_fp] * 9 + [i, i, i, f, f, u64])
        L.oracle_attn_fwd_dropout_f32_range.argtypes = [_fp] * 5 + [i, i, i, i, f, f, u64]
        L.oracle_attn_bwd_dropout_f32_range.argtypes = [_fp] * 7 + [i, i, i, i, f, f, u64]
        L.oracle_attn_fwd_dropout_f64.argtypes = [_dp, _dp, _dp, _dp, _dp, i, i, i, d, f, u64]
        L.oracle_attn_bwd_dropout_f64.argtypes = [_dp] * 7 + [i, i, i, d, f, u64]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref_lib():
    """The reference's own CPU operators (oracle/_ref), or None when not built."""
    global _ref
    if _ref is None:
        if not ref_available():
            return None
        R = ctypes.CDLL(REF_PATH)
        i, f = ctypes.c_int, ctypes.c_float
        R.ref_attn_fwd_f32.argtypes = [_fp, _fp, _fp, _fp, i, i, i, i, f]
        R.ref_attn_bwd_f32.argtypes = [_fp, _fp, _fp, _fp, _fp, _fp, _fp, i, i, i, i, f]
        R.ref_decode_f32.argtypes = [_fp, _fp, _fp, _fp, _ip, i, i, i, i, f]
        _ref = R
    return _ref


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _c64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def _check(rc, what):
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with code {rc}")


def attn_fwd(q, k, v, scale, threads: int = 1):
    """Causal forward in fp32, reference op order. q,k,v [BH,S,D]. Returns (O, lse)."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    o = np.empty_like(q)
    lse = np.empty((BH, S), np.float32)
    if threads > 1:
        rc = lib().oracle_attn_fwd_f32_mt(_f(o), _f(lse), _f(q), _f(k), _f(v), BH, S, D, scale,
                                          threads)
    else:
        rc = lib().oracle_attn_fwd_f32(_f(o), _f(lse), _f(q), _f(k), _f(v), BH, S, D, scale)
    _check(rc, "attn_fwd")
    return o, lse


def attn_fwd_slices(q, k, v, scale, bh0, bh1):
    """Forward over bh slices [bh0, bh1) only (bounded baseline samples). Returns O slices."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    o = np.zeros_like(q)
    rc = lib().oracle_attn_fwd_f32_range(_f(o), ctypes.cast(None, _fp), _f(q), _f(k), _f(v),
                                         bh0, bh1, S, D, scale)
    _check(rc, "attn_fwd_slices")
    return o[bh0:bh1]


def attn_bwd(dout, q, k, v, scale, out=None, threads: int = 1):
    """Causal backward in fp32, reference op order. Returns (dQ, dK, dV, delta|None)."""
    dout, q, k, v = _c32(dout), _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    delta = None
    if threads > 1:
        rc = lib().oracle_attn_bwd_f32_mt(_f(dq), _f(dk), _f(dv), _f(dout), _f(q), _f(k), _f(v),
                                          BH, S, D, scale, threads)
        _check(rc, "attn_bwd")
        if out is not None:
            delta = attn_delta(dout, out)
        return dq, dk, dv, delta
    if out is not None:
        out = _c32(out)
        delta = np.empty((BH, S), np.float32)
        rc = lib().oracle_attn_bwd_f32(_f(dq), _f(dk), _f(dv), _f(delta), _f(dout), _f(out),
                                       _f(q), _f(k), _f(v), BH, S, D, scale)
    else:
        rc = lib().oracle_attn_bwd_f32(_f(dq), _f(dk), _f(dv), ctypes.cast(None, _fp),
                                       _f(dout), ctypes.cast(None, _fp), _f(q), _f(k), _f(v),
                                       BH, S, D, scale)
    _check(rc, "attn_bwd")
    return dq, dk, dv, delta


def attn_bwd_slices(dout, q, k, v, scale, bh0, bh1):
    dout, q, k, v = _c32(dout), _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    rc = lib().oracle_attn_bwd_f32_range(_f(dq), _f(dk), _f(dv), _f(dout), _f(q), _f(k), _f(v),
                                         bh0, bh1, S, D, scale)
    _check(rc, "attn_bwd_slices")
    return dq[bh0:bh1], dk[bh0:bh1], dv[bh0:bh1]


def attn_delta(dout, out):
    dout, out = _c32(dout), _c32(out)
    D = dout.shape[-1]
    rows = dout.size // D
    delta = np.empty(dout.shape[:-1], np.float32)
    lib().oracle_attn_delta_f32(_f(delta), _f(dout), _f(out), rows, D)
    return delta


def decode(q, k_cache, v_cache, lens, scale):
    """Ragged KV-cache decode, fp32. q [n,H,D]; caches [n,H,max_len,D]; lens [n]."""
    q, k_cache, v_cache = _c32(q), _c32(k_cache), _c32(v_cache)
    lens = np.ascontiguousarray(lens, dtype=np.int32)
    n, H, max_len, D = k_cache.shape
    out = np.empty((n, H, D), np.float32)
    rc = lib().oracle_decode_f32(_f(out), _f(q), _f(k_cache), _f(v_cache),
                                 lens.ctypes.data_as(_ip), n, H, max_len, D, scale)
    _check(rc, "decode")
    return out


def attn_fwd_f64(q, k, v, scale):
    q, k, v = _c64(q), _c64(k), _c64(v)
    BH, S, D = q.shape
    o = np.empty_like(q)
    lse = np.empty((BH, S), np.float64)
    _check(lib().oracle_attn_fwd_f64(_d(o), _d(lse), _d(q), _d(k), _d(v), BH, S, D, scale),
           "attn_fwd_f64")
    return o, lse


def attn_bwd_f64(dout, q, k, v, scale):
    dout, q, k, v = _c64(dout), _c64(q), _c64(k), _c64(v)
    BH, S, D = q.shape
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    _check(lib().oracle_attn_bwd_f64(_d(dq), _d(dk), _d(dv), _d(dout), _d(q), _d(k), _d(v), BH,
                                     S, D, scale), "attn_bwd_f64")
    return dq, dk, dv


# ---- attention-probability dropout (Philox4x32-10 mask; see attn_oracle.h) ----

def philox4x32_10(ctr, key):
    """Philox4x32-10 block: ctr 4 x uint32, key 2 x uint32 -> 4 x uint32."""
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.empty(4, np.uint32)
    u32p = ctypes.POINTER(ctypes.c_uint32)
    lib().oracle_philox4x32_10(c.ctypes.data_as(u32p), k.ctypes.data_as(u32p),
                               out.ctypes.data_as(u32p))
    return out


def dropout_threshold(p):
    return int(lib().oracle_dropout_threshold(p))


def dropout_mask(BH, S, seed, p):
    """Keep bits [BH, S, S] (1 = kept) of the dropout mask for (seed, p)."""
    m = np.empty((BH, S, S), np.uint8)
    lib().oracle_dropout_mask(m.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), BH, S, seed, p)
    return m


def attn_fwd_dropout(q, k, v, scale, p, seed):
    """Causal forward with dropout of the probabilities, fp32. Returns (O, lse)."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    o = np.empty_like(q)
    lse = np.empty((BH, S), np.float32)
    _check(lib().oracle_attn_fwd_dropout_f32(_f(o), _f(lse), _f(q), _f(k), _f(v), BH, S, D,
                                             scale, p, seed), "attn_fwd_dropout")
    return o, lse


def attn_fwd_dropout_slices(q, k, v, scale, p, seed, bh0, bh1):
    """Forward with dropout over bh slices [bh0, bh1) of [BH, S, D] inputs (the mask rows keep
    their global index). Returns O of those slices."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    o = np.zeros_like(q)
    _check(lib().oracle_attn_fwd_dropout_f32_range(_f(o), ctypes.cast(None, _fp), _f(q), _f(k),
                                                   _f(v), bh0, bh1, S, D, scale, p, seed),
           "attn_fwd_dropout_slices")
    return o[bh0:bh1]


def attn_bwd_dropout(dout, q, k, v, scale, p, seed, out=None):
    """Causal backward with dropout, fp32. Returns (dQ, dK, dV, delta|None)."""
    dout, q, k, v = _c32(dout), _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    delta = None
    null = ctypes.cast(None, _fp)
    if out is not None:
        out = _c32(out)
        delta = np.empty((BH, S), np.float32)
    rc = lib().oracle_attn_bwd_dropout_f32(_f(dq), _f(dk), _f(dv),
                                           _f(delta) if delta is not None else null, _f(dout),
                                           _f(out) if out is not None else null, _f(q), _f(k),
                                           _f(v), BH, S, D, scale, p, seed)
    _check(rc, "attn_bwd_dropout")
    return dq, dk, dv, delta


def attn_bwd_dropout_slices(dout, q, k, v, scale, p, seed, bh0, bh1):
    """Backward with dropout over bh slices [bh0, bh1) of [BH, S, D] inputs (the mask rows
    keep their global index). Returns (dQ, dK, dV) of those slices."""
    dout, q, k, v = _c32(dout), _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    _check(lib().oracle_attn_bwd_dropout_f32_range(_f(dq), _f(dk), _f(dv), _f(dout), _f(q), _f(k),
                                                   _f(v), bh0, bh1, S, D, scale, p, seed),
           "attn_bwd_dropout_slices")
    return dq[bh0:bh1], dk[bh0:bh1], dv[bh0:bh1]


def attn_fwd_dropout_f64(q, k, v, scale, p, seed):
    q, k, v = _c64(q), _c64(k), _c64(v)
    BH, S, D = q.shape
    o = np.empty_like(q)
    lse = np.empty((BH, S), np.float64)
    _check(lib().oracle_attn_fwd_dropout_f64(_d(o), _d(lse), _d(q), _d(k), _d(v), BH, S, D,
                                             scale, p, seed), "attn_fwd_dropout_f64")
    return o, lse


def attn_bwd_dropout_f64(dout, q, k, v, scale, p, seed):
    dout, q, k, v = _c64(dout), _c64(q), _c64(k), _c64(v)
    BH, S, D = q.shape
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    _check(lib().oracle_attn_bwd_dropout_f64(_d(dq), _d(dk), _d(dv), _d(dout), _d(q), _d(k),
                                             _d(v), BH, S, D, scale, p, seed),
           "attn_bwd_dropout_f64")
    return dq, dk, dv


# ---- the reference's own operators (oracle/_ref) ----

def ref_attn_fwd(q, k, v, scale, bh0=0, bh1=None):
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref/libref_attn.so is not built")
    q, k, v = _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    bh1 = BH if bh1 is None else bh1
    o = np.zeros_like(q)
    _check(R.ref_attn_fwd_f32(_f(o), _f(q), _f(k), _f(v), bh0, bh1, S, D, scale), "ref fwd")
    return o


def ref_attn_bwd(dout, q, k, v, scale, bh0=0, bh1=None):
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref/libref_attn.so is not built")
    dout, q, k, v = _c32(dout), _c32(q), _c32(k), _c32(v)
    BH, S, D = q.shape
    bh1 = BH if bh1 is None else bh1
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    _check(R.ref_attn_bwd_f32(_f(dq), _f(dk), _f(dv), _f(dout), _f(q), _f(k), _f(v), bh0, bh1,
                              S, D, scale), "ref bwd")
    return dq, dk, dv


def ref_decode(q, k_cache, v_cache, lens, scale):
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref/libref_attn.so is not built")
    q, k_cache, v_cache = _c32(q), _c32(k_cache), _c32(v_cache)
    lens = np.ascontiguousarray(lens, dtype=np.int32)
    n, H, max_len, D = k_cache.shape
    out = np.empty((n, H, D), np.float32)
    _check(R.ref_decode_f32(_f(out), _f(q), _f(k_cache), _f(v_cache), lens.ctypes.data_as(_ip),
                            n, H, max_len, D, scale), "ref decode")
    return out


# ---- the reference's own CPU tensor operators (src/tensor_ops.cpp, C++ linkage) ----

_REF_OPS = {
    "matmul": ("_Z6matmulPfPKfS1_iii", [_fp, _fp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "matmul_tb": ("_Z19matmul_transposed_bPfPKfS1_iii",
                  [_fp, _fp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "layernorm": ("_Z9layernormPfPKfS1_S1_iif",
                  [_fp, _fp, _fp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_float]),
    "gelu": ("_Z4geluPfPKfi", [_fp, _fp, ctypes.c_int]),
    "embedding": ("_Z16embedding_lookupPfPKtPKfii",
                  [_fp, ctypes.POINTER(ctypes.c_uint16), _fp, ctypes.c_int, ctypes.c_int]),
    "add": ("_Z11add_vectorsPfPKfS1_i", [_fp, _fp, _fp, ctypes.c_int]),
}


def ref_op(name):
    """A reference CPU operator from oracle/_ref (raises when not built)."""
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref/libref_attn.so is not built")
    sym, argtypes = _REF_OPS[name]
    fn = getattr(R, sym)
    fn.argtypes = argtypes
    fn.restype = None
    return fn


def ref_layernorm(x, w, b, eps=1e-5):
    x, w, b = _c32(x), _c32(w), _c32(b)
    out = np.empty_like(x)
    ref_op("layernorm")(_f(out), _f(x), _f(w), _f(b), x.shape[0], x.shape[1], eps)
    return out


def ref_gelu(x):
    x = _c32(x)
    out = np.empty_like(x)
    ref_op("gelu")(_f(out), _f(x), x.size)
    return out


def ref_matmul(a, b):
    a, b = _c32(a), _c32(b)
    out = np.empty((a.shape[0], b.shape[1]), np.float32)
    ref_op("matmul")(_f(out), _f(a), _f(b), a.shape[0], a.shape[1], b.shape[1])
    return out


def ref_matmul_tb(a, b):
    a, b = _c32(a), _c32(b)
    out = np.empty((a.shape[0], b.shape[0]), np.float32)
    ref_op("matmul_tb")(_f(out), _f(a), _f(b), a.shape[0], a.shape[1], b.shape[0])
    return out


def ref_gpt2_forward(params, cfg, tokens):
    """Logits [S, V] of one sequence, composed from the reference's own CPU operators in the
    order of model_forward (src/model.cpp:334-475, batch 1); attention is the reference's
    materialized composition (ref_attn_fwd). Bias adds and the head split/merge are index
    work done in numpy."""
    from . import gpt2_oracle

    P = gpt2_oracle.unpack(_c32(params), cfg)
    d, H, L = cfg["d_model"], cfg["n_heads"], cfg["n_layers"]
    dh = d // H
    toks = np.ascontiguousarray(tokens, dtype=np.uint16)
    S = len(toks)
    emb = np.empty((S, d), np.float32)
    ref_op("embedding")(_f(emb), toks.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                        _f(_c32(P["tok_emb"])), S, d)
    x = np.empty_like(emb)
    pos = _c32(P["pos_emb"][:S])
    ref_op("add")(_f(x), _f(emb), _f(pos), S * d)
    scale = np.float32(1.0) / np.sqrt(np.float32(dh))

    def add(a, b):
        a, b = _c32(a), _c32(b)
        out = np.empty_like(a)
        ref_op("add")(_f(out), _f(a), _f(b), a.size)
        return out

    for l in range(L):
        g = lambda nm: P[f"{l}.{nm}"]
        h = ref_layernorm(x, g("ln1_w"), g("ln1_b"))
        q = ref_matmul(h, g("Wq")) + g("bq")
        k = ref_matmul(h, g("Wk")) + g("bk")
        v = ref_matmul(h, g("Wv")) + g("bv")
        split = lambda t: np.ascontiguousarray(t.reshape(S, H, dh).transpose(1, 0, 2))
        a = ref_attn_fwd(split(q), split(k), split(v), float(scale))
        a = np.ascontiguousarray(a.transpose(1, 0, 2).reshape(S, d))
        x = add(x, ref_matmul(a, g("Wo")) + g("bo"))
        h = ref_layernorm(x, g("ln2_w"), g("ln2_b"))
        f = ref_gelu(ref_matmul(h, g("fc1_w")) + g("fc1_b"))
        x = add(x, ref_matmul(f, g("fc2_w")) + g("fc2_b"))
    h = ref_layernorm(x, P["lnf_w"], P["lnf_b"])
    return ref_matmul_tb(h, P["tok_emb"])
