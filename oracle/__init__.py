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
