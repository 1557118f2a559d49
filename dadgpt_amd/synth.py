"""Seeded synthetic inputs, bit-identical on every machine.

splitmix64 (Steele, Lea & Flood, "Fast splittable pseudorandom number generators",
OOPSLA 2014) gives the uniform stream; Box–Muller turns pairs of uniforms into N(0,1) in
float64, rounded once to float32. ``bf16_round`` is IEEE round-to-nearest-even to bfloat16,
returned as float32 values (exactly representable) or as raw uint16 bits.

Tensor seeds: ``seed ^ tensor_id`` per tensor, so Q, K, V, dO of one config never share a
stream.
"""
from __future__ import annotations

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
BASE_SEED = 0xDAD6B7

TENSOR_ID = {"q": 1, "k": 2, "v": 3, "dout": 4, "lens": 5, "kcache": 6, "vcache": 7}


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of splitmix64 started at state ``seed``."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + np.arange(1, n + 1, dtype=np.uint64) * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, n: int) -> np.ndarray:
    """n doubles in (0, 1]: the top 53 bits of each output, plus one ulp."""
    z = splitmix64(seed, n)
    return ((z >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)


def normal(shape, seed: int) -> np.ndarray:
    """N(0,1) float32 of the given shape (Box–Muller over pairs of uniforms)."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = uniform01(seed, 2 * m)
    r = np.sqrt(-2.0 * np.log(u[0::2]))
    t = 2.0 * np.pi * u[1::2]
    z = np.empty(2 * m, np.float64)
    z[0::2] = r * np.cos(t)
    z[1::2] = r * np.sin(t)
    return z[:n].astype(np.float32).reshape(shape)


def uniform_int(lo: int, hi: int, n: int, seed: int) -> np.ndarray:
    """n integers uniform on [lo, hi] inclusive."""
    z = splitmix64(seed, n)
    span = np.uint64(hi - lo + 1)
    return (z % span).astype(np.int64) + lo


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even (NaN stays NaN)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounding = ((u >> np.uint32(16)) & np.uint32(1)) + np.uint32(0x7FFF)
    with np.errstate(over="ignore"):
        out = ((u + rounding) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.uint16(0x7FC0)
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(
        np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16, as float32."""
    return bf16_to_f32(bf16_bits(x))


def attn_inputs(BH: int, S: int, D: int, seed: int = BASE_SEED, with_dout: bool = False,
                bf16: bool = False):
    """Q, K, V (and dO) [BH,S,D] float32, i.i.d. N(0,1); bf16-rounded when ``bf16``."""
    names = ["q", "k", "v"] + (["dout"] if with_dout else [])
    out = []
    for nm in names:
        x = normal((BH, S, D), seed ^ TENSOR_ID[nm])
        out.append(bf16_round(x) if bf16 else x)
    return out


def decode_inputs(n_seq: int, H: int, max_len: int, D: int, seed: int = BASE_SEED,
                  bf16: bool = True, min_len: int = 1):
    """q [n,H,D], k/v caches [n,H,max_len,D] (every row filled; a kernel reads only the first
    lens[s] rows of sequence s), lens ~ U[min_len,max_len]."""
    lens = uniform_int(min_len, max_len, n_seq, seed ^ TENSOR_ID["lens"]).astype(np.int32)
    q = normal((n_seq, H, D), seed ^ TENSOR_ID["q"])
    kc = normal((n_seq, H, max_len, D), seed ^ TENSOR_ID["kcache"])
    vc = normal((n_seq, H, max_len, D), seed ^ TENSOR_ID["vcache"])
    if bf16:
        q, kc, vc = bf16_round(q), bf16_round(kc), bf16_round(vc)
    return q, kc, vc, lens


# GPT-2 124M generation, 16 prompts of U[16, 256] random tokens, 128 greedy
# tokens each (the parameter arena is seeded with CFG5_SEED too).
CFG5_N, CFG5_NEW, CFG5_SEED = 16, 128, 0x5EED


def cfg5_prompts(vocab_size: int, n: int = CFG5_N, seed: int = CFG5_SEED):
    """The config 5 prompts: lengths U[16, 256], token ids U[0, vocab_size - 1]."""
    lens = uniform_int(16, 256, n, seed ^ 0x10)
    return [list(uniform_int(0, vocab_size - 1, int(L), seed + 0x100 + i))
            for i, L in enumerate(lens)]
