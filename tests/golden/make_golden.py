"""Writes the golden fixtures of the attention path from the reference's OWN CPU operators.

Run in the build container (needs /root/reference to build oracle/_ref):

    make -C oracle ref && python tests/golden/make_golden.py

It loads oracle/_ref/libref_attn.so — /root/reference/src/tensor_ops.cpp and backward.cpp
compiled where they lie, driven by oracle/ref_glue.cpp in the op order of the reference's
materialized attention (src/model.cpp:396-419, :585-615) and decode (src/model.cpp:765-790) —
and stores inputs and outputs as float32 .npz fixtures next to this script:

  cfg1_fwd_bwd.npz    BASELINE config 1: B1 H4 T64 D32, scale 1/sqrt(32): q k v dout -> o dq dk dv
  ragged70_fwd_bwd.npz  S=70 (ragged last tile, the shape of test_backward.cpp:432-480), D=64
  decode_small.npz    4 sequences, H=2, max_len 40, D=32, lens seeded in [1, 40]

The reference has no CPU logsumexp, so no lse is stored; the oracle's lse is pinned by the
closed-form and brute-force checks in tests/test_oracle.py instead.
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from dadgpt_amd import synth  # noqa: E402


def fwd_bwd_case(path, BH, S, D, seed):
    q, k, v, dout = synth.attn_inputs(BH, S, D, seed=seed, with_dout=True)
    scale = np.float32(1.0 / math.sqrt(D))
    o = oracle.ref_attn_fwd(q, k, v, float(scale))
    dq, dk, dv = oracle.ref_attn_bwd(dout, q, k, v, float(scale))
    np.savez_compressed(path, q=q, k=k, v=v, dout=dout, o=o, dq=dq, dk=dk, dv=dv,
                        scale=np.array([scale], np.float32), seed=np.array([seed], np.int64))


def decode_case(path, n, H, max_len, D, seed):
    q, kc, vc, lens = synth.decode_inputs(n, H, max_len, D, seed=seed, bf16=False)
    scale = np.float32(1.0 / math.sqrt(D))
    out = oracle.ref_decode(q, kc, vc, lens, float(scale))
    np.savez_compressed(path, q=q, k_cache=kc, v_cache=vc, lens=lens, out=out,
                        scale=np.array([scale], np.float32), seed=np.array([seed], np.int64))


def main():
    oracle.build(with_ref=True)
    fwd_bwd_case(os.path.join(HERE, "cfg1_fwd_bwd.npz"), 4, 64, 32, synth.BASE_SEED)
    fwd_bwd_case(os.path.join(HERE, "ragged70_fwd_bwd.npz"), 1, 70, 64, synth.BASE_SEED + 70)
    decode_case(os.path.join(HERE, "decode_small.npz"), 4, 2, 40, 32, synth.BASE_SEED + 4)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
