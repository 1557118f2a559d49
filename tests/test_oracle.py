"""CPU tests that pin the oracle (oracle/attn_oracle.c) before it is trusted as the checker.

1. Golden vectors: bit-exact against fixtures written from the reference's own CPU
   operators (tests/golden/make_golden.py, oracle/_ref).
2. Live agreement with oracle/_ref on shapes the fixtures do not cover, when it is built.
3. The pins of tests/pins.py: torch's causal SDPA (float64) and its autograd, closed forms,
   invariants, finite differences, and the decode identities.
"""
import os

import numpy as np
import pytest

import oracle
from dadgpt_amd import synth
from tests import pins


def _load(golden_dir, name):
    return np.load(os.path.join(golden_dir, name))


@pytest.mark.parametrize("name", ["cfg1_fwd_bwd.npz", "ragged70_fwd_bwd.npz"])
def test_oracle_matches_golden_fwd_bwd(golden_dir, name):
    z = _load(golden_dir, name)
    scale = float(z["scale"][0])
    o, lse = oracle.attn_fwd(z["q"], z["k"], z["v"], scale)
    dq, dk, dv, _ = oracle.attn_bwd(z["dout"], z["q"], z["k"], z["v"], scale)
    for got, key in ((o, "o"), (dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert np.array_equal(got, z[key]), f"{name}:{key} differs from the reference's ops"
    assert np.all(np.isfinite(lse))


def test_oracle_matches_golden_decode(golden_dir):
    z = _load(golden_dir, "decode_small.npz")
    out = oracle.decode(z["q"], z["k_cache"], z["v_cache"], z["lens"], float(z["scale"][0]))
    assert np.array_equal(out, z["out"])


def test_golden_inputs_regenerate_from_seed(golden_dir):
    """The fixtures' inputs are the repo PRNG's output for their seed (so GPU tests can
    rebuild them), including the bf16 rounding helpers' identity on fp32."""
    z = _load(golden_dir, "cfg1_fwd_bwd.npz")
    q, k, v, g = synth.attn_inputs(4, 64, 32, seed=int(z["seed"][0]), with_dout=True)
    for a, key in ((q, "q"), (k, "k"), (v, "v"), (g, "dout")):
        assert np.array_equal(a, z[key])


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built here")
@pytest.mark.parametrize("BH,S,D", [(2, 37, 64), (1, 129, 32), (3, 1, 32)])
def test_oracle_matches_reference_build(BH, S, D):
    q, k, v, g = synth.attn_inputs(BH, S, D, seed=900 + S, with_dout=True)
    scale = float(np.float32(1 / np.sqrt(D)))
    o, _ = oracle.attn_fwd(q, k, v, scale)
    assert np.array_equal(o, oracle.ref_attn_fwd(q, k, v, scale))
    got = oracle.attn_bwd(g, q, k, v, scale)[:3]
    want = oracle.ref_attn_bwd(g, q, k, v, scale)
    for a, b in zip(got, want):
        assert np.array_equal(a, b)
    qd, kc, vc, lens = synth.decode_inputs(3, 2, S, D, seed=77, bf16=False)
    assert np.array_equal(oracle.decode(qd, kc, vc, lens, scale),
                          oracle.ref_decode(qd, kc, vc, lens, scale))


def _fwd32(q, k, v, scale):
    return oracle.attn_fwd(q, k, v, float(scale))


def _bwd32(g, q, k, v, scale):
    return oracle.attn_bwd(g, q, k, v, float(scale))[:3]


def _dec32(q, kc, vc, lens, scale):
    return oracle.decode(q, kc, vc, lens, float(scale))


@pytest.mark.parametrize("check", pins.FWD_CHECKS, ids=lambda c: c.__name__)
def test_oracle_forward_pins(check):
    ok, detail = check(_fwd32)
    assert ok, detail


@pytest.mark.parametrize("check", pins.BWD_CHECKS, ids=lambda c: c.__name__)
def test_oracle_backward_pins(check):
    ok, detail = check(_bwd32)
    assert ok, detail


def test_oracle_f64_finite_differences():
    ok, detail = pins.check_bwd_fd(lambda q, k, v, s: oracle.attn_fwd_f64(q, k, v, s),
                                   lambda g, q, k, v, s: oracle.attn_bwd_f64(g, q, k, v, s))
    assert ok, detail


def test_oracle_f64_twin_agrees():
    q, k, v, g = synth.attn_inputs(4, 64, 32, seed=5, with_dout=True)
    scale = 1 / np.sqrt(32)
    o, lse = oracle.attn_fwd(q, k, v, scale)
    o64, l64 = oracle.attn_fwd_f64(q, k, v, scale)
    assert np.max(np.abs(o - o64)) < 1e-5 and np.max(np.abs(lse - l64)) < 1e-5
    d32 = oracle.attn_bwd(g, q, k, v, scale)[:3]
    d64 = oracle.attn_bwd_f64(g, q, k, v, scale)
    for a, b in zip(d32, d64):
        assert np.max(np.abs(a - b)) < 1e-5


@pytest.mark.parametrize("check", pins.DEC_CHECKS, ids=lambda c: c.__name__)
def test_oracle_decode_pins(check):
    ok, detail = check(_dec32)
    assert ok, detail


def test_oracle_decode_matches_causal_row():
    ok, detail = pins.check_dec_matches_causal_row(_dec32, _fwd32)
    assert ok, detail


def test_oracle_delta_is_p_dot_dp():
    """delta_i = sum_d dO_i O_i equals sum_j P_ij dP_ij (the softmax-backward row term)."""
    q, k, v, g = synth.attn_inputs(2, 21, 32, seed=6, with_dout=True)
    scale = 1 / np.sqrt(32)
    o, lse = oracle.attn_fwd(q, k, v, scale)
    delta = oracle.attn_delta(g, o)
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) * scale
    p = np.where(np.tril(np.ones((21, 21), bool))[None], np.exp(s - lse[:, :, None]), 0.0)
    dp = np.einsum("bid,bjd->bij", g.astype(np.float64), v.astype(np.float64))
    assert np.max(np.abs(delta - (p * dp).sum(-1))) < 1e-5


def test_oracle_threaded_equals_serial():
    q, k, v, g = synth.attn_inputs(6, 40, 32, seed=7, with_dout=True)
    o1, l1 = oracle.attn_fwd(q, k, v, 0.2)
    o2, l2 = oracle.attn_fwd(q, k, v, 0.2, threads=3)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)
    a = oracle.attn_bwd(g, q, k, v, 0.2)[:3]
    b = oracle.attn_bwd(g, q, k, v, 0.2, threads=4)[:3]
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
