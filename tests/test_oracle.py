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


# ---- attention-probability dropout ----

# Published known-answer vectors of Philox4x32-10 (Random123's kat_vectors, "philox4x32 10"
# lines): (counter, key) -> output.
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,expect", PHILOX_KAT)
def test_philox_known_answers(ctr, key, expect):
    assert [int(x) for x in oracle.philox4x32_10(ctr, key)] == list(expect)


def test_dropout_mask_definition():
    """Keep bit of (row, j) = 16-bit half j%2 (low first) of word (j%8)/2 of Philox at counter
    {row lo, row hi, j/8, 0}, key {seed lo, seed hi}, compared as a 16-bit uniform;
    spot-checked against the block function itself."""
    seed, p, BH, S = 0x1234_5678_9ABC_DEF0, 0.3, 3, 37
    m = oracle.dropout_mask(BH, S, seed, p)
    thr = oracle.dropout_threshold(p)
    assert thr == int(np.ceil(np.float32(p) * 2.0 ** 16))
    rng = np.random.default_rng(0)
    for _ in range(50):
        bh, i, j = int(rng.integers(BH)), int(rng.integers(S)), int(rng.integers(S))
        row = bh * S + i
        w = oracle.philox4x32_10((row & 0xFFFFFFFF, row >> 32, j >> 3, 0),
                                 (seed & 0xFFFFFFFF, seed >> 32))
        u = (int(w[(j & 7) >> 1]) >> (16 * (j & 1))) & 0xFFFF
        assert m[bh, i, j] == int(u >= thr)


@pytest.mark.parametrize("p", [0.0, 0.1, 0.5, 0.9])
def test_dropout_mask_rate(p):
    m = oracle.dropout_mask(8, 256, 77, p)
    keep = 1.0 - oracle.dropout_threshold(p) / 2.0 ** 16
    n = m.size
    sigma = np.sqrt(max(keep * (1 - keep), 1e-12) / n)
    assert abs(m.mean() - keep) <= 5 * sigma + 1e-12
    if p == 0.0:
        assert m.all()
    # rows and columns are not correlated with position: halves agree to 5 sigma
    assert abs(m[:, :, :128].mean() - m[:, :, 128:].mean()) <= 10 * sigma + 1e-12


def _fwd_d32(q, k, v, scale, p, seed):
    return oracle.attn_fwd_dropout(q, k, v, float(scale), p, seed)


def _bwd_d32(g, q, k, v, scale, p, seed):
    return oracle.attn_bwd_dropout(g, q, k, v, float(scale), p, seed)[:3]


def test_oracle_dropout_pins():
    for ok, detail in (
            pins.check_drop_p0_identity(_fwd_d32, _bwd_d32, _fwd32, _bwd32),
            pins.check_drop_lse_undropped(_fwd_d32, _fwd32),
            pins.check_drop_library(_fwd_d32, oracle.dropout_mask),
            pins.check_drop_bwd_library(_bwd_d32, oracle.dropout_mask),
            pins.check_drop_unbiased(_fwd_d32, _fwd32)):
        assert ok, detail


def test_oracle_dropout_p0_is_bitwise_undropped():
    q, k, v, g = synth.attn_inputs(3, 50, 32, seed=8, with_dout=True)
    o, lse = oracle.attn_fwd(q, k, v, 0.17)
    od, ld = oracle.attn_fwd_dropout(q, k, v, 0.17, 0.0, 11)
    assert np.array_equal(o, od) and np.array_equal(lse, ld)
    a = oracle.attn_bwd(g, q, k, v, 0.17, out=o)
    b = oracle.attn_bwd_dropout(g, q, k, v, 0.17, 0.0, 11, out=o)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_oracle_dropout_f64_finite_differences_and_twin():
    ok, detail = pins.check_drop_bwd_fd(oracle.attn_fwd_dropout_f64, oracle.attn_bwd_dropout_f64)
    assert ok, detail
    q, k, v, g = synth.attn_inputs(3, 48, 32, seed=9, with_dout=True)
    s = 1 / np.sqrt(32)
    o, lse = oracle.attn_fwd_dropout(q, k, v, s, 0.2, 21)
    o64, l64 = oracle.attn_fwd_dropout_f64(q, k, v, s, 0.2, 21)
    assert np.max(np.abs(o - o64)) < 1e-5 and np.max(np.abs(lse - l64)) < 1e-5
    for a, b in zip(oracle.attn_bwd_dropout(g, q, k, v, s, 0.2, 21)[:3],
                    oracle.attn_bwd_dropout_f64(g, q, k, v, s, 0.2, 21)):
        assert np.max(np.abs(a - b)) < 1e-5


def test_oracle_dropout_rejects_bad_rate():
    q, k, v = synth.attn_inputs(1, 8, 32, seed=1)
    for p in (1.0, -0.1, float("nan")):
        with pytest.raises(RuntimeError):
            oracle.attn_fwd_dropout(q, k, v, 0.1, p, 1)


def test_dropout_slice_ranges_equal_full():
    """The slice-range forward and backward with dropout keep each slice's global mask rows:
    they equal the corresponding slices of the full computation exactly."""
    BH, S, D, p, seed = 4, 45, 16, 0.3, 99
    q, k, v, g = synth.attn_inputs(BH, S, D, seed=5, with_dout=True)
    o_full = oracle.attn_fwd_dropout(q, k, v, 0.25, p, seed)[0]
    grads = oracle.attn_bwd_dropout(g, q, k, v, 0.25, p, seed)[:3]
    o_part = oracle.attn_fwd_dropout_slices(q, k, v, 0.25, p, seed, 1, 3)
    g_part = oracle.attn_bwd_dropout_slices(g, q, k, v, 0.25, p, seed, 1, 3)
    assert np.array_equal(o_full[1:3], o_part)
    for a, b in zip(grads, g_part):
        assert np.array_equal(a[1:3], b)
