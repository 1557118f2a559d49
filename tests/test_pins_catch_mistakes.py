"""The pins in tests/pins.py are only worth something if a plausible mistake fails one of
them. This file plants such mistakes in a float64 numpy stand-in for the oracle (on the CPU,
never in the product) and checks that (a) the unmodified stand-in passes every pin and
(b) every planted mistake fails at least one.
"""
import numpy as np
import pytest

from tests import pins


def _fwd_factory(bug=None):
    def fwd(q, k, v, scale):
        q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
        S = q.shape[1]
        s = np.einsum("bid,bjd->bij", q, k)
        if bug == "transposed_scores":
            s = s.transpose(0, 2, 1)
        if bug != "no_scale":
            s = s * scale
        if bug == "double_scale":
            s = s * scale
        vis = np.tril(np.ones((S, S), bool))
        if bug == "no_mask":
            vis = np.ones((S, S), bool)
        if bug == "mask_off_by_one":
            vis = np.tril(np.ones((S, S), bool), 1)
        s = np.where(vis[None], s, -np.inf)
        m = s.max(-1, keepdims=True)
        e = np.exp(s - m)
        tot = e.sum(-1, keepdims=True)
        lse = (np.log(tot) + (0 if bug == "lse_drops_max" else m))[..., 0]
        if bug == "lse_log2":
            lse = (np.log2(tot) + m)[..., 0]
        p = e / tot
        if bug == "softmax_over_queries":
            p = e / e.sum(-2, keepdims=True)
        o = np.einsum("bij,bjd->bid", p, k if bug == "uses_k_for_v" else v)
        return o, lse
    return fwd


def _bwd_factory(bug=None):
    def bwd(g, q, k, v, scale):
        g, q, k, v = (np.asarray(x, np.float64) for x in (g, q, k, v))
        S = q.shape[1]
        s = np.einsum("bid,bjd->bij", q, k) * scale
        vis = np.tril(np.ones((S, S), bool))[None]
        s = np.where(vis, s, -np.inf)
        p = np.exp(s - s.max(-1, keepdims=True))
        p = p / p.sum(-1, keepdims=True)
        dp = np.einsum("bid,bjd->bij", g, v)
        dv = np.einsum("bij,bid->bjd", p, g)
        if bug == "dv_not_transposed":
            dv = np.einsum("bij,bjd->bid", p, g)
        delta = (p * dp).sum(-1, keepdims=True)
        ds = p * (dp - (0 if bug == "drops_delta" else delta))
        if bug == "wrong_sign":
            ds = p * (delta - dp)
        if bug == "no_mask_on_ds":
            ds = np.exp(np.einsum("bid,bjd->bij", q, k) * scale) * 0 + ds + (~vis) * 0.01
        if bug != "no_scale_on_ds":
            ds = ds * scale
        dq = np.einsum("bij,bjd->bid", ds, k)
        dk = np.einsum("bij,bid->bjd", ds, k if bug == "dk_uses_k" else q)
        if bug == "dq_uses_q":
            dq = np.einsum("bij,bjd->bid", ds, q)
        return dq, dk, dv
    return bwd


def _dec_factory(bug=None):
    def dec(q, kc, vc, lens, scale):
        out = np.zeros(q.shape, np.float64)
        for s in range(q.shape[0]):
            L = int(lens[s]) + (1 if bug == "len_plus_one" else 0)
            L = max(1, L - (1 if bug == "len_minus_one" else 0))
            sc = np.einsum("hd,hjd->hj", q[s].astype(np.float64), kc[s, :, :L].astype(np.float64))
            if bug != "no_scale":
                sc = sc * scale
            e = np.exp(sc - sc.max(-1, keepdims=True))
            p = e / e.sum(-1, keepdims=True)
            out[s] = np.einsum("hj,hjd->hd", p, (kc if bug == "uses_k_for_v" else vc)[s, :, :L])
        return out
    return dec


def _fails_some(checks, *impl):
    results = [c(*impl) for c in checks]
    return [r for r in results if not r[0]], results


def test_unmodified_stand_in_passes_every_pin():
    fwd, bwd, dec = _fwd_factory(), _bwd_factory(), _dec_factory()
    for c in pins.FWD_CHECKS:
        ok, detail = c(fwd)
        assert ok, (c.__name__, detail)
    for c in pins.BWD_CHECKS:
        ok, detail = c(bwd)
        assert ok, (c.__name__, detail)
    ok, detail = pins.check_bwd_fd(fwd, bwd)
    assert ok, detail
    for c in pins.DEC_CHECKS:
        ok, detail = c(dec)
        assert ok, (c.__name__, detail)
    ok, detail = pins.check_dec_matches_causal_row(dec, fwd)
    assert ok, detail


@pytest.mark.parametrize("bug", ["transposed_scores", "no_scale", "double_scale", "no_mask",
                                 "mask_off_by_one", "lse_drops_max", "lse_log2",
                                 "softmax_over_queries", "uses_k_for_v"])
def test_forward_mistake_is_caught(bug):
    with np.errstate(all="ignore"):
        failed, results = _fails_some(pins.FWD_CHECKS, _fwd_factory(bug))
    assert failed, f"planted forward mistake {bug!r} passed every pin: {results}"


@pytest.mark.parametrize("bug", ["dv_not_transposed", "drops_delta", "wrong_sign",
                                 "no_mask_on_ds", "no_scale_on_ds", "dk_uses_k", "dq_uses_q"])
def test_backward_mistake_is_caught(bug):
    with np.errstate(all="ignore"):
        failed, results = _fails_some(pins.BWD_CHECKS, _bwd_factory(bug))
        fd_ok, fd_detail = pins.check_bwd_fd(_fwd_factory(), _bwd_factory(bug))
    assert failed or not fd_ok, f"planted backward mistake {bug!r} passed: {results} {fd_detail}"


@pytest.mark.parametrize("bug", ["len_plus_one", "len_minus_one", "no_scale", "uses_k_for_v"])
def test_decode_mistake_is_caught(bug):
    with np.errstate(all="ignore"):
        failed, results = _fails_some(pins.DEC_CHECKS, _dec_factory(bug))
    assert failed, f"planted decode mistake {bug!r} passed every pin: {results}"
