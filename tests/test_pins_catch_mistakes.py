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


# ---- dropout: a float64 stand-in with the mask of oracle.dropout_mask ----

def _keep(BH, S, seed, p):
    import oracle
    return oracle.dropout_mask(BH, S, seed, p).astype(np.float64)


def _drop_fwd_factory(bug=None):
    def fwd(q, k, v, scale, p, seed):
        q, k, v = (np.asarray(x, np.float64) for x in (q, k, v))
        BH, S, _ = q.shape
        s = np.einsum("bid,bjd->bij", q, k) * scale
        s = np.where(np.tril(np.ones((S, S), bool))[None], s, -np.inf)
        keep = _keep(BH, S, seed, p)
        if bug == "mask_before_softmax":  # drops scores and renormalises over the kept ones
            s = np.where(keep > 0, s, -np.inf)
        m = s.max(-1, keepdims=True)
        e = np.exp(s - m)
        lse = (np.log(e.sum(-1, keepdims=True)) + m)[..., 0]
        pr = e / e.sum(-1, keepdims=True)
        pd = pr * keep / (1.0 if bug == "no_rescale" else 1.0 - p)
        if bug == "lse_of_kept":
            lse = np.log(np.where(keep > 0, e, 0).sum(-1) + 1e-300) + m[..., 0]
        return np.einsum("bij,bjd->bid", pd, v), lse
    return fwd


def _drop_bwd_factory(bug=None):
    def bwd(g, q, k, v, scale, p, seed):
        g, q, k, v = (np.asarray(x, np.float64) for x in (g, q, k, v))
        BH, S, _ = q.shape
        s = np.einsum("bid,bjd->bij", q, k) * scale
        vis = np.tril(np.ones((S, S), bool))[None]
        s = np.where(vis, s, -np.inf)
        pr = np.exp(s - s.max(-1, keepdims=True))
        pr = pr / pr.sum(-1, keepdims=True)
        keep = _keep(BH, S, seed, p)
        f = keep / (1.0 - p)
        pd = pr * f
        dpd = np.einsum("bid,bjd->bij", g, v)
        dv = np.einsum("bij,bid->bjd", pr if bug == "dv_undropped" else pd, g)
        dp = dpd if bug == "dp_unmasked" else dpd * f
        if bug == "dp_scaled_twice":
            dp = dp / (1.0 - p)
        delta = (pr * dp).sum(-1, keepdims=True)
        if bug == "delta_undropped":
            delta = (pr * dpd).sum(-1, keepdims=True)
        ds = pr * (dp - delta) * scale
        return np.einsum("bij,bjd->bid", ds, k), np.einsum("bij,bid->bjd", ds, q), dv
    return bwd


def _drop_fwd_checks(fwd_d):
    return [pins.check_drop_p0_identity(fwd_d, _drop_bwd_factory(), _fwd_factory(),
                                        _bwd_factory()),
            pins.check_drop_lse_undropped(fwd_d, _fwd_factory()),
            pins.check_drop_library(fwd_d, _keep),
            pins.check_drop_unbiased(fwd_d, _fwd_factory(), n=200)]


def _drop_bwd_checks(bwd_d):
    return [pins.check_drop_p0_identity(_drop_fwd_factory(), bwd_d, _fwd_factory(),
                                        _bwd_factory()),
            pins.check_drop_bwd_library(bwd_d, _keep),
            pins.check_drop_bwd_fd(_drop_fwd_factory(), bwd_d)]


def test_unmodified_dropout_stand_in_passes_every_pin():
    for ok, detail in _drop_fwd_checks(_drop_fwd_factory()) + _drop_bwd_checks(
            _drop_bwd_factory()):
        assert ok, detail


@pytest.mark.parametrize("bug", ["mask_before_softmax", "no_rescale", "lse_of_kept"])
def test_dropout_forward_mistake_is_caught(bug):
    with np.errstate(all="ignore"):
        results = _drop_fwd_checks(_drop_fwd_factory(bug))
    assert [r for r in results if not r[0]], f"dropout mistake {bug!r} passed: {results}"


@pytest.mark.parametrize("bug", ["dv_undropped", "dp_unmasked", "dp_scaled_twice",
                                 "delta_undropped"])
def test_dropout_backward_mistake_is_caught(bug):
    with np.errstate(all="ignore"):
        results = _drop_bwd_checks(_drop_bwd_factory(bug))
    assert [r for r in results if not r[0]], f"dropout mistake {bug!r} passed: {results}"
