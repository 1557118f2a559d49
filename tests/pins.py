"""Checks that pin an attention implementation without retyping its formula.

Each check takes the implementation as callables and returns (ok, detail):
  fwd(q, k, v, scale) -> (O [BH,S,D], lse [BH,S])
  bwd(dout, q, k, v, scale) -> (dQ, dK, dV)
  dec(q [n,H,D], k_cache, v_cache [n,H,L,D], lens [n], scale) -> out [n,H,D]

They rest on an independent library routine (torch's causal scaled_dot_product_attention and
its autograd, float64 on the CPU), on closed forms (row 0, zero queries, a length-1 cache),
on invariants (causal prefix, normalisation of the logsumexp, the zero column-sum of dK, the
column-sum of dV), and on central finite differences. tests/test_oracle.py applies them to
the C oracle; tests/test_pins_catch_mistakes.py shows each plausible mistake fails one.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from dadgpt_amd import synth


def _max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def sdpa_f64(q, k, v, scale, dout=None):
    """torch.nn.functional.scaled_dot_product_attention(is_causal=True) in float64 on the
    CPU; with dout, also its autograd gradients. Also returns the logsumexp of the causal
    score rows via torch.logsumexp."""
    tq = torch.tensor(np.asarray(q, np.float64), requires_grad=dout is not None)
    tk = torch.tensor(np.asarray(k, np.float64), requires_grad=dout is not None)
    tv = torch.tensor(np.asarray(v, np.float64), requires_grad=dout is not None)
    o = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True, scale=float(scale))
    S = tq.shape[1]
    with torch.no_grad():
        s = torch.matmul(tq, tk.transpose(1, 2).contiguous()) * float(scale)
        s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
        lse = torch.logsumexp(s, dim=-1)
    grads = None
    if dout is not None:
        o.backward(torch.tensor(np.asarray(dout, np.float64)))
        grads = (tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy())
    return o.detach().numpy(), lse.numpy(), grads


# ------------------------------------------------------------------------- forward pins

def check_fwd_library(fwd, BH=3, S=45, D=32, seed=11, tol=1e-5):
    q, k, v = synth.attn_inputs(BH, S, D, seed=seed)
    scale = 1.0 / np.sqrt(D)
    o, lse = fwd(q, k, v, scale)
    ro, rl, _ = sdpa_f64(q, k, v, scale)
    e_o, e_l = _max_abs(o, ro), _max_abs(lse, rl)
    return e_o <= tol and e_l <= tol, f"O err {e_o:.2e}, lse err {e_l:.2e} (tol {tol})"


def check_fwd_row0(fwd, BH=2, S=20, D=32, seed=12):
    """Row 0 sees only key 0: O_0 = V_0 and lse_0 = scale * q_0 . k_0."""
    q, k, v = synth.attn_inputs(BH, S, D, seed=seed)
    scale = 1.0 / np.sqrt(D)
    o, lse = fwd(q, k, v, scale)
    s00 = np.einsum("bd,bd->b", q[:, 0].astype(np.float64), k[:, 0].astype(np.float64)) * scale
    e_o, e_l = _max_abs(o[:, 0], v[:, 0]), _max_abs(lse[:, 0], s00)
    return e_o <= 1e-6 and e_l <= 1e-5, f"row0 O err {e_o:.2e}, lse err {e_l:.2e}"


def check_fwd_zero_q(fwd, BH=2, S=33, D=32, seed=13):
    """Q = 0 makes every visible score equal: O_i = mean(V_0..i), lse_i = ln(i+1)."""
    _, k, v = synth.attn_inputs(BH, S, D, seed=seed)
    q = np.zeros_like(k)
    o, lse = fwd(q, k, v, 1.0 / np.sqrt(D))
    mean = np.cumsum(v.astype(np.float64), axis=1) / np.arange(1, S + 1)[None, :, None]
    e_o = _max_abs(o, mean)
    e_l = _max_abs(lse, np.log(np.arange(1, S + 1))[None, :].repeat(BH, 0))
    return e_o <= 1e-5 and e_l <= 1e-5, f"zero-Q O err {e_o:.2e}, lse err {e_l:.2e}"


def check_fwd_prefix(fwd, BH=2, S=40, D=32, seed=14, cut=17):
    """Causality: changing K, V rows after `cut` leaves O rows 0..cut unchanged."""
    q, k, v = synth.attn_inputs(BH, S, D, seed=seed)
    scale = 1.0 / np.sqrt(D)
    o1, l1 = fwd(q, k, v, scale)
    k2, v2 = k.copy(), v.copy()
    k2[:, cut + 1:] = synth.normal(k2[:, cut + 1:].shape, seed + 1000)
    v2[:, cut + 1:] = synth.normal(v2[:, cut + 1:].shape, seed + 2000)
    o2, l2 = fwd(q, k2, v2, scale)
    e = max(_max_abs(o1[:, :cut + 1], o2[:, :cut + 1]), _max_abs(l1[:, :cut + 1], l2[:, :cut + 1]))
    changed = _max_abs(o1[:, cut + 1:], o2[:, cut + 1:])
    return e <= 1e-6 and changed > 1e-3, f"prefix diff {e:.2e}, suffix diff {changed:.2e}"


def check_fwd_lse_normalises(fwd, BH=2, S=30, D=32, seed=15):
    """sum_{j<=i} exp(scale q_i.k_j - lse_i) = 1 for every row."""
    q, k, v = synth.attn_inputs(BH, S, D, seed=seed)
    scale = 1.0 / np.sqrt(D)
    _, lse = fwd(q, k, v, scale)
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) * scale
    mask = np.tril(np.ones((S, S), bool))
    tot = np.where(mask[None], np.exp(s - np.asarray(lse, np.float64)[:, :, None]), 0.0).sum(-1)
    e = float(np.max(np.abs(tot - 1.0)))
    return e <= 1e-5, f"row-sum of exp(s - lse) off by {e:.2e}"


FWD_CHECKS = (check_fwd_library, check_fwd_row0, check_fwd_zero_q, check_fwd_prefix,
              check_fwd_lse_normalises)


# ------------------------------------------------------------------------ backward pins

def check_bwd_library(bwd, BH=2, S=37, D=32, seed=21, tol=1e-4):
    q, k, v, g = synth.attn_inputs(BH, S, D, seed=seed, with_dout=True)
    scale = 1.0 / np.sqrt(D)
    dq, dk, dv = bwd(g, q, k, v, scale)
    _, _, (rq, rk, rv) = sdpa_f64(q, k, v, scale, dout=g)
    e = (_max_abs(dq, rq), _max_abs(dk, rk), _max_abs(dv, rv))
    return max(e) <= tol, "dQ/dK/dV err " + ", ".join(f"{x:.2e}" for x in e)


def check_bwd_sums(bwd, BH=2, S=29, D=32, seed=22):
    """Softmax shift invariance: sum_j dK_j = 0. P rows sum to 1: sum_j dV_j = sum_i dO_i."""
    q, k, v, g = synth.attn_inputs(BH, S, D, seed=seed, with_dout=True)
    dq, dk, dv = bwd(g, q, k, v, 1.0 / np.sqrt(D))
    e_k = float(np.max(np.abs(np.asarray(dk, np.float64).sum(1))))
    e_v = _max_abs(np.asarray(dv, np.float64).sum(1), g.astype(np.float64).sum(1))
    return e_k <= 1e-4 and e_v <= 1e-4, f"|sum dK| {e_k:.2e}, sum dV err {e_v:.2e}"


def check_bwd_fd(fwd64, bwd64, BH=1, S=6, D=4, seed=23, h=1e-6):
    """Central finite differences of L = sum(O * dO) against the analytic gradients."""
    q, k, v, g = (x.astype(np.float64) for x in
                  synth.attn_inputs(BH, S, D, seed=seed, with_dout=True))
    scale = 0.7
    dq, dk, dv = bwd64(g, q, k, v, scale)
    worst = 0.0
    for which, grad in ((0, dq), (1, dk), (2, dv)):
        for idx in np.ndindex(q.shape):
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += h
            lp = float(np.sum(fwd64(*args, scale)[0] * g))
            args[which][idx] -= 2 * h
            lm = float(np.sum(fwd64(*args, scale)[0] * g))
            worst = max(worst, abs((lp - lm) / (2 * h) - float(grad[idx])))
    return worst <= 1e-6, f"finite-difference err {worst:.2e}"


BWD_CHECKS = (check_bwd_library, check_bwd_sums)


# -------------------------------------------------------------------------- decode pins

def check_dec_len1(dec, seed=31):
    """A one-row cache returns its V row."""
    q, kc, vc, _ = synth.decode_inputs(3, 2, 8, 32, seed=seed, bf16=False)
    lens = np.ones(3, np.int32)
    out = dec(q, kc, vc, lens, 1.0 / np.sqrt(32))
    e = _max_abs(out, vc[:, :, 0])
    return e <= 1e-6, f"len-1 err {e:.2e}"


def check_dec_matches_causal_row(dec, fwd, seed=32, S=23, D=32):
    """Decoding query t over cache rows 0..t equals row t of the causal forward."""
    q, k, v = synth.attn_inputs(2, S, D, seed=seed)
    scale = 1.0 / np.sqrt(D)
    o, _ = fwd(q, k, v, scale)
    worst = 0.0
    for t in (0, 5, S - 1):
        kc = np.zeros((1, 2, S, D), np.float32)
        vc = np.zeros((1, 2, S, D), np.float32)
        kc[0], vc[0] = k, v
        out = dec(q[None, :, t], kc, vc, np.array([t + 1], np.int32), scale)
        worst = max(worst, _max_abs(out[0], o[:, t]))
    return worst <= 1e-5, f"decode vs causal row err {worst:.2e}"


def check_dec_library(dec, seed=33):
    q, kc, vc, lens = synth.decode_inputs(4, 3, 50, 32, seed=seed, bf16=False)
    scale = 1.0 / np.sqrt(32)
    out = dec(q, kc, vc, lens, scale)
    worst = 0.0
    for s in range(4):
        L = int(lens[s])
        # one query over L keys = the last row of a causal problem with the query at L-1
        qq = np.zeros((3, L, 32))
        qq[:, L - 1] = q[s]
        ro, _, _ = sdpa_f64(qq, kc[s][:, :L], vc[s][:, :L], scale)
        worst = max(worst, _max_abs(out[s], ro[:, L - 1]))
    return worst <= 1e-5, f"decode vs library err {worst:.2e}"


DEC_CHECKS = (check_dec_len1, check_dec_library)


# ------------------------------------------------------------------------- dropout pins
# Implementations with attention-probability dropout take (p, seed) after the scale:
#   fwd_d(q, k, v, scale, p, seed) -> (O, lse); bwd_d(dout, q, k, v, scale, p, seed) -> grads
# and keep(BH, S, seed, p) -> keep bits [BH, S, S] (the mask definition, pinned separately by
# the Philox known-answer vectors). The undropped fwd/bwd are the pinned ones above.

def _drop_reference_f64(q, k, v, scale, keep, p, dout=None):
    """torch float64 on the CPU: O = (causal softmax(QK^T * scale) * keep / (1-p)) V, and with
    dout its autograd gradients (the mask is a constant)."""
    req = dout is not None
    tq, tk, tv = (torch.tensor(np.asarray(x, np.float64), requires_grad=req) for x in (q, k, v))
    S = tq.shape[1]
    s = torch.matmul(tq, tk.transpose(1, 2).contiguous()) * float(scale)
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    pr = torch.softmax(s, dim=-1) * torch.tensor(keep, dtype=torch.float64) / (1.0 - float(p))
    o = torch.matmul(pr, tv)
    grads = None
    if req:
        o.backward(torch.tensor(np.asarray(dout, np.float64)))
        grads = (tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy())
    return o.detach().numpy(), grads


def check_drop_p0_identity(fwd_d, bwd_d, fwd, bwd, BH=2, S=37, D=32, seed=41):
    """p = 0 keeps everything with factor 1: the undropped results."""
    q, k, v, g = synth.attn_inputs(BH, S, D, seed=seed, with_dout=True)
    scale = 1.0 / np.sqrt(D)
    (o, l), (ro, rl) = fwd_d(q, k, v, scale, 0.0, 7), fwd(q, k, v, scale)
    e = [_max_abs(o, ro), _max_abs(l, rl)]
    e += [_max_abs(a, b) for a, b in zip(bwd_d(g, q, k, v, scale, 0.0, 7), bwd(g, q, k, v, scale))]
    return max(e) <= 1e-6, "p=0 vs undropped err " + ", ".join(f"{x:.2e}" for x in e)


def check_drop_lse_undropped(fwd_d, fwd, BH=2, S=40, D=32, seed=42):
    """The saved logsumexp is that of the undropped scores (the backward recomputes P)."""
    q, k, v = synth.attn_inputs(BH, S, D, seed=seed)
    scale = 1.0 / np.sqrt(D)
    e = _max_abs(fwd_d(q, k, v, scale, 0.4, 3)[1], fwd(q, k, v, scale)[1])
    return e <= 1e-5, f"lse with dropout vs without err {e:.2e}"


def check_drop_library(fwd_d, keep, BH=2, S=45, D=32, seed=43, p=0.3, dseed=1234):
    q, k, v = synth.attn_inputs(BH, S, D, seed=seed)
    scale = 1.0 / np.sqrt(D)
    ro, _ = _drop_reference_f64(q, k, v, scale, keep(BH, S, dseed, p), p)
    e = _max_abs(fwd_d(q, k, v, scale, p, dseed)[0], ro)
    return e <= 1e-5, f"O with dropout vs library err {e:.2e}"


def check_drop_bwd_library(bwd_d, keep, BH=2, S=33, D=32, seed=44, p=0.3, dseed=99):
    q, k, v, g = synth.attn_inputs(BH, S, D, seed=seed, with_dout=True)
    scale = 1.0 / np.sqrt(D)
    _, ref = _drop_reference_f64(q, k, v, scale, keep(BH, S, dseed, p), p, dout=g)
    e = [_max_abs(a, b) for a, b in zip(bwd_d(g, q, k, v, scale, p, dseed), ref)]
    return max(e) <= 1e-4, "dQ/dK/dV with dropout err " + ", ".join(f"{x:.2e}" for x in e)


def check_drop_unbiased(fwd_d, fwd, BH=1, S=24, D=16, seed=45, p=0.25, n=300):
    """E[keep / (1-p)] = 1 (p = 0.25 is exactly representable as a 16-bit threshold), so the
    mean output over seeds tends to the undropped output: within 6 standard errors."""
    q, k, v = synth.attn_inputs(BH, S, D, seed=seed)
    scale = 1.0 / np.sqrt(D)
    outs = np.stack([np.asarray(fwd_d(q, k, v, scale, p, 1000 + i)[0], np.float64)
                     for i in range(n)])
    ro = np.asarray(fwd(q, k, v, scale)[0], np.float64)
    se = outs.std(0) / np.sqrt(n)
    z = np.abs(outs.mean(0) - ro) / np.maximum(se, 1e-12)
    return float(z.max()) <= 6.0, f"max |mean - undropped| / std.err {float(z.max()):.2f}"


def check_drop_bwd_fd(fwd64_d, bwd64_d, BH=1, S=6, D=4, seed=46, p=0.3, dseed=5, h=1e-6):
    """Central finite differences of L = sum(O * dO) at a fixed mask."""
    q, k, v, g = (x.astype(np.float64) for x in
                  synth.attn_inputs(BH, S, D, seed=seed, with_dout=True))
    scale = 0.7
    grads = bwd64_d(g, q, k, v, scale, p, dseed)
    worst = 0.0
    for which, grad in enumerate(grads):
        for idx in np.ndindex(q.shape):
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += h
            lp = float(np.sum(fwd64_d(*args, scale, p, dseed)[0] * g))
            args[which][idx] -= 2 * h
            lm = float(np.sum(fwd64_d(*args, scale, p, dseed)[0] * g))
            worst = max(worst, abs((lp - lm) / (2 * h) - float(grad[idx])))
    return worst <= 1e-6, f"finite-difference err {worst:.2e}"
