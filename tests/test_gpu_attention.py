"""GPU parity tests of the HIP attention kernels, through the C ABI, against the CPU oracle.

Tolerances (from the path's specification):
  fp32 kernels             max-abs <= 1e-5 against the fp32 CPU path (O, lse, dQ, dK, dV)
  bf16 forward             O max-abs <= 2e-2 against the fp32 CPU path on the same
                           bf16-rounded inputs; lse <= 1e-3
  bf16 backward            dQ, dK, dV max-abs <= 5e-2
  bf16 decode              max-abs <= 2e-2; fp32 decode <= 1e-5
Full-size configurations are checked against the oracle on sampled (b,h) slices and through
size-independent properties on every slice (row 0, causal prefix, column sums of dK and dV,
bitwise repeatability).
"""
import ctypes
import math
import os

import numpy as np
import pytest
import torch

import oracle
from dadgpt_amd import attention as A
from dadgpt_amd import synth

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_O = 2e-2
TOL_LSE = 1e-3
TOL_GRAD = 5e-2
TOL_DEC = 2e-2


def case(msg):
    print(f"[case] {msg}", flush=True)


def dev(x, dtype):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to("cuda").to(dtype)


def host(t):
    return t.float().cpu().numpy()


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def scale_of(D):
    return float(np.float32(1.0 / math.sqrt(D)))


# ----------------------------------------------------------------------------- fp32 path

@pytest.mark.parametrize("name", ["cfg1_fwd_bwd.npz", "ragged70_fwd_bwd.npz"])
def test_fp32_forward_backward_golden(gpu, golden_dir, name):
    z = np.load(os.path.join(golden_dir, name))
    BH, S, D = z["q"].shape
    case(f"fp32 golden {name} BH={BH} S={S} D={D}")
    scale = float(z["scale"][0])
    q, k, v, g = (dev(z[n], torch.float32) for n in ("q", "k", "v", "dout"))
    out, lse = A.attention_forward(q, k, v, scale)
    dq, dk, dv, delta = A.attention_backward(g, out, lse, q, k, v, scale)
    torch.cuda.synchronize()
    _, lse_ref = oracle.attn_fwd(z["q"], z["k"], z["v"], scale)
    assert max_abs(host(out), z["o"]) <= TOL_F32
    assert max_abs(host(lse), lse_ref) <= TOL_F32
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert max_abs(host(got), z[key]) <= TOL_F32, key
    assert max_abs(host(delta), oracle.attn_delta(z["dout"], host(out))) <= TOL_F32


def test_fp32_reference_named_symbols(gpu):
    """The C++-linkage wrappers with the reference's names run the same kernels."""
    case("fp32 via gpu_flash_attention_forward/backward symbols")
    BH, S, D = 3, 100, 64
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=41, with_dout=True)
    q, k, v, g = (dev(x, torch.float32) for x in (qn, kn, vn, gn))
    scale = scale_of(D)
    out = torch.empty_like(q)
    lse = torch.empty(BH, S, device="cuda")
    L = A.lib()
    fwd = getattr(L, "_Z27gpu_flash_attention_forwardPfS_PKfS1_S1_iiif")
    fwd.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 3 + [ctypes.c_float]
    fwd.restype = None
    torch.cuda.synchronize()
    fwd(out.data_ptr(), lse.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), BH, S, D,
        scale)
    bwd = getattr(L, "_Z28gpu_flash_attention_backwardPfS_S_S_PKfS1_S1_S1_S1_S1_iiif")
    bwd.argtypes = [ctypes.c_void_p] * 10 + [ctypes.c_int] * 3 + [ctypes.c_float]
    bwd.restype = None
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    delta = torch.empty(BH, S, device="cuda")
    bwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), delta.data_ptr(), g.data_ptr(),
        out.data_ptr(), lse.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), BH, S, D,
        scale)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle.attn_fwd(qn, kn, vn, scale)
    dq_r, dk_r, dv_r, _ = oracle.attn_bwd(gn, qn, kn, vn, scale)
    assert max_abs(host(out), o_ref) <= TOL_F32
    assert max_abs(host(lse), l_ref) <= TOL_F32
    for a, b in ((dq, dq_r), (dk, dk_r), (dv, dv_r)):
        assert max_abs(host(a), b) <= TOL_F32


@pytest.mark.parametrize("BH,S,D", [(2, 1024, 64), (4, 257, 32), (1, 1, 64)])
def test_fp32_against_oracle(gpu, BH, S, D):
    case(f"fp32 oracle BH={BH} S={S} D={D}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=50 + S, with_dout=True)
    scale = scale_of(D)
    q, k, v, g = (dev(x, torch.float32) for x in (qn, kn, vn, gn))
    out, lse = A.attention_forward(q, k, v, scale)
    dq, dk, dv, _ = A.attention_backward(g, out, lse, q, k, v, scale)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle.attn_fwd(qn, kn, vn, scale, threads=8)
    assert max_abs(host(out), o_ref) <= TOL_F32
    assert max_abs(host(lse), l_ref) <= TOL_F32
    ref = oracle.attn_bwd(gn, qn, kn, vn, scale, threads=8)[:3]
    for a, b in zip((dq, dk, dv), ref):
        assert max_abs(host(a), b) <= TOL_F32


# ----------------------------------------------------------------------------- bf16 path

SMALL_BF16 = [(1, 1, 64), (2, 70, 64), (3, 129, 64), (1, 64, 64), (2, 300, 32), (1, 65, 32),
              (4, 256, 64), (1, 1000, 64)]


def _sweep_shapes(n=10, seed=2026):
    """Seeded random shapes: BH in [1, 6], S in [2, 600] with a bias to tile edges (multiples
    of 32 and 64, plus or minus one), D in {32, 64}, scale in [0.05, 1/sqrt(D)] (at most the
    model's scale, so gradient magnitudes stay those the tolerances are stated for)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        S = int(rng.integers(2, 601))
        if rng.random() < 0.5:
            S = max(1, int(rng.choice([32, 64])) * int(rng.integers(1, 10)) +
                    int(rng.integers(-1, 2)))
        D = int(rng.choice([32, 64]))
        out.append((int(rng.integers(1, 7)), S, D,
                    float(np.float32(rng.uniform(0.05, 1.0 / math.sqrt(D))))))
    return out


@pytest.mark.parametrize("BH,S,D,scale", _sweep_shapes(n=30))
def test_bf16_and_fp32_random_shapes(gpu, BH, S, D, scale):
    """bf16 and fp32 kernels, forward and backward, on seeded random shapes and scales against
    the oracle at the path's tolerances (the fixed shapes above cover the named edge cases)."""
    case(f"random shape BH={BH} S={S} D={D} scale={scale:.4f}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=900 + S + 7 * BH + D, with_dout=True,
                                       bf16=True)
    o_ref, l_ref = oracle.attn_fwd(qn, kn, vn, scale, threads=8)
    ref = oracle.attn_bwd(gn, qn, kn, vn, scale, threads=8)[:3]
    for dtype, tol_o, tol_l, tol_g in ((torch.bfloat16, TOL_O, TOL_LSE, TOL_GRAD),
                                       (torch.float32, TOL_F32, TOL_F32, TOL_F32)):
        q, k, v, g = (dev(x, dtype) for x in (qn, kn, vn, gn))
        out, lse = A.attention_forward(q, k, v, scale)
        dq, dk, dv, _ = A.attention_backward(g, out, lse, q, k, v, scale)
        torch.cuda.synchronize()
        assert max_abs(host(out), o_ref) <= tol_o, dtype
        assert max_abs(host(lse), l_ref) <= tol_l, dtype
        for a, b, nm in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
            assert max_abs(host(a), b) <= tol_g, (dtype, nm)


@pytest.mark.parametrize("BH,S,D", SMALL_BF16)
def test_bf16_forward_backward_small(gpu, BH, S, D):
    case(f"bf16 small BH={BH} S={S} D={D}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=70 + S + D, with_dout=True, bf16=True)
    scale = scale_of(D)
    q, k, v, g = (dev(x, torch.bfloat16) for x in (qn, kn, vn, gn))
    out, lse = A.attention_forward(q, k, v, scale)
    dq, dk, dv, _ = A.attention_backward(g, out, lse, q, k, v, scale)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle.attn_fwd(qn, kn, vn, scale, threads=8)
    assert max_abs(host(out), o_ref) <= TOL_O
    assert max_abs(host(lse), l_ref) <= TOL_LSE
    ref = oracle.attn_bwd(gn, qn, kn, vn, scale, threads=8)[:3]
    for a, b, nm in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        assert max_abs(host(a), b) <= TOL_GRAD, nm


@pytest.mark.parametrize("scale", [0.0, -0.125, 1.0])
@pytest.mark.parametrize("D", [64, 32])
def test_bf16_scale_zero_negative_large(gpu, scale, D):
    """Zero scale (uniform weights over the causal prefix), a negative scale (applied by
    negating Q) and a large one (sharp rows that move the running maximum often)."""
    BH, S = 2, 200
    case(f"bf16 scale={scale} BH={BH} S={S} D={D}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=90 + D, with_dout=True, bf16=True)
    q, k, v, g = (dev(x, torch.bfloat16) for x in (qn, kn, vn, gn))
    out, lse = A.attention_forward(q, k, v, scale)
    dq, dk, dv, _ = A.attention_backward(g, out, lse, q, k, v, scale)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle.attn_fwd(qn, kn, vn, scale, threads=8)
    assert max_abs(host(out), o_ref) <= TOL_O
    assert max_abs(host(lse), l_ref) <= TOL_LSE
    if scale == 0.0:  # row i is the mean of V_0..V_i; lse = ln(i + 1)
        assert max_abs(host(lse)[0], np.log(np.arange(1, S + 1))) <= TOL_LSE
    # dQ and dK carry the scale factor, and a large scale sharpens P: the bf16 rounding of
    # dS (relative 2^-9) grows with |scale|, so the gradient bound scales with it.
    tol_grad = TOL_GRAD * max(1.0, abs(scale) / scale_of(D))
    ref = oracle.attn_bwd(gn, qn, kn, vn, scale, threads=8)[:3]
    for a, b, nm in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        assert max_abs(host(a), b) <= tol_grad, nm


@pytest.mark.parametrize("scale", [0.0, -0.125, 1.0, 4.0])
@pytest.mark.parametrize("D", [64, 32])
def test_fp32_scale_zero_negative_large(gpu, scale, D):
    """The fp32 kernels' lazy running maximum at the scales that stress it: zero (every weight
    exp(0) = 1), negative, and large ones whose sharp rows move the maximum on many chunks
    (scale 4 with N(0,1) inputs puts score gaps of ~100 natural-log units between keys)."""
    BH, S = 2, 300
    case(f"fp32 scale={scale} BH={BH} S={S} D={D}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=190 + D, with_dout=True)
    q, k, v, g = (dev(x, torch.float32) for x in (qn, kn, vn, gn))
    out, lse = A.attention_forward(q, k, v, scale)
    dq, dk, dv, _ = A.attention_backward(g, out, lse, q, k, v, scale)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle.attn_fwd(qn, kn, vn, scale, threads=8)
    ref = oracle.attn_bwd(gn, qn, kn, vn, scale, threads=8)[:3]
    # The bound is relative to the largest reference value (gradients grow with |scale|), and
    # above the default scale it grows with |scale| / default: the weights exponentiate the
    # scores times the scale, so fp32 rounding in a score moves them that much more (any fp32
    # product reaches 0.7-1.0e-5 of max |O| at |scale| = 4, D = 64: 32x the default).
    tol = TOL_F32 * max(1.0, abs(scale) / scale_of(D))
    assert max_abs(host(out), o_ref) <= tol * max(1.0, np.abs(o_ref).max())
    assert max_abs(host(lse), l_ref) <= tol * max(1.0, np.abs(l_ref).max())
    if scale == 0.0:
        assert max_abs(host(lse)[0], np.log(np.arange(1, S + 1))) <= TOL_F32 * np.log(S)
    for a, b, nm in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        assert max_abs(host(a), b) <= tol * max(1.0, np.abs(b).max()), nm


def torch_reference(q, k, v, scale, dout=None, chunk=16):
    """Materialized fp32 causal attention on the GPU with torch (GEMMs on contiguous
    operands): O, lse and, with dout, dQ/dK/dV plus the two quantities the column-sum bounds
    need. Processes `chunk` (b,h) slices at a time."""
    BH, S, _ = q.shape
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool, device=q.device), 1)
    res = {n: [] for n in ("o", "lse", "dq", "dk", "dv", "sig_dk")}
    for a in range(0, BH, chunk):
        qf, kf, vf = (x[a:a + chunk].float() for x in (q, k, v))
        s = torch.bmm(qf, kf.transpose(1, 2).contiguous()) * scale
        s.masked_fill_(mask, float("-inf"))
        lse = torch.logsumexp(s, -1)
        p = torch.exp(s - lse[..., None])
        o = torch.bmm(p, vf)
        res["o"].append(o)
        res["lse"].append(lse)
        if dout is None:
            continue
        gf = dout[a:a + chunk].float()
        dp = torch.bmm(gf, vf.transpose(1, 2).contiguous())
        delta = (gf * o).sum(-1)
        ds = p * (dp - delta[..., None]) * scale
        res["dq"].append(torch.bmm(ds, kf))
        res["dk"].append(torch.bmm(ds.transpose(1, 2).contiguous(), qf))
        res["dv"].append(torch.bmm(p.transpose(1, 2).contiguous(), gf))
        # sqrt(sum_ij dS_ij^2 Q_id^2) per (slice, d): scale of the bf16 rounding of dS in dK
        res["sig_dk"].append(torch.sqrt(torch.bmm((ds * ds).sum(2).unsqueeze(1), qf * qf)))
        del s, p, dp, ds
    return {n: torch.cat(x).cpu().numpy().astype(np.float64) for n, x in res.items() if x}


def test_bf16_forward_cfg2_full(gpu):
    """B8 H12 T1024 D64 bf16 forward. Every slice against a materialized
    fp32 torch reference on the GPU, three slices against the CPU oracle."""
    BH, S, D = 96, 1024, 64
    case("bf16 cfg2 forward B8 H12 T1024 D64")
    qn, kn, vn = synth.attn_inputs(BH, S, D, seed=synth.BASE_SEED + 2, bf16=True)
    scale = 0.125
    q, k, v = (dev(x, torch.bfloat16) for x in (qn, kn, vn))
    out, lse = A.attention_forward(q, k, v, scale)
    out2, lse2 = A.attention_forward(q, k, v, scale)
    torch.cuda.synchronize()
    o, l = host(out), host(lse)
    assert np.isfinite(o).all() and np.isfinite(l).all()
    assert torch.equal(out, out2) and torch.equal(lse, lse2), "forward not repeatable"
    assert np.array_equal(o[:, 0], vn[:, 0]), "row 0 must equal V row 0"
    ref = torch_reference(q, k, v, scale)
    assert max_abs(o, ref["o"]) <= TOL_O
    assert max_abs(l, ref["lse"]) <= TOL_LSE
    sl = [0, 37, 95]
    o_ref, l_ref = oracle.attn_fwd(qn[sl], kn[sl], vn[sl], scale, threads=8)
    assert max_abs(o[sl], o_ref) <= TOL_O
    assert max_abs(l[sl], l_ref) <= TOL_LSE


# bf16 unit roundoff: 8 significant bits, round to nearest -> relative error <= 2^-8.
U_BF16 = 2.0 ** -8


def test_bf16_forward_backward_cfg3_full(gpu):
    """B16 H12 T1024 D64 bf16 forward + backward from the saved lse.
    Two slices against the CPU oracle; every slice against a materialized fp32 torch
    reference on the GPU; and on every slice the column sums fixed by the softmax:
    sum_j dK_j = 0 and sum_j dV_j = sum_i dO_i."""
    BH, S, D = 192, 1024, 64
    case("bf16 cfg3 fwd+bwd B16 H12 T1024 D64")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=synth.BASE_SEED + 3, with_dout=True,
                                       bf16=True)
    scale = 0.125
    q, k, v, g = (dev(x, torch.bfloat16) for x in (qn, kn, vn, gn))
    out, lse = A.attention_forward(q, k, v, scale)
    dq, dk, dv, delta = A.attention_backward(g, out, lse, q, k, v, scale)
    dq2, dk2, dv2, _ = A.attention_backward(g, out, lse, q, k, v, scale)
    torch.cuda.synchronize()
    assert torch.equal(dq, dq2) and torch.equal(dk, dk2) and torch.equal(dv, dv2), \
        "backward not bitwise repeatable"
    hq, hk, hv, ho = host(dq), host(dk), host(dv), host(out)
    for a in (hq, hk, hv):
        assert np.isfinite(a).all()
    sl = [0, 191]
    ref = oracle.attn_bwd(gn[sl], qn[sl], kn[sl], vn[sl], scale, threads=8)[:3]
    for a, b, nm in zip((hq[sl], hk[sl], hv[sl]), ref, ("dq", "dk", "dv")):
        assert max_abs(a, b) <= TOL_GRAD, nm
    tr = torch_reference(q, k, v, scale, dout=g)
    assert max_abs(ho, tr["o"]) <= TOL_O
    for a, nm in ((hq, "dq"), (hk, "dk"), (hv, "dv")):
        assert max_abs(a, tr[nm]) <= TOL_GRAD, nm
    # Column sums. Round-to-nearest errors are taken as independent, uniform in +-u|x|
    # (standard deviation u|x|/sqrt(3)); the bounds are 6 standard deviations of:
    #  dV: the bf16 rounding of P (sum_j P_ij^2 <= 1 per row) and of the dV outputs;
    #  dK: the bf16 rounding of dS, of the stored O (through delta = dO.O, which is what
    #      makes the rows of dS sum to zero) and of the dK outputs.
    k6 = 6 * U_BF16 / math.sqrt(3)
    g64, o64, q64 = gn.astype(np.float64), ho.astype(np.float64), qn.astype(np.float64)
    err_v = np.abs(hv.astype(np.float64).sum(1) - g64.sum(1))
    bound_v = k6 * (np.sqrt((g64 ** 2).sum(1)) + np.sqrt((hv.astype(np.float64) ** 2).sum(1)))
    assert (err_v <= bound_v + 1e-3).all(), f"dV column sum off by {float(err_v.max()):.3e}"
    err_k = np.abs(hk.astype(np.float64).sum(1))
    row_delta_var = ((g64 * o64) ** 2).sum(-1, keepdims=True)  # [BH,S,1]
    sig_delta = scale * np.sqrt((q64 ** 2 * row_delta_var).sum(1))
    bound_k = k6 * (tr["sig_dk"][:, 0] + sig_delta +
                    np.sqrt((hk.astype(np.float64) ** 2).sum(1)))
    assert (err_k <= bound_k + 1e-3).all(), f"dK column sum off by {float(err_k.max()):.3e}"


def test_bf16_causal_prefix(gpu):
    """Changing K/V rows after a cut leaves O, lse and dQ of earlier rows bitwise equal."""
    BH, S, D, cut = 4, 333, 64, 150
    case("bf16 causal prefix")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=88, with_dout=True, bf16=True)
    k2, v2 = kn.copy(), vn.copy()
    k2[:, cut + 1:] = synth.bf16_round(synth.normal(k2[:, cut + 1:].shape, 5))
    v2[:, cut + 1:] = synth.bf16_round(synth.normal(v2[:, cut + 1:].shape, 6))
    scale = 0.125
    q, g = dev(qn, torch.bfloat16), dev(gn, torch.bfloat16)
    o1, l1 = A.attention_forward(q, dev(kn, torch.bfloat16), dev(vn, torch.bfloat16), scale)
    o2, l2 = A.attention_forward(q, dev(k2, torch.bfloat16), dev(v2, torch.bfloat16), scale)
    torch.cuda.synchronize()
    assert torch.equal(o1[:, :cut + 1], o2[:, :cut + 1])
    assert torch.equal(l1[:, :cut + 1], l2[:, :cut + 1])
    assert not torch.equal(o1[:, cut + 1:], o2[:, cut + 1:])


@pytest.mark.parametrize("S,bad", [(23, [22]), (19, [18]), (2, [1]), (130, [129]),
                                   (70, list(range(40, 50)))])
@pytest.mark.parametrize("D", [64, 32])
def test_forward_rows_independent_of_nan_query_rows(gpu, S, bad, D):
    """A query row's output and logsumexp depend only on its own query and the keys up to it,
    as in the reference's fused kernel (cuda/attention.cu:17-73: one thread per query row):
    NaN query rows (the last row included, which the rows past S of its wave read as well)
    leave every other row bit-identical, in bf16 and fp32. Padded prompt rows of a batched
    prefill hold whatever their buffer held, so the generation path relies on this."""
    case(f"forward rows independent of NaN query rows S={S} D={D} bad={bad[0]}..{bad[-1]}")
    qn, kn, vn = synth.attn_inputs(3, S, D, seed=91, bf16=True)
    q2 = qn.copy()
    q2[1, bad] = np.nan
    ok = np.ones(S, bool)
    ok[bad] = False
    for dtype in (torch.bfloat16, torch.float32):
        k, v = dev(kn, dtype), dev(vn, dtype)
        o1, l1 = A.attention_forward(dev(qn, dtype), k, v, 0.125)
        o2, l2 = A.attention_forward(dev(q2, dtype), k, v, 0.125)
        torch.cuda.synchronize()
        assert torch.equal(o1[:, ok], o2[:, ok]) and torch.equal(l1[:, ok], l2[:, ok]), dtype
        assert torch.equal(o1[0], o2[0]) and torch.equal(o1[2], o2[2])
        assert bool(torch.isnan(o2[1, bad].float()).all())


def test_bf16_errors_raise(gpu):
    case("bf16 error paths")
    q = torch.zeros(2, 16, 48, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(A.AttentionError, match="unsupported d_head 48"):
        A.attention_forward(q, q, q)
    q64 = torch.zeros(2, 16, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(TypeError):
        A.flash_attention_forward_bf16(torch.empty_like(q64).float(),
                                       torch.empty(2, 16, device="cuda"), q64, q64, q64, 2, 16,
                                       64, 0.125)
    with pytest.raises(ValueError):
        A.flash_attention_forward_bf16(torch.empty_like(q64), torch.empty(2, 8, device="cuda"),
                                       q64, q64, q64, 2, 16, 64, 0.125)


# ----------------------------------------------------------------------------- decode

def run_decode(qn, kc, vc, lens, scale, dtype, ws=None):
    n, H, L, D = kc.shape
    q = dev(qn, dtype)
    k_cache, v_cache = dev(kc, dtype), dev(vc, dtype)
    lens_d = torch.from_numpy(np.asarray(lens, np.int32)).cuda()
    out = torch.empty(n, H, D, dtype=dtype, device="cuda")
    ws = A.decode_workspace(n, H, L, D) if ws is None else ws
    A.decode_attention(out, q, k_cache, v_cache, lens_d, n, H, L, D, scale, ws)
    return out, ws


def test_decode_cfg4_full(gpu):
    """32 ragged sequences, H12, D64, bf16 cache, lens ~ U[1,1024]."""
    n, H, L, D = 32, 12, 1024, 64
    case("decode cfg4 bf16 32x12x1024x64")
    qn, kc, vc, lens = synth.decode_inputs(n, H, L, D, seed=synth.BASE_SEED + 4)
    scale = 0.125
    out, ws = run_decode(qn, kc, vc, lens, scale, torch.bfloat16)
    out2, _ = run_decode(qn, kc, vc, lens, scale, torch.bfloat16, ws=ws)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "decode not repeatable"
    ref = oracle.decode(qn, kc, vc, lens, scale)
    assert max_abs(host(out), ref) <= TOL_DEC


def test_decode_fp32_against_oracle(gpu):
    n, H, L, D = 5, 3, 700, 64
    case("decode fp32")
    qn, kc, vc, lens = synth.decode_inputs(n, H, L, D, seed=101, bf16=False)
    lens[0], lens[1] = 1, L
    out, _ = run_decode(qn, kc, vc, lens, 0.125, torch.float32)
    torch.cuda.synchronize()
    assert max_abs(host(out), oracle.decode(qn, kc, vc, lens, 0.125)) <= TOL_F32


@pytest.mark.parametrize("D", [32, 64])
def test_decode_edge_lengths(gpu, D):
    n, H, L = 8, 2, 600
    case(f"decode edge lengths D={D}")
    qn, kc, vc, _ = synth.decode_inputs(n, H, L, D, seed=102 + D)
    lens = np.array([1, 2, 63, 64, 255, 256, 257, 600], np.int32)
    out, ws = run_decode(qn, kc, vc, lens, 0.2, torch.bfloat16)
    torch.cuda.synchronize()
    assert max_abs(host(out), oracle.decode(qn, kc, vc, lens, 0.2)) <= TOL_DEC
    assert np.array_equal(host(out)[0], vc[0, :, 0]), "length 1 must return V row 0"
    # same workspace, different lengths
    lens2 = np.array([600, 1, 300, 512, 513, 7, 64, 65], np.int32)
    out2, _ = run_decode(qn, kc, vc, lens2, 0.2, torch.bfloat16, ws=ws)
    torch.cuda.synchronize()
    assert max_abs(host(out2), oracle.decode(qn, kc, vc, lens2, 0.2)) <= TOL_DEC


def test_decode_length_clamping(gpu):
    n, H, L, D = 3, 2, 100, 64
    case("decode length clamping")
    qn, kc, vc, _ = synth.decode_inputs(n, H, L, D, seed=103)
    out, _ = run_decode(qn, kc, vc, np.array([0, 100, 1000], np.int32), 0.125, torch.bfloat16)
    torch.cuda.synchronize()
    o = host(out)
    assert np.all(o[0] == 0.0), "length 0 gives a zero row"
    ref = oracle.decode(qn[1:], kc[1:], vc[1:], np.array([100, 100], np.int32), 0.125)
    assert max_abs(o[1:], ref) <= TOL_DEC, "lengths beyond max_len clamp to max_len"


def _decode_sweep(n=8, seed=77):
    """Seeded random decode shapes: 1-24 sequences, 1-12 heads, max_len 1-2600 (so 1 to 6
    chunks of a bf16 cache and up to 11 of an fp32 one), d_head 32 or 64, bf16 and fp32 caches
    alternately; at most 400k cache rows (about 100 MB per fp32 cache)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        n_seq, H = int(rng.integers(1, 25)), int(rng.integers(1, 13))
        L = int(rng.integers(1, 2601))
        L = max(1, min(L, 400_000 // (n_seq * H)))
        out.append((n_seq, H, L, int(rng.choice([32, 64])), i % 2 == 0))
    return out


@pytest.mark.parametrize("n,H,L,D,bf", _decode_sweep())
def test_decode_random_shapes(gpu, n, H, L, D, bf):
    """Ragged decode on seeded random shapes against the oracle; the longest and shortest
    lengths (max_len and 1) are always among the sequences."""
    dtype = torch.bfloat16 if bf else torch.float32
    case(f"decode random n={n} H={H} max_len={L} D={D} {dtype}")
    qn, kc, vc, lens = synth.decode_inputs(n, H, L, D, seed=300 + n * H + L, bf16=bf)
    lens[0] = L
    lens[-1] = min(lens[-1], 1) if n > 1 else L
    scale = scale_of(D)
    out, ws = run_decode(qn, kc, vc, lens, scale, dtype)
    torch.cuda.synchronize()
    assert max_abs(host(out), oracle.decode(qn, kc, vc, lens, scale)) <= (TOL_DEC if bf else
                                                                          TOL_F32)


@pytest.mark.parametrize("dtype,L", [(torch.bfloat16, 2500), (torch.float32, 1300)])
def test_decode_split_spans(gpu, dtype, L):
    """Caches longer than one workgroup chunk publish partials that the last chunk merges."""
    n, H, D = 5, 3, 64
    case(f"decode split chunks {dtype} max_len={L}")
    bf = dtype == torch.bfloat16
    qn, kc, vc, lens = synth.decode_inputs(n, H, L, D, seed=105, bf16=bf)
    lens[:4] = [L, 1, 1024, 1025]
    ws = A.decode_workspace(n, H, L, D)
    assert ws is not None
    out, _ = run_decode(qn, kc, vc, lens, 0.125, dtype, ws=ws)
    out2, _ = run_decode(qn, kc, vc, lens, 0.125, dtype, ws=ws)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    assert max_abs(host(out), oracle.decode(qn, kc, vc, lens, 0.125)) <= (TOL_DEC if bf else
                                                                          TOL_F32)


def ws_counters(ws, n, H):
    """The arrival counters at the start of a decode workspace (n*H uint32)."""
    return ws[:4 * n * H].view(torch.int32)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.float32, 64),
                                     (torch.bfloat16, 32)])
def test_decode_workspace_reuse(gpu, dtype, D):
    """One workspace (sized for 6 sequences) across calls with changing lengths and changing
    sequence counts: every call matches the oracle and leaves the arrival counters at zero
    (the last chunk of each cache rearms its counter; partials never land on counters)."""
    n, H, L = 6, 4, 3000
    case(f"decode workspace reuse {dtype} D={D}")
    bf = dtype == torch.bfloat16
    qn, kc, vc, _ = synth.decode_inputs(n, H, L, D, seed=106 + D, bf16=bf)
    ws = A.decode_workspace(n, H, L, D)
    rng = np.random.default_rng(7)
    tol = TOL_DEC if bf else TOL_F32
    for it, m in enumerate([6, 2, 6, 3, 1, 6]):
        lens = rng.integers(0, L + 1, m).astype(np.int32)
        lens[it % m] = L  # always one cache of every chunk
        out, _ = run_decode(qn[:m], kc[:m], vc[:m], lens, 0.125, dtype, ws=ws)
        torch.cuda.synchronize()
        ref = oracle.decode(qn[:m], kc[:m], vc[:m], lens, 0.125)
        assert max_abs(host(out), ref) <= tol, f"call {it} (n_seq {m})"
        assert int(ws_counters(ws, n, H).abs().sum()) == 0, f"counters after call {it}"


def test_decode_matches_forward_rows(gpu):
    """Decoding query t over cache rows 0..t equals row t of the causal forward (GPU vs GPU,
    both bf16)."""
    BH, S, D = 12, 400, 64
    case("decode vs forward rows")
    qn, kn, vn = synth.attn_inputs(BH, S, D, seed=104, bf16=True)
    q, k, v = (dev(x, torch.bfloat16) for x in (qn, kn, vn))
    out, _ = A.attention_forward(q, k, v, 0.125)
    ts = [0, 1, 63, 64, 255, 256, 399]
    qd = np.stack([qn[:, t] for t in ts])  # [len(ts), H=BH, D]
    kc = np.broadcast_to(kn[None], (len(ts), BH, S, D)).copy()
    vc = np.broadcast_to(vn[None], (len(ts), BH, S, D)).copy()
    dec, _ = run_decode(qd, kc, vc, np.array([t + 1 for t in ts], np.int32), 0.125,
                        torch.bfloat16)
    torch.cuda.synchronize()
    o = host(out)
    for i, t in enumerate(ts):
        assert max_abs(host(dec)[i], o[:, t]) <= TOL_DEC, f"row {t}"


@pytest.mark.parametrize("D", [64, 32])
def test_bf16_long_sequence(gpu, D):
    """S = 2048 (twice the configs' length): rows far from their first key exercise the
    running maximum and the fp32 sums over long rows."""
    BH, S = 2, 2048
    case(f"bf16 long sequence BH={BH} S={S} D={D}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=2048 + D, with_dout=True, bf16=True)
    scale = scale_of(D)
    q, k, v, g = (dev(x, torch.bfloat16) for x in (qn, kn, vn, gn))
    out, lse = A.attention_forward(q, k, v, scale)
    dq, dk, dv, _ = A.attention_backward(g, out, lse, q, k, v, scale)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle.attn_fwd(qn, kn, vn, scale, threads=2)
    assert max_abs(host(out), o_ref) <= TOL_O
    assert max_abs(host(lse), l_ref) <= TOL_LSE
    ref = oracle.attn_bwd(gn, qn, kn, vn, scale, threads=2)[:3]
    for a, b, nm in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        assert max_abs(host(a), b) <= TOL_GRAD, nm


@pytest.mark.parametrize("D", [64, 32])
def test_fp32_long_sequence(gpu, D):
    """fp32 at S = 2048: 64 query tiles of 32 rows in dK/dV and key tiles in dQ, 32 of 64 rows
    in the forward, and fp32 sums over rows twice the configs' length. The bound is relative
    to the largest reference value: the gradients are sums over up to 2048 rows."""
    BH, S = 2, 2048
    case(f"fp32 long sequence BH={BH} S={S} D={D}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=4096 + D, with_dout=True)
    scale = scale_of(D)
    q, k, v, g = (dev(x, torch.float32) for x in (qn, kn, vn, gn))
    out, lse = A.attention_forward(q, k, v, scale)
    dq, dk, dv, _ = A.attention_backward(g, out, lse, q, k, v, scale)
    torch.cuda.synchronize()
    o_ref, l_ref = oracle.attn_fwd(qn, kn, vn, scale, threads=8)
    assert max_abs(host(out), o_ref) <= TOL_F32 * max(1.0, np.abs(o_ref).max())
    assert max_abs(host(lse), l_ref) <= TOL_F32 * max(1.0, np.abs(l_ref).max())
    ref = oracle.attn_bwd(gn, qn, kn, vn, scale, threads=8)[:3]
    for a, b, nm in zip((dq, dk, dv), ref, ("dq", "dk", "dv")):
        assert max_abs(host(a), b) <= TOL_F32 * max(1.0, np.abs(b).max()), nm
