"""GPU tests of the bf16 attention with attention-probability dropout, through the C ABI.

The keep bits are a fixed function of (seed, bh*S + query, key) (Philox4x32-10; the CPU
oracle implements the same definition and is pinned by the generator's published
known-answer vectors), so for a given seed the GPU kernels and the oracle drop the same
probabilities, and the results are compared at the bf16 tolerances: O <= 2e-2, lse <= 1e-3,
dQ/dK/dV <= 5e-2 (max-abs, against the fp32 oracle on the same bf16-rounded inputs), for every
drop rate up to 0.5. Kept probabilities are scaled by 1/(1-p), and so are O, dP's kept terms,
dS and the gradients built from them, together with every bf16 rounding of those values on the
way (P f as the P V operand, dS as the dQ and dK operands, the stored outputs): at p = 0.9,
|O| reaches 16, where storing it in bf16 alone moves it by up to 0.03. Above p = 0.5, O and the
gradients are therefore held to the tolerance times 1/(1-p), the factor their values carry;
lse carries no factor.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from dadgpt_amd import attention as A
from dadgpt_amd import synth

pytestmark = pytest.mark.gpu

TOL_O = 2e-2
TOL_LSE = 1e-3
TOL_GRAD = 5e-2


def case(msg):
    print(f"[case] {msg}", flush=True)


def within_scaled(got, ref, tol, p, what):
    """max |got - ref| <= tol for p <= 0.5; above, tol / (1 - p): the bf16 tolerance at the
    magnitude dropout scales the values to."""
    bound = tol if p <= 0.5 else tol / (1.0 - p)
    err = max_abs(got, ref)
    print(f"  {what}: max-abs {err:.3e} (p={p}, bound {bound:.3e})", flush=True)
    assert err <= bound, f"{what}: max-abs {err:.3e} > {bound:.3e}"


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to("cuda").to(torch.bfloat16)


def host(t):
    return t.float().cpu().numpy()


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def run(q, k, v, g, scale, p, seed):
    BH, S, D = q.shape
    out = torch.empty_like(q)
    lse = torch.empty((BH, S), dtype=torch.float32, device="cuda")
    A.flash_attention_forward_bf16_dropout(out, lse, q, k, v, BH, S, D, scale, p, seed)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty_like(lse)
    A.flash_attention_backward_bf16_dropout(dq, dk, dv, delta, g, out, lse, q, k, v, BH, S, D,
                                            scale, p, seed)
    torch.cuda.synchronize()
    return out, lse, dq, dk, dv, delta


@pytest.mark.parametrize("BH,S,D,p", [(2, 70, 64, 0.1), (3, 129, 64, 0.5), (1, 300, 32, 0.25),
                                      (2, 64, 32, 0.9), (1, 1, 64, 0.3), (2, 257, 64, 0.2)])
def test_dropout_matches_oracle(gpu, BH, S, D, p):
    case(f"bf16 dropout BH={BH} S={S} D={D} p={p}")
    seed = 0x0DAD_6B7F_0000_0000 + 31 * S + D
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=500 + S + D, with_dout=True, bf16=True)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    q, k, v, g = (dev(x) for x in (qn, kn, vn, gn))
    out, lse, dq, dk, dv, _ = run(q, k, v, g, scale, p, seed)
    o_ref, l_ref = oracle.attn_fwd_dropout(qn, kn, vn, scale, p, seed)
    within_scaled(host(out), o_ref, TOL_O, p, "out")
    assert max_abs(host(lse), l_ref) <= TOL_LSE
    # the backward from the GPU's own O (delta uses it), as the reference's caller would
    refs = oracle.attn_bwd_dropout(gn, qn, kn, vn, scale, p, seed)[:3]
    for got, ref, nm in zip((dq, dk, dv), refs, ("dq", "dk", "dv")):
        within_scaled(host(got), ref, TOL_GRAD, p, nm)


def _dropout_shapes(n=8, seed=909):
    """Seeded random dropout cases: BH in [1, 4], S in [1, 500], D in {32, 64}, p in
    {0.05, 0.1, 0.3, 0.5}."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 5)), int(rng.integers(1, 501)), int(rng.choice([32, 64])),
             float(rng.choice([0.05, 0.1, 0.3, 0.5]))) for _ in range(n)]


@pytest.mark.parametrize("BH,S,D,p", _dropout_shapes())
def test_dropout_random_shapes(gpu, BH, S, D, p):
    """The bf16 and fp32 dropout checks on seeded random shapes and rates."""
    test_dropout_matches_oracle(gpu, BH, S, D, p)
    test_dropout_f32_matches_oracle(gpu, BH, S, D, p)


def test_dropout_rate_zero_equals_plain(gpu):
    """p = 0 keeps every probability with factor 1: the forward and dQ are bit for bit the
    plain kernels' (dK/dV folds delta in after its products instead of before: within
    rounding)."""
    BH, S, D = 3, 300, 64
    case(f"bf16 dropout p=0 vs plain BH={BH} S={S} D={D}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=611, with_dout=True, bf16=True)
    q, k, v, g = (dev(x) for x in (qn, kn, vn, gn))
    out, lse, dq, dk, dv, delta = run(q, k, v, g, 0.125, 0.0, 5)
    o2, l2 = A.attention_forward(q, k, v, 0.125)
    dq2, dk2, dv2, d2 = A.attention_backward(g, o2, l2, q, k, v, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(out, o2) and torch.equal(lse, l2)
    assert torch.equal(dq, dq2) and torch.equal(delta, d2)
    assert max_abs(host(dk), host(dk2)) <= 1e-2 and max_abs(host(dv), host(dv2)) <= 1e-2


def test_dropout_seed_changes_mask_and_is_deterministic(gpu):
    BH, S, D = 2, 200, 64
    case(f"bf16 dropout determinism BH={BH} S={S}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=612, with_dout=True, bf16=True)
    q, k, v, g = (dev(x) for x in (qn, kn, vn, gn))
    a = run(q, k, v, g, 0.125, 0.3, 11)
    b = run(q, k, v, g, 0.125, 0.3, 11)
    c = run(q, k, v, g, 0.125, 0.3, 12)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    assert not torch.equal(a[0], c[0])
    assert torch.equal(a[1], c[1])  # lse does not depend on the mask


def test_dropout_cfg3_full(gpu):
    """B16 H12 T1024 D64 with p = 0.1: finite, repeatable, and the forward and backward of
    sampled slices (first, middle, last: mask counters up to 191*1024 + 1023) against the
    oracle (its full cfg3 backward would take minutes on the CPU)."""
    BH, S, D = 192, 1024, 64
    case(f"bf16 dropout cfg3 BH={BH} S={S} D={D}")
    gen = torch.Generator(device="cuda").manual_seed(77)
    mk = lambda: torch.randn((BH, S, D), generator=gen, device="cuda").to(torch.bfloat16)
    q, k, v, g = mk(), mk(), mk(), mk()
    seed, p = 2024, 0.1
    a = run(q, k, v, g, 0.125, p, seed)
    b = run(q, k, v, g, 0.125, p, seed)
    for x, y in zip(a, b):
        assert torch.equal(x, y) and bool(torch.isfinite(x).all())
    qn, kn, vn, gn = host(q), host(k), host(v), host(g)
    for bh in (0, 97, 191):  # the mask rows of slice bh are bh*S + i
        o_ref = oracle.attn_fwd_dropout_slices(qn, kn, vn, 0.125, p, seed, bh, bh + 1)
        within_scaled(host(a[0][bh]), o_ref[0], TOL_O, p, f"out[{bh}]")
        refs = oracle.attn_bwd_dropout_slices(gn, qn, kn, vn, 0.125, p, seed, bh, bh + 1)
        for got, ref, nm in zip(a[2:5], refs, ("dq", "dk", "dv")):
            within_scaled(host(got[bh]), ref[0], TOL_GRAD, p, f"{nm}[{bh}]")


# ---- fp32 (the reference's precision): max-abs <= 1e-5 against the oracle ----

TOL_F32 = 1e-5


def run_f32(q, k, v, g, scale, p, seed):
    BH, S, D = q.shape
    out = torch.empty_like(q)
    lse = torch.empty((BH, S), dtype=torch.float32, device="cuda")
    A.flash_attention_forward_dropout(out, lse, q, k, v, BH, S, D, scale, p, seed)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    delta = torch.empty_like(lse)
    A.flash_attention_backward_dropout(dq, dk, dv, delta, g, out, lse, q, k, v, BH, S, D, scale,
                                       p, seed)
    torch.cuda.synchronize()
    return out, lse, dq, dk, dv, delta


@pytest.mark.parametrize("BH,S,D,p", [(2, 70, 64, 0.1), (1, 129, 32, 0.5), (2, 200, 64, 0.3),
                                      (1, 1, 32, 0.2)])
def test_dropout_f32_matches_oracle(gpu, BH, S, D, p):
    case(f"fp32 dropout BH={BH} S={S} D={D} p={p}")
    seed = 99 + S
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=700 + S + D, with_dout=True)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    f32 = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).to("cuda")
    q, k, v, g = (f32(x) for x in (qn, kn, vn, gn))
    out, lse, dq, dk, dv, delta = run_f32(q, k, v, g, scale, p, seed)
    o_ref, l_ref = oracle.attn_fwd_dropout(qn, kn, vn, scale, p, seed)
    assert max_abs(host(out), o_ref) <= TOL_F32
    assert max_abs(host(lse), l_ref) <= TOL_F32
    refs = oracle.attn_bwd_dropout(gn, qn, kn, vn, scale, p, seed, out=o_ref)
    for got, ref, nm in zip((dq, dk, dv, delta), refs, ("dq", "dk", "dv", "delta")):
        assert max_abs(host(got), ref) <= TOL_F32, nm


def test_dropout_f32_rate_zero_equals_plain(gpu):
    BH, S, D = 2, 150, 64
    case(f"fp32 dropout p=0 vs plain BH={BH} S={S}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=711, with_dout=True)
    f32 = lambda x: torch.from_numpy(np.ascontiguousarray(x, np.float32)).to("cuda")
    q, k, v, g = (f32(x) for x in (qn, kn, vn, gn))
    a = run_f32(q, k, v, g, 0.125, 0.0, 3)
    o2, l2 = A.attention_forward(q, k, v, 0.125)
    dq2, dk2, dv2, d2 = A.attention_backward(g, o2, l2, q, k, v, 0.125)
    torch.cuda.synchronize()
    for x, y in zip(a, (o2, l2, dq2, dk2, dv2, d2)):
        assert torch.equal(x, y)
