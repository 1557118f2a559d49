"""GPU tests of the strided and token-major bf16 attention entry points, through the C ABI.

The kernels are the contiguous bf16 kernels with each tensor's rows read and written where they
lie, in the same arithmetic order, so every result (out, lse, delta, dq, dk, dv) must equal the
contiguous call's on the same values bit for bit; small cases are also checked against the CPU
oracle at the bf16 tolerances (O <= 2e-2, lse <= 1e-3, grads <= 5e-2). Padding between rows
and the columns of other heads must be left untouched.
"""
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
SENTINEL = -12345.0  # exactly representable in bf16; no kernel output equals it here


def case(msg):
    print(f"[case] {msg}", flush=True)


def heads_bf16(B, H, S, D, seed, n):
    """n tensors [B, H, S, D] of bf16-rounded N(0,1) values (as numpy fp32)."""
    out = []
    for i in range(n):
        x = synth.normal((B * H, S, D), seed + i).astype(np.float32)
        out.append(synth.bf16_round(x).reshape(B, H, S, D))
    return out


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to("cuda").to(torch.bfloat16)


def contiguous_run(q, k, v, g, scale):
    """The contiguous C-ABI path on [B, H, S, D] tensors: (out, lse, dq, dk, dv, delta)."""
    B, H, S, D = q.shape
    flat = [t.contiguous().view(B * H, S, D) for t in (q, k, v, g)]
    out, lse = A.attention_forward(*flat[:3], scale)
    dq, dk, dv, delta = A.attention_backward(flat[3], out, lse, *flat[:3], scale)
    return [t.view(B, H, S, D) for t in (out,)] + [lse] + [
        t.view(B, H, S, D) for t in (dq, dk, dv)] + [delta]


def same(a, b, what):
    assert a.shape == b.shape, what
    assert torch.equal(a, b), f"{what}: max diff {float((a.float() - b.float()).abs().max())}"


@pytest.mark.parametrize("B,H,S,D", [(2, 3, 70, 64), (1, 2, 129, 32), (2, 12, 300, 64),
                                     (3, 1, 1, 64), (1, 4, 1000, 32)])
def test_tokens_fused_qkv(gpu, B, H, S, D):
    """q, k, v sliced out of one fused [B*S, 3*H*D] projection output; out and dout
    token-major with a padded pitch; dq, dk, dv into one fused gradient buffer."""
    case(f"tokens fused qkv B={B} H={H} S={S} D={D}")
    scale = float(np.float32(1.0 / np.sqrt(D)))
    qn, kn, vn, gn = heads_bf16(B, H, S, D, 9100 + S + D, 4)
    q, k, v, g = (dev(x) for x in (qn, kn, vn, gn))
    ref = contiguous_run(q, k, v, g, scale)

    HD, pad = H * D, 8
    # fused rows [q heads | k heads | v heads], token-major
    qkv = torch.stack([t.permute(0, 2, 1, 3).reshape(B, S, HD) for t in (q, k, v)], dim=2)
    qkv = qkv.reshape(B * S, 3 * HD).contiguous()
    out = torch.full((B * S, HD + pad), SENTINEL, dtype=torch.bfloat16, device="cuda")
    dout = torch.zeros((B * S, HD + pad), dtype=torch.bfloat16, device="cuda")
    dout[:, :HD] = g.permute(0, 2, 1, 3).reshape(B * S, HD)
    lse = torch.empty(B * H * S, dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    dqkv = torch.full((B * S, 3 * HD), SENTINEL, dtype=torch.bfloat16, device="cuda")

    A.flash_attention_forward_bf16_tokens(out, HD + pad, lse, qkv, qkv[:, HD:], qkv[:, 2 * HD:],
                                          3 * HD, B, H, S, D, scale)
    A.flash_attention_backward_bf16_tokens(dqkv, dqkv[:, HD:], dqkv[:, 2 * HD:], 3 * HD, delta,
                                           dout, out, HD + pad, lse, qkv, qkv[:, HD:],
                                           qkv[:, 2 * HD:], 3 * HD, B, H, S, D, scale)
    torch.cuda.synchronize()

    to_heads = lambda t: t.reshape(B, S, H, D).permute(0, 2, 1, 3)
    same(to_heads(out[:, :HD]), ref[0], "out")
    assert bool((out[:, HD:] == SENTINEL).all()), "padding of out written"
    same(lse, ref[1].view(-1), "lse")
    same(delta, ref[5].view(-1), "delta")
    for i, nm in enumerate(("dq", "dk", "dv")):
        same(to_heads(dqkv[:, i * HD:(i + 1) * HD]), ref[2 + i], nm)

    if B * H * S <= 4000:  # the oracle on the same values
        flat = lambda x: x.reshape(B * H, S, D)
        o_ref, l_ref = oracle.attn_fwd(flat(qn), flat(kn), flat(vn), scale, threads=8)
        got = to_heads(out[:, :HD]).float().cpu().numpy().reshape(B * H, S, D)
        assert np.max(np.abs(got - o_ref)) <= TOL_O
        assert np.max(np.abs(lse.cpu().numpy().reshape(B * H, S) - l_ref)) <= TOL_LSE
        grads = oracle.attn_bwd(flat(gn), flat(qn), flat(kn), flat(vn), scale, threads=8)[:3]
        for i, (r, nm) in enumerate(zip(grads, ("dq", "dk", "dv"))):
            got = to_heads(dqkv[:, i * HD:(i + 1) * HD]).float().cpu().numpy()
            assert np.max(np.abs(got.reshape(B * H, S, D) - r)) <= TOL_GRAD, nm


def _token_shapes(n=8, seed=707):
    """Seeded random token-major shapes: B in [1, 3], H in [1, 4], S in [1, 700], D in {32, 64}."""
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 4)), int(rng.integers(1, 5)), int(rng.integers(1, 701)),
             int(rng.choice([32, 64]))) for _ in range(n)]


@pytest.mark.parametrize("B,H,S,D", _token_shapes())
def test_tokens_fused_qkv_random_shapes(gpu, B, H, S, D):
    """The fused-QKV token-major check above on seeded random shapes (tiles crossing S at every
    offset, both head sizes)."""
    test_tokens_fused_qkv(gpu, B, H, S, D)


@pytest.mark.parametrize("D", [64, 32])
def test_strided_views_cache_rows(gpu, D):
    """Tensor views of different placements in one call: q contiguous, k and v the first S
    rows of a [B, H, ctx, D] cache, out token-major; the backward writes dk, dv into cache-
    shaped buffers and dq token-major."""
    B, H, S, ctx = 2, 3, 200, 320
    case(f"strided views cache rows B={B} H={H} S={S} ctx={ctx} D={D}")
    scale = float(np.float32(1.0 / np.sqrt(D)))
    qn, kn, vn, gn = heads_bf16(B, H, S, D, 9300 + D, 4)
    q, k, v, g = (dev(x) for x in (qn, kn, vn, gn))
    ref = contiguous_run(q, k, v, g, scale)

    kc = torch.zeros((B, H, ctx, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    kc[:, :, :S], vc[:, :, :S] = k, v
    kc[:, :, S:], vc[:, :, S:] = float("nan"), float("inf")  # rows past S are never read
    tok = lambda: torch.full((B, S, H, D), SENTINEL, dtype=torch.bfloat16, device="cuda")
    out, dq = tok(), tok()
    dk = torch.full((B, H, ctx, D), SENTINEL, dtype=torch.bfloat16, device="cuda")
    dv = torch.full_like(dk, SENTINEL)
    lse = torch.empty(B * H * S, dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    heads = lambda t: t.permute(0, 2, 1, 3)  # [B, S, H, D] -> [B, H, S, D] view
    A.flash_attention_forward_bf16_strided(heads(out), lse, q, kc[:, :, :S], vc[:, :, :S], scale)
    A.flash_attention_backward_bf16_strided(heads(dq), dk[:, :, :S], dv[:, :, :S], delta, g,
                                            heads(out), lse, q, kc[:, :, :S], vc[:, :, :S], scale)
    torch.cuda.synchronize()
    same(heads(out), ref[0], "out")
    same(lse, ref[1].view(-1), "lse")
    same(heads(dq), ref[2], "dq")
    same(dk[:, :, :S], ref[3], "dk")
    same(dv[:, :, :S], ref[4], "dv")
    same(delta, ref[5].view(-1), "delta")
    assert bool((dk[:, :, S:] == SENTINEL).all()) and bool((dv[:, :, S:] == SENTINEL).all())


def test_tokens_cfg3_full(gpu):
    """B16 H12 T1024 D64 (the headline shape) through the fused-QKV token-major calls:
    bitwise equal to the contiguous calls on every slice."""
    B, H, S, D = 16, 12, 1024, 64
    case(f"tokens fused qkv cfg3 B={B} H={H} S={S} D={D}")
    scale = 0.125
    gen = torch.Generator(device="cuda").manual_seed(1234)
    HD = H * D
    qkv = torch.randn((B * S, 3 * HD), generator=gen, device="cuda").to(torch.bfloat16)
    dout = torch.randn((B * S, HD), generator=gen, device="cuda").to(torch.bfloat16)
    heads = lambda t: t.reshape(B, S, H, D).permute(0, 2, 1, 3)
    q, k, v = (heads(qkv[:, i * HD:(i + 1) * HD]) for i in range(3))
    ref = contiguous_run(q, k, v, heads(dout), scale)
    out = torch.empty((B * S, HD), dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B * H * S, dtype=torch.float32, device="cuda")
    delta = torch.empty_like(lse)
    dqkv = torch.empty_like(qkv)
    A.flash_attention_forward_bf16_tokens(out, HD, lse, qkv, qkv[:, HD:], qkv[:, 2 * HD:],
                                          3 * HD, B, H, S, D, scale)
    A.flash_attention_backward_bf16_tokens(dqkv, dqkv[:, HD:], dqkv[:, 2 * HD:], 3 * HD, delta,
                                           dout, out, HD, lse, qkv, qkv[:, HD:], qkv[:, 2 * HD:],
                                           3 * HD, B, H, S, D, scale)
    torch.cuda.synchronize()
    same(heads(out), ref[0], "out")
    same(lse, ref[1].view(-1), "lse")
    same(delta, ref[5].view(-1), "delta")
    for i, nm in enumerate(("dq", "dk", "dv")):
        same(heads(dqkv[:, i * HD:(i + 1) * HD]), ref[2 + i], nm)
