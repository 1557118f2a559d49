"""Tests of the generation path (libdadgpt_gen: hipBLASLt projections and the batched GPT-2
prefill/decode driver).

CPU (no GPU): the numpy GPT-2 oracle against the reference's own CPU operators composed in
model_forward's order (oracle/_ref), the parameter layout, the library's exports and its
host-side argument checks.

GPU: the bf16 GEMMs against torch fp32 on the same bf16 inputs; generation on small configs
against the oracle (teacher-forced: each step's logits are compared on the GPU's own token
history); the KV-cache invariant (decoding a token equals prefilling the longer prompt,
tests/test_model.cpp:216-252); and bf16 attention against fp32 attention on the GPT-2 124M
shape (logits within 5e-2 of each other while the token history is shared, observed 1.3e-2
against a logit spread of ~0.55; tokens identical except at near-ties: random-init GPT-2
logits have top-1/top-2 margins down to ~1e-4, inside the logit difference that bf16
attention itself makes).

Tolerances: logits max-abs <= 2e-2 against the oracle with the product's bf16 rounding points
(round_bf16=True); the GPU tokens must equal the oracle's wherever the oracle's top-1/top-2
margin exceeds twice that tolerance. GEMMs: max-abs <= 1e-4 * sqrt(K) (fp32 accumulation of
exact bf16 products, different order).
"""
import os
import re
import subprocess

import numpy as np
import pytest

import oracle
from dadgpt_amd import synth
from oracle import gpt2_oracle as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

TINY = dict(d_model=128, n_layers=2, n_heads=4, d_ff=512, ctx_len=64, vocab_size=512)
TINY64 = dict(d_model=256, n_layers=2, n_heads=4, d_ff=512, ctx_len=96, vocab_size=384)
GPT2 = dict(d_model=768, n_layers=12, n_heads=12, d_ff=3072, ctx_len=1024, vocab_size=50257)
# GPT-2's layer shapes (d 768, d_ff 3072: the skinny decode kernels' 8-wave LayerNorm prologue,
# 16-wave K-blocked fc2, 4-column Wo tiles) on two layers, with a vocabulary whose logits
# projection ends in a partial 16-column tile and leaves 626 candidates per row for the pick
MID = dict(d_model=768, n_layers=2, n_heads=12, d_ff=3072, ctx_len=128, vocab_size=10007)
# the other reduction lengths of the 8-wave LayerNorm prologue (K = 512 with a 2048-deep fc2,
# K = 1024 with d_head 64 over 16 heads)
W512 = dict(d_model=512, n_layers=2, n_heads=8, d_ff=2048, ctx_len=64, vocab_size=3001)
W1024 = dict(d_model=1024, n_layers=1, n_heads=16, d_ff=3072, ctx_len=64, vocab_size=2053)
TOL_LOGIT = 2e-2


def case(msg):
    print(f"[case] {msg}", flush=True)


# ------------------------------------------------------------------------------- CPU

def test_param_count_is_the_reference_layout():
    """GPT-2 124M has 124,439,808 parameters with the tied lm_head (the arena of
    src/model.cpp:17-56 holds each once)."""
    assert G.offsets(GPT2)["total"][0] == 124_439_808
    from dadgpt_amd import gpt2

    assert gpt2.param_count(GPT2) == 124_439_808
    assert gpt2.param_count(TINY) == G.offsets(TINY)["total"][0]
    assert gpt2.param_count(dict(TINY, n_heads=3)) == 0  # d_head 128/3 is not integral
    assert gpt2.param_count(dict(TINY, n_heads=1)) == 0  # d_head 128 is unsupported


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
def test_oracle_primitives_match_reference_operators():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((7, 96)).astype(np.float32) * 3
    w, b = rng.standard_normal(96).astype(np.float32), rng.standard_normal(96).astype(np.float32)
    assert np.abs(G.layernorm(x, w, b) - oracle.ref_layernorm(x, w, b)).max() <= 2e-6
    assert np.abs(G.gelu(x) - oracle.ref_gelu(x)).max() <= 2e-6
    a, m = rng.standard_normal((5, 96)).astype(np.float32), rng.standard_normal((96, 40))
    assert np.abs(a @ m.astype(np.float32) - oracle.ref_matmul(a, m)).max() <= 1e-4


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("cfg", [dict(d_model=64, n_layers=2, n_heads=2, d_ff=128, ctx_len=40,
                                      vocab_size=97), TINY])
def test_oracle_forward_matches_reference_composition(cfg):
    """The numpy forward equals the reference's CPU operators composed as model_forward."""
    n = G.offsets(cfg)["total"][0]
    params = synth.normal((n,), 77) * np.float32(0.05)
    toks = synth.uniform_int(0, cfg["vocab_size"] - 1, 33, 78)
    a = G.forward(params, cfg, toks)
    b = oracle.ref_gpt2_forward(params, cfg, toks)
    assert np.abs(a - b).max() <= 1e-5 * max(1.0, np.abs(b).max())


def test_oracle_greedy_is_causal_recompute():
    """Greedy continuation's step t logits equal the full forward's last row over the prompt
    plus tokens 0..t-1, and rows of a longer sequence do not see later tokens (causality:
    a dropped mask fails this)."""
    cfg = dict(d_model=64, n_layers=1, n_heads=2, d_ff=64, ctx_len=32, vocab_size=50)
    n = G.offsets(cfg)["total"][0]
    params = synth.normal((n,), 5) * np.float32(0.1)
    prompt = [3, 1, 4, 1, 5]
    toks, rows = G.greedy(params, cfg, prompt, 4)
    full = G.forward(params, cfg, prompt + list(toks[:3]))
    for t in range(4):
        np.testing.assert_array_equal(rows[t], G.forward(params, cfg, prompt + list(toks[:t]))[-1])
    np.testing.assert_allclose(full[len(prompt) - 1:], rows[:4], rtol=0, atol=1e-5)


# Hand-worked cases of src/generate.cpp:97-110 (limit = min(max_len, ctx_len); a prompt of
# len >= limit, len > 1, keeps token 0 and its last max(limit - 2, 0) tokens): (len, max_len,
# ctx_len, indices of the prompt that are kept).
TRUNC_CASES = [
    (10, 6, 1024, [0, 6, 7, 8, 9]),          # keep 4
    (10, 11, 1024, list(range(10))),         # room left: unchanged
    (10, 10, 1024, [0] + list(range(2, 10))),  # len == limit: one token goes
    (10, 100, 8, [0] + list(range(4, 10))),  # the context caps the limit (keep 6)
    (1, 0, 8, [0]),                          # a single token is never truncated
    (3, 1, 8, [0]),                          # keep max(-1, 0) = 0
    (3, 2, 8, [0]),                          # keep 0
    (3, 3, 8, [0, 2]),                       # keep 1
    (5, -4, 8, [0]),                         # a negative limit keeps the first token
    (7, 8, 8, list(range(7))),               # len = limit - 1: unchanged
]


def _trunc_pins(fn):
    """Every pin of a truncation function: the hand-worked cases, then invariants over a
    grid (the first token and a suffix survive; a truncated prompt leaves room for one token
    when the limit allows; truncation is idempotent). Returns the first failure or None."""
    for n, max_len, ctx, keep in TRUNC_CASES:
        prompt = [100 + i for i in range(n)]
        got = list(fn(prompt, max_len, ctx))
        if got != [prompt[i] for i in keep]:
            return ("case", n, max_len, ctx, got)
    for n in range(1, 13):
        prompt = [50 + 3 * i for i in range(n)]
        for ctx in (1, 2, 5, 9, 16):
            for max_len in range(-2, 19):
                got = list(fn(prompt, max_len, ctx))
                limit = min(max_len, ctx)
                if not got or got[0] != prompt[0]:
                    return ("first", n, max_len, ctx, got)
                if len(got) > 1 and got[1:] != prompt[n - (len(got) - 1):]:
                    return ("suffix", n, max_len, ctx, got)
                if limit >= 2 and len(got) >= limit:
                    return ("room", n, max_len, ctx, got)
                if (n < limit or n == 1) and got != prompt:
                    return ("unchanged", n, max_len, ctx, got)
                if n >= limit and n > 1 and len(got) != max(limit - 1, 1):
                    return ("length", n, max_len, ctx, got)
                if list(fn(got, max_len, ctx)) != got:
                    return ("idempotent", n, max_len, ctx, got)
    return None


def _trunc_bug(bug):
    """The oracle's truncation with one plausible mistake. (Dropping the reference's len > 1
    guard changes nothing: a one-token prompt keeps its token either way.)"""
    def fn(prompt, max_len, ctx):
        limit = max_len if bug == "no_ctx_cap" else min(max_len, ctx)
        toks = list(prompt)
        cond = len(toks) > limit if bug == "strict_compare" else len(toks) >= limit
        if cond and len(toks) > 1:
            keep = max(limit - 2, 0)
            if bug == "keep_off_by_one":
                keep = max(limit - 1, 0)
            if bug == "keep_too_few":
                keep = max(limit - 3, 0)
            tail = toks[len(toks) - keep:] if keep else []
            if bug == "head_not_tail":
                tail = toks[1:1 + keep]
            return tail if bug == "drops_first" else [toks[0]] + tail
        return toks
    return fn


def test_truncation_oracle_pins():
    """The oracle's truncation passes every pin."""
    assert _trunc_pins(G.truncate_prompt) is None


@pytest.mark.parametrize("bug", ["no_ctx_cap", "strict_compare", "keep_off_by_one",
                                 "keep_too_few", "head_not_tail", "drops_first"])
def test_truncation_pins_catch_mistakes(bug):
    assert _trunc_pins(_trunc_bug(bug)) is not None, bug


def test_library_truncation_equals_oracle():
    """dadgpt_gpt2_truncate_prompt (the host half of dadgpt_gpt2_generate_tokens) against the
    oracle over the pin grid, and its argument checks."""
    from dadgpt_amd import attention as A
    from dadgpt_amd import gpt2

    assert _trunc_pins(gpt2.truncate_prompt) is None
    for n in range(1, 40, 3):
        prompt = list(range(7, 7 + n))
        for ctx in (1, 4, 16, 1024):
            for max_len in (-1, 0, 1, 2, 3, n - 1, n, n + 1, 2000):
                assert gpt2.truncate_prompt(prompt, max_len, ctx) == \
                    G.truncate_prompt(prompt, max_len, ctx), (n, max_len, ctx)
    with pytest.raises(A.AttentionError):
        gpt2.truncate_prompt([], 5, 8)
    with pytest.raises(A.AttentionError):
        gpt2.truncate_prompt([1, 2], 5, 0)


def test_oracle_stop_token_cuts_the_greedy_continuation():
    """generate_tokens with a stop token equals the no-stop continuation cut after the stop
    token's first occurrence among the picks (src/generate.cpp:131), and the sequence never
    exceeds min(max_len, ctx_len); the picks themselves are greedy()'s."""
    cfg = dict(d_model=64, n_layers=1, n_heads=2, d_ff=64, ctx_len=24, vocab_size=13)
    n = G.offsets(cfg)["total"][0]
    params = synth.normal((n,), 9) * np.float32(0.3)
    prompt = [3, 1, 4, 1, 5]
    full = G.generate_tokens(params, cfg, prompt, 18)
    assert len(full) == 18 and full[:5] == prompt
    toks, _ = G.greedy(params, cfg, prompt, 13)
    assert full[5:] == [int(t) for t in toks]
    for k in (0, 2, 7):
        stop = full[5 + k]
        first = full[5:].index(stop)
        assert G.generate_tokens(params, cfg, prompt, 18, stop) == full[:5 + first + 1]
    assert G.generate_tokens(params, cfg, prompt, 500) == G.generate_tokens(params, cfg, prompt,
                                                                              24)
    assert len(G.generate_tokens(params, cfg, prompt, 500)) == 24
    long = list(range(13)) * 3  # 39 tokens, ctx 24: truncated to 23, one pick
    out = G.generate_tokens(params, cfg, long, 100)
    assert out[:23] == G.truncate_prompt(long, 100, 24) and len(out) == 24


def gen_header_functions():
    names = set()
    for h in ("gpt2_generate.h", "gpu_matmul.h"):
        names |= set(re.findall(r"\b(dadgpt_\w+)\s*\(", open(os.path.join(ROOT, "include",
                                                                       "dadgpt", h)).read()))
    return sorted(names)


def test_gen_library_exports_declared_symbols():
    from dadgpt_amd import gpt2

    assert gen_header_functions() == sorted(gpt2.GEN_SYMBOLS)
    out = subprocess.run(["nm", "-D", "--defined-only", gpt2.GEN_PATH], check=True,
                         capture_output=True, text=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert not [s for s in gpt2.GEN_SYMBOLS if s not in syms]
    L = gpt2.gen_lib()
    for s in gpt2.GEN_SYMBOLS:
        assert hasattr(L, s)


def test_gen_argument_checks_before_any_hip_call():
    import ctypes

    from dadgpt_amd import gpt2

    L = gpt2.gen_lib()
    bad = gpt2.Config(d_model=100, n_layers=1, n_heads=3, d_ff=8, ctx_len=8, vocab_size=8)
    m = ctypes.c_void_p()
    assert L.dadgpt_gpt2_create(ctypes.byref(bad), 0x1000, 1, 0, ctypes.byref(m)) == 1
    assert "d_head" in gpt2.last_error()
    good = gpt2.Config(**TINY)
    assert L.dadgpt_gpt2_create(ctypes.byref(good), None, 1, 0, ctypes.byref(m)) == 1
    assert L.dadgpt_gpt2_create(ctypes.byref(good), 0x1000, 0, 0, ctypes.byref(m)) == 1
    assert L.dadgpt_gpt2_init_params(None, ctypes.byref(good), 1, None) == 1
    assert L.dadgpt_gpt2_generate(None, None, None, 1, 1, 1, None, None, None, None) == 1
    assert L.dadgpt_matmul_bf16(None, 0x1000, 0x1000, 0x1000, 1, 1, 1, None) == 1
    # materialized attention with dropout: the rate, and probs kept apart from dropped
    P = 0x1000
    assert L.dadgpt_attention_materialized_forward_dropout(P, P, P, P + 64, P, P, P, 2, 8, 64,
                                                           0.125, 1.0, 7, None) == 1
    assert "dropout_p" in gpt2.last_error()
    assert L.dadgpt_attention_materialized_forward_dropout(P, P, P, P, P, P, P, 2, 8, 64, 0.125,
                                                           0.1, 7, None) == 1
    assert "dropped" in gpt2.last_error()
    assert L.dadgpt_attention_materialized_backward_dropout(*[P] * 10, 2, 8, 64, 0.125, -0.1, 7,
                                                            None) == 1


# ------------------------------------------------------------------------------- GPU

def _gpu_model(cfg, seed, max_batch, attention="bf16"):
    import torch

    from dadgpt_amd import gpt2

    params = gpt2.init_params(cfg, seed)
    torch.cuda.synchronize()
    host = params.float().cpu().numpy()
    return gpt2.GPT2(cfg, params, max_batch, attention), host


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N", [(1, 768, 2304), (16, 768, 3072), (37, 96, 50), (256, 3072, 768)])
def test_matmul_bf16_against_torch(gpu, M, K, N):
    import torch

    from dadgpt_amd import gpt2

    case(f"matmul bf16 M={M} K={K} N={N}")
    a = torch.from_numpy(synth.normal((M, K), 11)).to(gpu).to(torch.bfloat16)
    b = torch.from_numpy(synth.normal((K, N), 12)).to(gpu).to(torch.bfloat16)
    bt = b.t().contiguous()
    h = gpt2.Blas()
    out = h.matmul(a, b)
    out_t = h.matmul_transposed_b(a, bt)
    torch.cuda.synchronize()
    ref = a.float().cpu() @ b.float().cpu()
    tol = 1e-4 * np.sqrt(K) * float(ref.abs().max().clamp(min=1.0))
    assert float((out.cpu() - ref).abs().max()) <= tol
    assert float((out_t.cpu() - ref).abs().max()) <= tol
    h.close()


@pytest.mark.gpu
def test_matmul_logits_shape_against_torch(gpu):
    """The weight-tied logits GEMM: [16, 768] x [50257, 768]^T (odd N)."""
    import torch

    from dadgpt_amd import gpt2

    case("matmul transposed_b logits 16x768x50257")
    a = torch.from_numpy(synth.normal((16, 768), 13)).to(gpu).to(torch.bfloat16)
    w = (torch.from_numpy(synth.normal((50257, 768), 14)) * 0.02).to(gpu).to(torch.bfloat16)
    h = gpt2.Blas()
    out = h.matmul_transposed_b(a, w)
    torch.cuda.synchronize()
    ref = a.float() @ w.float().t()
    assert float((out - ref).abs().max()) <= 1e-4 * np.sqrt(768)
    h.close()


def _prompts(cfg, lens, seed):
    return [list(synth.uniform_int(0, cfg["vocab_size"] - 1, int(n), seed + i))
            for i, n in enumerate(lens)]


@pytest.mark.gpu
@pytest.mark.parametrize("cfg,attention", [(TINY, "bf16"), (TINY, "fp32"),
                                           (TINY, "fp32_materialized"), (TINY64, "bf16"),
                                           (TINY64, "fp32"), (TINY64, "fp32_materialized"),
                                           (MID, "bf16"), (MID, "fp32"), (W512, "bf16"),
                                           (W1024, "bf16")])
def test_generate_matches_oracle(gpu, cfg, attention):
    case(f"generate vs oracle d={cfg['d_model']} H={cfg['n_heads']} attention={attention}")
    model, params = _gpu_model(cfg, seed=21, max_batch=4, attention=attention)
    prompts = _prompts(cfg, [5, 17, 1, 30], 300)
    new = 12
    out = model.generate(prompts, new, logits=True)
    for b, p in enumerate(prompts):
        seq = list(p)
        for t in range(new):
            ref = G.forward(params, cfg, seq, round_bf16=True)[-1]
            got = out["logits"][t, b]
            assert np.abs(got - ref).max() <= TOL_LOGIT, (b, t, np.abs(got - ref).max())
            top = np.sort(ref)[-2:]
            if top[1] - top[0] > 2 * TOL_LOGIT:
                assert out["tokens"][b, t] == int(np.argmax(ref)), (b, t)
            assert out["tokens"][b, t] == int(np.argmax(got)), "pick is the first maximum"
            seq.append(int(out["tokens"][b, t]))  # teacher forcing on the GPU's history
    model.close()


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [TINY64, MID])
def test_decode_step_equals_prefill_of_longer_prompt(gpu, cfg):
    """KV cache invariant: the logits of decode step t equal the prefill logits of the prompt
    extended by the first t generated tokens (tests/test_model.cpp:216-252, 375-414). On MID
    the decode steps run the skinny kernels and the prefill hipBLASLt, two independent
    implementations of every projection. Bound: 1e-2 at d 256; at d 768 the two paths' bf16
    activations (the same rounding points, different summation orders) flip in more elements
    (measured 1.09e-2), so the bound is the oracle tolerance, which each path meets alone."""
    case(f"decode step == prefill of the longer prompt d={cfg['d_model']}")
    tol = 1e-2 if cfg is TINY64 else TOL_LOGIT
    model, _ = _gpu_model(cfg, seed=22, max_batch=3)
    prompts = _prompts(cfg, [9, 40, 2], 400)
    out = model.generate(prompts, 6, logits=True)
    for t in (1, 3, 5):
        longer = [list(p) + list(out["tokens"][b, :t]) for b, p in enumerate(prompts)]
        again = model.generate(longer, 1, logits=True)
        err = float(np.abs(again["logits"][0] - out["logits"][t]).max())
        print(f"step {t}: max |decode - prefill| = {err:.3g}", flush=True)
        assert err <= tol, t
    model.close()


@pytest.mark.gpu
def test_generate_beyond_the_skinny_batch_matches_oracle(gpu):
    """More than 16 sequences: the decode step runs on the hipBLASLt projections and the
    two-stage greedy pick (whose last stage also embeds the next step's input rows), instead
    of the skinny kernels; teacher-forced against the oracle as test_generate_matches_oracle."""
    cfg = TINY
    n = 20
    case(f"generate vs oracle, {n} sequences (non-skinny decode step)")
    model, params = _gpu_model(cfg, seed=24, max_batch=n)
    prompts = _prompts(cfg, [1 + (7 * i) % 23 for i in range(n)], 600)
    new = 6
    out = model.generate(prompts, new, logits=True)
    for b, p in enumerate(prompts):
        seq = list(p)
        for t in range(new):
            ref = G.forward(params, cfg, seq, round_bf16=True)[-1]
            got = out["logits"][t, b]
            assert np.abs(got - ref).max() <= TOL_LOGIT, (b, t, np.abs(got - ref).max())
            assert out["tokens"][b, t] == int(np.argmax(got)), "pick is the first maximum"
            seq.append(int(out["tokens"][b, t]))
    model.close()


@pytest.mark.gpu
def test_generate_is_deterministic_and_batch_independent(gpu):
    """Same tokens run to run, and a sequence's tokens do not depend on its batch mates."""
    cfg = TINY
    case("generate determinism / batch independence")
    model, _ = _gpu_model(cfg, seed=23, max_batch=4)
    prompts = _prompts(cfg, [8, 3, 20, 11], 500)
    a = model.generate(prompts, 10)
    b = model.generate(prompts, 10)
    np.testing.assert_array_equal(a["tokens"], b["tokens"])
    alone = model.generate([prompts[2]], 10)
    np.testing.assert_array_equal(alone["tokens"][0], a["tokens"][2])
    model.close()


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [TINY, MID], ids=["tiny", "mid"])
def test_graph_replayed_steps_equal_eager_steps(gpu, cfg):
    """The captured decode step, replayed for every step after the first, gives the same
    tokens and logits as launching each step eagerly; checked over two calls in a row (the
    second with a smaller batch, so a second graph is captured) with eager work between.
    Both configs run the skinny decode step, the one that is captured (steps with hipBLASLt
    calls run eagerly whatever set_graphs says)."""
    case(f"graph replay vs eager decode steps d_model={cfg['d_model']}")
    model, _ = _gpu_model(cfg, seed=25, max_batch=4)
    for prompts in (_prompts(cfg, [7, 30, 2, 15], 700), _prompts(cfg, [11, 4], 800)):
        g = model.generate(prompts, 9, logits=True)
        model.set_graphs(False)
        e = model.generate(prompts, 9, logits=True)
        model.set_graphs(True)
        np.testing.assert_array_equal(g["tokens"], e["tokens"])
        np.testing.assert_array_equal(g["logits"], e["logits"])
    model.close()


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [TINY, TINY64], ids=["skinny_graph", "hipblaslt_eager"])
def test_nan_logits_pick_column_zero(gpu, cfg):
    """Rows whose logits are all NaN (a NaN parameter arena) have no first maximum to find:
    the pick takes column 0, as std::max_element does (src/generate.cpp:34-37), and the
    next step's input row is that token's embedding, so every index stays inside the
    vocabulary. Both pick paths: the skinny logits' candidates (TINY, replayed graph) and
    the two-stage pick after hipBLASLt logits (TINY64)."""
    import torch

    from dadgpt_amd import gpt2

    case(f"NaN logits pick column 0, d_model={cfg['d_model']}")
    params = gpt2.init_params(cfg, 26)
    params.fill_(float("nan"))
    torch.cuda.synchronize()
    model = gpt2.GPT2(cfg, params, 2)
    out = model.generate(_prompts(cfg, [5, 9], 900), 4, logits=True)
    assert np.isnan(out["logits"]).all()
    np.testing.assert_array_equal(out["tokens"], np.zeros((2, 4), np.int32))
    model.close()


@pytest.mark.gpu
def test_generate_rejects_overflowing_context(gpu):
    from dadgpt_amd import attention as A

    cfg = TINY
    case("generate context overflow")
    model, _ = _gpu_model(cfg, seed=24, max_batch=2)
    with pytest.raises(A.AttentionError):
        model.generate([[1] * 60], 5)  # 60 + 5 > ctx 64
    with pytest.raises(A.AttentionError):
        model.generate([[1, 2, cfg["vocab_size"]]], 2)
    model.close()


def _cut_at_stop(seq, n_prompt, stop):
    """A generated sequence cut after the first pick equal to stop (prompt untouched)."""
    picks = list(seq[n_prompt:])
    return list(seq[:n_prompt]) + (picks[:picks.index(stop) + 1] if stop in picks else picks)


@pytest.mark.gpu
@pytest.mark.parametrize("cfg", [TINY, TINY64, MID], ids=["skinny_graph", "hipblaslt_eager",
                                                           "mid"])
def test_generate_tokens_stop_token_leaves_other_rows_unchanged(gpu, cfg):
    """generate_tokens (src/generate.cpp:94-139) for a batch: with one row's stop token set to
    a token it picks mid-way, that row ends right after the stop token's first occurrence and
    every other row is token for token the run without stop tokens; each row with no stop
    token equals dadgpt_gpt2_generate of its prompt alone for max_len - len tokens."""
    case(f"generate_tokens stop token, d_model={cfg['d_model']}")
    model, _ = _gpu_model(cfg, seed=27, max_batch=4)
    prompts = _prompts(cfg, [6, 19, 2, 11], 1000)
    max_len = 34
    free = model.generate_tokens(prompts, max_len)
    for b, p in enumerate(prompts):
        assert len(free[b]) == max_len and free[b][:len(p)] == p
        alone = model.generate([p], max_len - len(p))["tokens"][0]
        assert free[b][len(p):] == [int(t) for t in alone], b
    for row, k in ((1, 4), (0, 0), (3, max_len - 12)):
        stops = [-1] * 4
        stops[row] = free[row][len(prompts[row]) + k]
        got = model.generate_tokens(prompts, max_len, stops)
        for b in range(4):
            want = _cut_at_stop(free[b], len(prompts[b]), stops[b]) if b == row else free[b]
            assert got[b] == want, (row, k, b)
        assert len(got[row]) <= len(prompts[row]) + k + 1
    # every row stops at its first pick: with the limit at the context (more than 32 steps)
    # the step loop ends early; the picks are kept
    firsts = [free[b][len(p)] for b, p in enumerate(prompts)]
    got = model.generate_tokens(prompts, cfg["ctx_len"], firsts)
    assert got == [p + [firsts[b]] for b, p in enumerate(prompts)]
    model.close()


@pytest.mark.gpu
def test_generate_tokens_truncates_and_matches_oracle(gpu):
    """A prompt longer than the context is truncated as the reference does (first token plus
    the last ctx_len - 2) and continued to the context; a prompt with no room is returned as
    it is; short prompts run to max_len. Picks against the oracle's generate_tokens, exact
    except at near-ties (the oracle's top-1/top-2 margin within twice the logit tolerance)."""
    import torch  # noqa: F401

    cfg = TINY
    case("generate_tokens truncation vs oracle")
    model, params = _gpu_model(cfg, seed=28, max_batch=3)
    ctx = cfg["ctx_len"]
    prompts = _prompts(cfg, [ctx + 9, 4, 30], 1100)
    for max_len, stops in ((200, None), (40, [-1, -1, -1]), (31, None)):
        got = model.generate_tokens(prompts, max_len, stops)
        for b, p in enumerate(prompts):
            limit = min(max_len, ctx)
            seq = G.truncate_prompt(p, max_len, ctx)
            assert got[b][:len(seq)] == seq, (max_len, b)
            assert len(got[b]) == max(limit, len(seq)), (max_len, b, len(got[b]))
            while len(seq) < len(got[b]):
                ref = G.forward(params, cfg, seq, round_bf16=True)[-1]
                top = np.sort(ref)[-2:]
                t = got[b][len(seq)]
                if top[1] - top[0] > 2 * TOL_LOGIT:
                    assert t == int(np.argmax(ref)), (max_len, b, len(seq))
                seq.append(t)  # teacher forcing on the GPU's history
    model.close()


# Fewer prompt rows (max_batch * ctx_len) than the skinny decode kernels' 16 K-blocked rows
SMALLCTX = dict(d_model=128, n_layers=2, n_heads=4, d_ff=512, ctx_len=8, vocab_size=512)


@pytest.mark.gpu
def test_generate_short_context_single_row_matches_oracle(gpu):
    """max_batch 1 and ctx_len 8: the decode step's final LayerNorm writes, and the skinny
    logits projection reads, 16 K-blocked rows of the LayerNorm output buffer whatever the
    batch (it is allocated for max(rows, 16)); teacher-forced against the oracle."""
    cfg = SMALLCTX
    case("generate vs oracle, ctx_len 8, max_batch 1")
    model, params = _gpu_model(cfg, seed=29, max_batch=1)
    prompt = _prompts(cfg, [3], 1200)[0]
    new = 5
    out = model.generate([prompt], new, logits=True)
    seq = list(prompt)
    for t in range(new):
        ref = G.forward(params, cfg, seq, round_bf16=True)[-1]
        got = out["logits"][t, 0]
        assert np.abs(got - ref).max() <= TOL_LOGIT, (t, np.abs(got - ref).max())
        assert out["tokens"][0, t] == int(np.argmax(got))
        seq.append(int(out["tokens"][0, t]))
    # to the context: the same 5 picks
    assert model.generate_tokens([prompt], 100)[0] == [int(t) for t in seq]
    model.close()


TOL_ATTN_LOGIT = 5e-2  # logits, bf16 vs fp32 attention, same history (observed 1.3e-2)


def first_divergence(a, b):
    """Per row, the first step where two token arrays differ (or their length)."""
    out = []
    for ra, rb in zip(a, b):
        d = np.nonzero(ra != rb)[0]
        out.append(int(d[0]) if len(d) else len(ra))
    return out


@pytest.mark.gpu
def test_gpt2_124m_bf16_attention_matches_fp32_attention(gpu):
    """GPT-2 124M shape, random init: bf16 attention against fp32 attention, everything else
    identical. While a row's history is the same in both runs (up to and including its first
    differing pick) the logits agree within TOL_ATTN_LOGIT; a pick can only differ where the
    top-1/top-2 margin is below twice that difference (random-init margins go down to ~1e-4),
    after which the histories differ and the rows are no longer comparable."""
    import torch

    from dadgpt_amd import gpt2

    case("gpt2-124m bf16 vs fp32 attention, 4 prompts x 24 tokens")
    params = gpt2.init_params(GPT2, 0x5EED)
    m16 = gpt2.GPT2(GPT2, params, 4, attention="bf16")
    m32 = gpt2.GPT2(GPT2, params, 4, attention="fp32")
    prompts = _prompts(GPT2, [16, 100, 37, 256], 600)
    a = m16.generate(prompts, 24, logits=True)
    b = m32.generate(prompts, 24, logits=True)
    div = first_divergence(a["tokens"], b["tokens"])
    worst = 0.0
    for r, t_div in enumerate(div):
        for t in range(min(t_div + 1, 24)):
            dev_t = float(np.abs(a["logits"][t, r] - b["logits"][t, r]).max())
            worst = max(worst, dev_t)
            assert dev_t <= TOL_ATTN_LOGIT, (r, t, dev_t)
        if t_div < 24:
            print(f"[gpt2] row {r} diverges at step {t_div}: margins bf16 "
                  f"{a['margins'][r, t_div]:.3g} fp32 {b['margins'][r, t_div]:.3g}", flush=True)
    print(f"[gpt2] identical prefix per row {div}; max logit difference on shared history "
          f"{worst:.3g}; min margin fp32 {b['margins'].min():.3g}", flush=True)
    m16.close()
    m32.close()
    torch.cuda.synchronize()


TOL_FP32_PATHS = 1e-3  # logits, fp32 flash vs fp32 materialized, fp32 projections, same history
GATE_MARGIN = 1e-4     # greedy gate: fp32 picks must agree wherever the margin exceeds this


def _shared_history_check(a, b, tol, label):
    """Rows of two runs of the same prompts: while a row's history is shared (up to and
    including its first differing pick) the logits agree within tol, and a differing pick
    falls where the reference run's top-1/top-2 margin is within twice the measured logit
    difference. Returns (first divergence per row, max logit difference, margins there)."""
    div = first_divergence(a["tokens"], b["tokens"])
    n_new = a["tokens"].shape[1]
    worst, at_div = 0.0, []
    for r, t_div in enumerate(div):
        for t in range(min(t_div + 1, n_new)):
            dev_t = float(np.abs(a["logits"][t, r] - b["logits"][t, r]).max())
            worst = max(worst, dev_t)
            assert dev_t <= tol, (label, r, t, dev_t)
        if t_div < n_new:
            dev_d = float(np.abs(a["logits"][t_div, r] - b["logits"][t_div, r]).max())
            margin = float(b["margins"][r, t_div])
            at_div.append(margin)
            assert margin <= 2 * dev_d, (label, r, t_div, margin, dev_d)
    print(f"[cfg5] {label}: rows identical {sum(d == n_new for d in div)}/{len(div)}, first "
          f"divergence {div}, max logit difference on shared history {worst:.3g}, reference "
          f"margins at divergences {[round(m, 6) for m in at_div]}", flush=True)
    return div, worst, at_div


@pytest.mark.gpu
def test_cfg5_generation_workload(gpu):
    """BASELINE config 5 at its real workload: GPT-2 124M architecture, random init, the 16
    prompts of U[16, 256] tokens, 128 greedy steps, max_batch 16 (with bf16 projections the
    decode step runs the skinny M = 16 kernels and replays as a captured graph). Four models
    over the same weights:
      bf16        bf16 attention, bf16 projections (the product);
      fp32        fp32 flash attention, bf16 projections (everything else as the product);
      fp32/fp32   fp32 flash attention, fp32 projections (the reference's precision);
      mat/fp32    fp32 materialized attention, fp32 projections (the reference's other
                  attention path: the GPU's own fp32 reference).

    - KV-cache invariant for every model (tests/test_model.cpp:216-252,375-414): decode-step
      logits at steps 1, 64 and 127 equal the prefill of the prompt extended by the generated
      tokens, for all 16 rows: within 2.5e-2 with bf16 projections, 1e-3 with fp32 ones. A bf16
      projection input is an fp32 activation rounded once; prefill (hipBLASLt) and decode
      (skinny kernels) compute those activations in different orders, and a one-ulp bf16 flip
      (2^-8 relative) carries through 12 layers (measured 1.0-1.4e-2).
    - bf16 vs fp32 attention (bf16 projections): logits within 5e-2 on shared history; a
      token may differ only at a near-tie (fp32 margin within twice the logit difference).
      The same bf16 rounding of projection inputs limits how closely any two attention
      implementations can agree under bf16 projections (~1e-2).
    - The greedy gate between the two fp32 attention paths with fp32 projections: logits within
      1e-3 on shared history, tokens identical wherever the fp32 margin exceeds 1e-4 (and
      twice the measured difference)."""
    import torch

    from dadgpt_amd import gpt2

    params = gpt2.init_params(GPT2, synth.CFG5_SEED)
    prompts = synth.cfg5_prompts(GPT2["vocab_size"])
    n_new = synth.CFG5_NEW
    runs = {}
    for name, attention, projections, kv_tol in (
            ("bf16", "bf16", "bf16", 2.5e-2), ("fp32", "fp32", "bf16", 2.5e-2),
            ("fp32/fp32", "fp32", "fp32", 1e-3), ("mat/fp32", "fp32_materialized", "fp32", 1e-3)):
        case(f"cfg5: 16 prompts x {n_new} greedy tokens, {attention} attention, {projections} "
             f"projections")
        m = gpt2.GPT2(GPT2, params, synth.CFG5_N, attention=attention, projections=projections)
        out = m.generate(prompts, n_new, logits=True)
        errs = []
        for t in (1, 64, n_new - 1):
            longer = [list(p) + list(out["tokens"][b, :t]) for b, p in enumerate(prompts)]
            again = m.generate(longer, 1, logits=True)
            errs.append(float(np.abs(again["logits"][0] - out["logits"][t]).max()))
        print(f"[cfg5] {name}: decode vs prefill logits at steps 1, 64, 127: "
              f"{[float(f'{e:.3g}') for e in errs]}", flush=True)
        assert max(errs) <= kv_tol, (name, errs)
        m.close()
        runs[name] = out
    _shared_history_check(runs["bf16"], runs["fp32"], TOL_ATTN_LOGIT, "bf16 vs fp32 attention")
    _, _, at_div = _shared_history_check(runs["fp32/fp32"], runs["mat/fp32"], TOL_FP32_PATHS,
                                         "fp32 flash vs fp32 materialized (fp32 projections)")
    assert all(m <= GATE_MARGIN for m in at_div), at_div
    for name, r in runs.items():
        print(f"[cfg5] {name}: min margin {r['margins'].min():.3g}", flush=True)
    del params
    torch.cuda.synchronize()
