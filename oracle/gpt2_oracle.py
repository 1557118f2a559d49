"""CPU oracle of the GPT-2 generation path — TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py`` import this module, as the checker. The product
(``dadgpt_amd.gpt2``, ``libdadgpt_gen.so``) never imports or calls it.

A numpy fp32 restatement of the reference's model forward for one sequence
(``src/model.cpp:334-475`` with batch 1): embedding + positional (``:347-348``), per layer
LayerNorm -> Q, K, V projections + bias -> causal attention -> Wo + bias -> residual ->
LayerNorm -> fc1 + bias -> GELU (tanh form) -> fc2 + bias -> residual, final LayerNorm and
the weight-tied logits (``:472``). The parameter arena has the reference's layout
(``src/model.cpp:17-56``). Attention is the materialized fp32 path (softmax of the scaled,
-1e9-masked scores), as ``oracle.attn_fwd``.

Greedy generation here recomputes the whole sequence at every step (no cache): the cached
decode of the product must equal it, which is the reference's own KV-cache invariant
(``tests/test_model.cpp:216-252`` KVCacheMatchesFullForward).

``round_bf16=True`` rounds to bf16 exactly where the product feeds bf16 into a GEMM or into
attention (LayerNorm outputs, Q/K/V, the attention output, the GELU output), so the remaining
difference is accumulation order only.

Pinning: ``layernorm``, ``gelu`` and the whole ``forward`` are checked in
``tests/test_x_generate.py`` against the reference's own CPU operators
(``src/tensor_ops.cpp:6-123`` compiled into ``oracle/_ref``) composed in the order of
``model_forward``. ``truncate_prompt`` and ``generate_tokens`` restate
``src/generate.cpp:94-139`` (which does not compile here: it needs the CUDA model and
``<format>``); the same tests pin them by hand-worked cases of the reference's index arithmetic
and by invariants (the first token and a suffix survive truncation; a stop token cuts the
no-stop continuation at its first occurrence).
"""
from __future__ import annotations

import numpy as np

from dadgpt_amd import synth


def offsets(cfg: dict) -> dict:
    """Element offsets of the reference's parameter arena (src/model.cpp:17-56)."""
    d, dff, V, ctx, L = (cfg["d_model"], cfg["d_ff"], cfg["vocab_size"], cfg["ctx_len"],
                         cfg["n_layers"])
    at = 0
    out = {}

    def take(name, n):
        nonlocal at
        out[name] = (at, n)
        at += n

    take("tok_emb", V * d)
    take("pos_emb", ctx * d)
    for l in range(L):
        for nm, n in (("ln1_w", d), ("ln1_b", d), ("Wq", d * d), ("bq", d), ("Wk", d * d),
                      ("bk", d), ("Wv", d * d), ("bv", d), ("Wo", d * d), ("bo", d),
                      ("ln2_w", d), ("ln2_b", d), ("fc1_w", d * dff), ("fc1_b", dff),
                      ("fc2_w", dff * d), ("fc2_b", d)):
            take(f"{l}.{nm}", n)
    take("lnf_w", d)
    take("lnf_b", d)
    out["total"] = (at, 0)
    return out


def unpack(params: np.ndarray, cfg: dict) -> dict:
    """Views of a float32 arena, shaped (weights row-major [in, out])."""
    d, dff, V, ctx = cfg["d_model"], cfg["d_ff"], cfg["vocab_size"], cfg["ctx_len"]
    shapes = {"tok_emb": (V, d), "pos_emb": (ctx, d), "Wq": (d, d), "Wk": (d, d),
              "Wv": (d, d), "Wo": (d, d), "fc1_w": (d, dff), "fc2_w": (dff, d)}
    out = {}
    for name, (at, n) in offsets(cfg).items():
        if name == "total":
            continue
        key = name.split(".")[-1]
        view = params[at:at + n]
        out[name] = view.reshape(shapes[key]) if key in shapes else view
    return out


def layernorm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """Two-pass mean and variance, 1/sqrt(var + eps) (src/tensor_ops.cpp:57-84)."""
    x = x.astype(np.float32)
    mean = x.mean(axis=-1, keepdims=True, dtype=np.float32)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True, dtype=np.float32)
    inv = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    return ((x - mean) * inv * w + b).astype(np.float32)


def gelu(x: np.ndarray) -> np.ndarray:
    """tanh form (src/tensor_ops.cpp:86-95)."""
    x = x.astype(np.float32)
    inner = np.float32(0.7978845608) * (x + np.float32(0.044715) * x * x * x)
    return (np.float32(0.5) * x * (np.float32(1.0) + np.tanh(inner))).astype(np.float32)


def _attention(q, k, v, scale):
    """[H, S, dh] causal softmax attention, materialized fp32 (src/model.cpp:396-419)."""
    s = np.einsum("hqd,hkd->hqk", q, k, dtype=np.float32) * np.float32(scale)
    S = q.shape[1]
    s = np.where(np.triu(np.ones((S, S), bool), 1)[None], np.float32(-1e9), s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum("hqk,hkd->hqd", p, v, dtype=np.float32)


def forward(params: np.ndarray, cfg: dict, tokens, round_bf16: bool = False) -> np.ndarray:
    """Logits [S, V] float32 of one sequence (src/model.cpp:334-475, batch 1)."""
    P = unpack(np.asarray(params, np.float32), cfg)
    d, H, L = cfg["d_model"], cfg["n_heads"], cfg["n_layers"]
    dh = d // H
    rb = synth.bf16_round if round_bf16 else (lambda a: a)
    tokens = np.asarray(tokens, np.int64)
    S = len(tokens)
    x = (P["tok_emb"][tokens] + P["pos_emb"][:S]).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(dh))
    for l in range(L):
        g = lambda nm: P[f"{l}.{nm}"]
        h = rb(layernorm(x, g("ln1_w"), g("ln1_b")))
        q = rb(h @ g("Wq") + g("bq"))
        k = rb(h @ g("Wk") + g("bk"))
        v = rb(h @ g("Wv") + g("bv"))
        split = lambda t: t.reshape(S, H, dh).transpose(1, 0, 2)
        a = _attention(split(q), split(k), split(v), scale)
        a = rb(a.transpose(1, 0, 2).reshape(S, d))
        x = (x + (a @ g("Wo") + g("bo"))).astype(np.float32)
        h = rb(layernorm(x, g("ln2_w"), g("ln2_b")))
        f = rb(gelu(h @ g("fc1_w") + g("fc1_b")))
        x = (x + (f @ g("fc2_w") + g("fc2_b"))).astype(np.float32)
    h = rb(layernorm(x, P["lnf_w"], P["lnf_b"]))
    return (h @ P["tok_emb"].T).astype(np.float32)


def greedy(params, cfg, prompt, new_tokens: int, round_bf16: bool = False):
    """Greedy continuation by full recompute; returns (tokens, last-row logits per step)."""
    seq = list(int(t) for t in prompt)
    toks, rows = [], []
    for _ in range(new_tokens):
        row = forward(params, cfg, seq, round_bf16)[-1]
        t = int(np.argmax(row))  # first maximum, as std::max_element
        toks.append(t)
        rows.append(row)
        seq.append(t)
    return np.array(toks, np.int32), np.stack(rows)


def truncate_prompt(prompt, max_len: int, ctx_len: int) -> list:
    """The prompt truncation of generate_tokens (src/generate.cpp:97-110): the length limit is
    min(max_len, ctx_len); a prompt of at least that many tokens (and more than one) becomes
    its first token followed by its last max(limit - 2, 0) tokens."""
    limit = min(max_len, ctx_len)
    toks = [int(t) for t in prompt]
    if len(toks) >= limit and len(toks) > 1:
        keep = max(limit - 2, 0)
        return [toks[0]] + (toks[len(toks) - keep:] if keep else [])
    return toks


def generate_tokens(params, cfg, prompt, max_len: int, stop_token: int = -1,
                    round_bf16: bool = False) -> list:
    """generate_tokens (src/generate.cpp:94-139) with greedy sample_token (:34-37): truncate,
    then append the first maximum of the last row's logits until the sequence holds
    min(max_len, ctx_len) tokens or the pick is the stop token (kept). Returns the whole
    sequence, truncated prompt included."""
    limit = min(max_len, cfg["ctx_len"])
    seq = truncate_prompt(prompt, max_len, cfg["ctx_len"])
    while len(seq) < limit:
        t = int(np.argmax(forward(params, cfg, seq, round_bf16)[-1]))
        seq.append(t)
        if t == stop_token or len(seq) >= limit:
            break
    return seq
