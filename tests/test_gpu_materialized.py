"""GPU tests of the hipBLASLt layer and the materialized attention path.

- The hipBLASLt behind a handle is the version the library was compiled against, also in a
  process that imported PyTorch first (PyTorch bundles an older libhipblaslt.so.1).
- fp32 GEMMs in the reference's three row-major forms (cuda/gpu_ops.cu:94-112) and its three
  strided-batched forms (:117-141), against float64 products on the host; the BF16 precision
  against products of bf16-rounded inputs; the reference-named C++ symbols; the bf16 GEMM at a
  training step's 16,384 rows.
- The materialized attention forward/backward (src/model.cpp:395-420, 575-616) against the
  golden vectors of the reference's own CPU operators, the CPU oracle, and the fp32 flash
  kernels; its row operators against float64 closed forms.
"""
import ctypes
import math
import os
import re
import subprocess

import numpy as np
import pytest
import torch

import oracle
from dadgpt_amd import attention as A
from dadgpt_amd import gpt2
from dadgpt_amd import synth

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOL_F32 = 1e-5


def case(msg):
    print(f"[case] {msg}", flush=True)


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to("cuda")


def host(t):
    return t.float().cpu().numpy()


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def compiled_hipblaslt_version():
    text = open("/opt/rocm/include/hipblaslt/hipblaslt-version.h").read()
    v = {k: int(re.search(rf"HIPBLASLT_VERSION_{k}\s+(\d+)", text).group(1))
         for k in ("MAJOR", "MINOR", "PATCH")}
    return v["MAJOR"] * 100000 + v["MINOR"] * 100 + v["PATCH"]


@pytest.fixture(scope="module")
def blas(gpu):
    h = gpt2.Blas()
    yield h
    h.close()


def test_hipblaslt_is_the_compiled_version(blas):
    case("hipBLASLt version behind the handle")
    assert "torch" in __import__("sys").modules  # PyTorch (with its own hipBLASLt) came first
    assert blas.library_version() == compiled_hipblaslt_version()
    maps = open("/proc/self/maps").read()
    assert re.search(r"/opt/rocm[^\s]*/lib/libhipblaslt\.so", maps), "private copy not mapped"


def _ref_gemm(a, b, op):
    a, b = a.astype(np.float64), b.astype(np.float64)
    if op == "A":
        return a.T @ b
    if op == "B":
        return a @ b.T
    return a @ b


def _operands(M, K, N, op, seed):
    a = synth.normal((K, M) if op == "A" else (M, K), seed)
    b = synth.normal((N, K) if op == "B" else (K, N), seed + 1)
    return a, b


def _gemm_tol(K, ref):
    # fp32 products summed over K: a few ulp of the largest partial sum per term
    return 4e-7 * math.sqrt(K) * max(1.0, float(np.abs(ref).max())) * 8


@pytest.mark.parametrize("op", ["N", "A", "B"])
@pytest.mark.parametrize("M,K,N", [(64, 96, 80), (1, 64, 1024), (300, 768, 2304), (7, 3, 5)])
def test_matmul_f32_against_float64(blas, op, M, K, N):
    case(f"matmul f32 op={op} M={M} K={K} N={N}")
    a, b = _operands(M, K, N, op, 100 + M + K)
    ref = _ref_gemm(a, b, op)
    out = torch.empty(M, N, device="cuda")
    blas.matmul_f32(out, dev(a), dev(b), M, K, N, op)
    torch.cuda.synchronize()
    assert max_abs(host(out), ref) <= _gemm_tol(K, ref)
    if op == "A":  # gpu_matmul_transposed_a(accumulate = true): out += a^T b
        blas.matmul_f32(out, dev(a), dev(b), M, K, N, op, beta=1.0)
        torch.cuda.synchronize()
        assert max_abs(host(out), 2 * ref) <= 2 * _gemm_tol(K, ref)


@pytest.mark.parametrize("op,beta", [("B", 0.0), ("N", 0.0), ("A", 1.0)])
def test_matmul_f32_strided_batched(blas, op, beta):
    """Each of the reference's batched forms, with strides larger than a matrix (padding
    between matrices must be left alone)."""
    M, K, N, count = 33, 40, 20, 5
    case(f"batched op={op} beta={beta}")
    a1, b1 = _operands(M, K, N, op, 200)
    sa, sb, sc = a1.size + 8, b1.size + 16, M * N + 4
    a = synth.normal((count * sa,), 210).astype(np.float32)
    b = synth.normal((count * sb,), 211).astype(np.float32)
    c0 = synth.normal((count * sc,), 212).astype(np.float32)
    out = dev(c0)
    blas.matmul_f32_batched(out, dev(a), dev(b), M, K, N, op, beta, sa, sb, sc, count)
    torch.cuda.synchronize()
    got = host(out)
    for i in range(count):
        ai = a[i * sa:i * sa + a1.size].reshape(a1.shape)
        bi = b[i * sb:i * sb + b1.size].reshape(b1.shape)
        ref = _ref_gemm(ai, bi, op) + beta * c0[i * sc:i * sc + M * N].reshape(M, N)
        gi = got[i * sc:i * sc + M * N].reshape(M, N)
        assert max_abs(gi, ref) <= 2 * _gemm_tol(K, ref), i
        assert np.array_equal(got[i * sc + M * N:(i + 1) * sc], c0[i * sc + M * N:(i + 1) * sc])


def test_matmul_precision_bf16(blas):
    """MatmulPrecision::BF16 rounds the inputs to bfloat16 and accumulates in fp32
    (CUBLAS_COMPUTE_32F_FAST_16BF, cuda/gpu_ops.cu:63-67): the result matches the fp32 product
    of the rounded inputs, not the exact one. TF32 runs as FP32 on gfx950."""
    M, K, N = 128, 512, 96
    case("matmul precision bf16 / tf32")
    a, b = _operands(M, K, N, "N", 300)
    ref_exact = _ref_gemm(a, b, "N")
    ref_bf16 = _ref_gemm(synth.bf16_round(a), synth.bf16_round(b), "N")
    out = torch.empty(M, N, device="cuda")
    try:
        gpt2.set_matmul_precision("bf16")
        assert gpt2.get_matmul_precision() == "bf16"
        blas.matmul_f32(out, dev(a), dev(b), M, K, N, "N")
        torch.cuda.synchronize()
        err_rounded, err_exact = max_abs(host(out), ref_bf16), max_abs(host(out), ref_exact)
        assert err_rounded <= _gemm_tol(K, ref_bf16)
        assert err_exact > 20 * err_rounded, (err_exact, err_rounded)
        gpt2.set_matmul_precision("tf32")
        blas.matmul_f32(out, dev(a), dev(b), M, K, N, "N")
        torch.cuda.synchronize()
        assert max_abs(host(out), ref_exact) <= _gemm_tol(K, ref_exact)
    finally:
        gpt2.set_matmul_precision("fp32")
    assert gpt2.get_matmul_precision() == "fp32"


def test_reference_named_matmul_symbols(blas):
    """gpu_matmul / _transposed_a / _transposed_b / _strided_batched_bt by their C++ names
    (include/dadgpt/gpu_ops_matmul.hpp) run the same GEMMs."""
    case("gpu_matmul* C++ symbols")
    L = gpt2.gen_lib()
    vp, i = ctypes.c_void_p, ctypes.c_int
    fns = {}
    for name, extra in (("_Z10gpu_matmulP11dadgpt_blasPfPKfS3_iii", []),
                        ("_Z23gpu_matmul_transposed_aP11dadgpt_blasPfPKfS3_iiib", [ctypes.c_bool]),
                        ("_Z23gpu_matmul_transposed_bP11dadgpt_blasPfPKfS3_iii", [])):
        f = getattr(L, name)
        f.argtypes = [vp] * 4 + [i, i, i] + extra
        f.restype = None
        fns[name] = f
    M, K, N = 50, 70, 30
    for name, op in zip(fns, "NAB"):
        a, b = _operands(M, K, N, op, 400 + ord(op))
        out = torch.empty(M, N, device="cuda")
        da, db = dev(a), dev(b)
        torch.cuda.synchronize()
        args = [blas._h, out.data_ptr(), da.data_ptr(), db.data_ptr(), M, K, N]
        fns[name](*(args + ([False] if op == "A" else [])))
        torch.cuda.synchronize()
        ref = _ref_gemm(a, b, op)
        assert max_abs(host(out), ref) <= _gemm_tol(K, ref), name
    bt = getattr(L, "_Z29gpu_matmul_strided_batched_btP11dadgpt_blasPfPKfS3_iiixxxi")
    ll = ctypes.c_longlong
    bt.argtypes = [vp] * 4 + [i, i, i, ll, ll, ll, i]
    bt.restype = None
    q = synth.normal((3, 20, 16), 450)
    k = synth.normal((3, 24, 16), 451)
    out = torch.empty(3, 20, 24, device="cuda")
    dq, dk = dev(q), dev(k)
    torch.cuda.synchronize()
    bt(blas._h, out.data_ptr(), dq.data_ptr(), dk.data_ptr(), 20, 16, 24, 320, 384, 480, 3)
    torch.cuda.synchronize()
    ref = np.einsum("bik,bjk->bij", q.astype(np.float64), k.astype(np.float64))
    assert max_abs(host(out), ref) <= _gemm_tol(16, ref)


def test_matmul_bf16_training_rows(blas):
    """The bf16 projection GEMM at a training step's rows (B16 x T1024 = 16,384 rows, the
    QKV shape K 768, N 2304) against torch's fp32 product on the GPU."""
    M, K, N = 16384, 768, 2304
    case(f"matmul bf16 M={M} K={K} N={N} (hipBLASLt {blas.library_version()})")
    assert blas.library_version() == compiled_hipblaslt_version()
    g = torch.Generator(device="cuda").manual_seed(5)
    a = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    b = (torch.randn(K, N, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    out = blas.matmul(a, b)
    ref = a.float() @ b.float()
    torch.cuda.synchronize()
    assert float((out - ref).abs().max()) <= 1e-4 * math.sqrt(K)


# ------------------------------------------------------------------ materialized attention

def _materialized(blas, qn, kn, vn, gn, scale):
    BH, S, D = qn.shape
    q, k, v, g = dev(qn), dev(kn), dev(vn), dev(gn)
    out = torch.empty_like(q)
    probs = torch.empty(BH, S, S, device="cuda")
    blas.attention_materialized_forward(out, probs, q, k, v, BH, S, D, scale)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    ds = torch.empty(BH, S, S, device="cuda")
    blas.attention_materialized_backward(dq, dk, dv, ds, g, probs, q, k, v, BH, S, D, scale)
    torch.cuda.synchronize()
    return host(out), host(probs), host(dq), host(dk), host(dv)


@pytest.mark.parametrize("name", ["cfg1_fwd_bwd.npz", "ragged70_fwd_bwd.npz"])
def test_materialized_golden(blas, golden_dir, name):
    z = np.load(os.path.join(golden_dir, name))
    BH, S, D = z["q"].shape
    case(f"materialized golden {name} BH={BH} S={S} D={D}")
    out, probs, dq, dk, dv = _materialized(blas, z["q"], z["k"], z["v"], z["dout"],
                                           float(z["scale"][0]))
    assert max_abs(out, z["o"]) <= TOL_F32
    for got, key in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert max_abs(got, z[key]) <= TOL_F32, key
    assert np.all(np.triu(probs, 1) == 0.0)  # masked probabilities are exactly zero
    assert np.abs(probs.sum(-1) - 1.0).max() <= 1e-5


@pytest.mark.parametrize("BH,S,D", [(2, 1024, 64), (3, 129, 32), (1, 1, 64), (2, 70, 48)])
def test_materialized_against_oracle(blas, BH, S, D):
    case(f"materialized vs oracle BH={BH} S={S} D={D}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=600 + S + D, with_dout=True)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    out, _, dq, dk, dv = _materialized(blas, qn, kn, vn, gn, scale)
    o_ref, _ = oracle.attn_fwd(qn, kn, vn, scale)
    dq_r, dk_r, dv_r, _ = oracle.attn_bwd(gn, qn, kn, vn, scale)
    assert max_abs(out, o_ref) <= TOL_F32
    for a, b in ((dq, dq_r), (dk, dk_r), (dv, dv_r)):
        assert max_abs(a, b) <= TOL_F32


def test_materialized_matches_fused_fp32(blas):
    """The two fp32 paths the reference chooses between agree (the reference's own
    FusedAttentionMatchesMaterialized, tests/test_backward.cpp:432-480, at 1e-4; here 1e-5)."""
    BH, S, D = 8, 512, 64
    case(f"materialized vs fused fp32 BH={BH} S={S}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=700, with_dout=True)
    scale = 0.125
    out, _, dq, dk, dv = _materialized(blas, qn, kn, vn, gn, scale)
    q, k, v, g = dev(qn), dev(kn), dev(vn), dev(gn)
    fo, lse = A.attention_forward(q, k, v, scale)
    fdq, fdk, fdv, _ = A.attention_backward(g, fo, lse, q, k, v, scale)
    torch.cuda.synchronize()
    assert max_abs(out, host(fo)) <= TOL_F32
    for a, b in ((dq, fdq), (dk, fdk), (dv, fdv)):
        assert max_abs(a, host(b)) <= TOL_F32


def _materialized_dropout(blas, qn, kn, vn, gn, scale, p, seed):
    BH, S, D = qn.shape
    q, k, v, g = dev(qn), dev(kn), dev(vn), dev(gn)
    out = torch.empty_like(q)
    probs = torch.empty(BH, S, S, device="cuda")
    dropped = torch.empty(BH, S, S, device="cuda")
    blas.attention_materialized_forward_dropout(out, probs, dropped, q, k, v, BH, S, D, scale, p,
                                                seed)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    ds = torch.empty(BH, S, S, device="cuda")
    blas.attention_materialized_backward_dropout(dq, dk, dv, ds, g, probs, q, k, v, BH, S, D,
                                                 scale, p, seed)
    torch.cuda.synchronize()
    return host(out), host(probs), host(dropped), host(dq), host(dk), host(dv)


@pytest.mark.parametrize("BH,S,D,p", [(2, 70, 64, 0.1), (3, 129, 32, 0.5), (2, 256, 64, 0.25),
                                      (1, 1, 64, 0.3), (2, 64, 48, 0.9)])
def test_materialized_dropout_against_oracle(blas, BH, S, D, p):
    """The materialized path with attention dropout (src/model.cpp:406-416, 594-599), the one
    use_fused_attention picks for dropout: O and dQ/dK/dV against the oracle's dropout path
    (the same keep mask, the materialized op order) at the fp32 tolerance; the dropped
    probabilities are exactly probs * keep * 1/(1-p) with the oracle's mask."""
    seed = 0x5EED_0000_0000_0000 + 97 * S + D
    case(f"materialized dropout vs oracle BH={BH} S={S} D={D} p={p}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=650 + S + D, with_dout=True)
    scale = float(np.float32(1.0 / math.sqrt(D)))
    out, probs, dropped, dq, dk, dv = _materialized_dropout(blas, qn, kn, vn, gn, scale, p, seed)
    keep = oracle.dropout_mask(BH, S, seed, p).astype(bool)
    # the keep factor in fp32, as the reference's 1.0f / (1.0f - rate) (cuda/gpu_ops.cu:719)
    factor = np.float32(1.0) / (np.float32(1.0) - np.float32(p))
    want = np.where(keep, probs * factor, np.float32(0.0))
    assert np.array_equal(dropped, want.astype(np.float32))
    o_ref, _ = oracle.attn_fwd_dropout(qn, kn, vn, scale, p, seed)
    dq_r, dk_r, dv_r, _ = oracle.attn_bwd_dropout(gn, qn, kn, vn, scale, p, seed)
    tol = TOL_F32 / (1.0 - p)  # the values carry the factor 1/(1-p)
    assert max_abs(out, o_ref) <= tol
    for a, b, nm in ((dq, dq_r, "dq"), (dk, dk_r, "dk"), (dv, dv_r, "dv")):
        assert max_abs(a, b) <= tol, nm


def test_materialized_dropout_matches_flash_dropout_and_p0(blas):
    """With the same seed and rate the materialized and the fp32 flash dropout paths drop the
    same probabilities (one mask definition): outputs and gradients agree at 1e-5. At p = 0 the
    dropout path's forward (O and the probabilities) equals the plain materialized path bit for
    bit; its gradients agree at 1e-5 (the dropout row pass sums each row's dP.P in 8-column
    groups, the plain one in 64-column strides: another fp32 summation order)."""
    BH, S, D, p, seed = 4, 300, 64, 0.2, 1234567
    case(f"materialized dropout vs flash fp32 dropout BH={BH} S={S}")
    qn, kn, vn, gn = synth.attn_inputs(BH, S, D, seed=710, with_dout=True)
    scale = 0.125
    out, _, _, dq, dk, dv = _materialized_dropout(blas, qn, kn, vn, gn, scale, p, seed)
    q, k, v, g = dev(qn), dev(kn), dev(vn), dev(gn)
    fo = torch.empty_like(q)
    lse = torch.empty(BH, S, device="cuda")
    A.flash_attention_forward_dropout(fo, lse, q, k, v, BH, S, D, scale, p, seed)
    fdq, fdk, fdv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    delta = torch.empty_like(lse)
    A.flash_attention_backward_dropout(fdq, fdk, fdv, delta, g, fo, lse, q, k, v, BH, S, D, scale,
                                       p, seed)
    torch.cuda.synchronize()
    assert max_abs(out, host(fo)) <= TOL_F32 / (1 - p)
    for a, b in ((dq, fdq), (dk, fdk), (dv, fdv)):
        assert max_abs(a, host(b)) <= TOL_F32 / (1 - p)
    plain = _materialized(blas, qn, kn, vn, gn, scale)
    zero = _materialized_dropout(blas, qn, kn, vn, gn, scale, 0.0, seed)
    assert np.array_equal(plain[0], zero[0]) and np.array_equal(plain[1], zero[1])
    assert np.array_equal(zero[1], zero[2])  # nothing dropped, factor exactly 1
    for a, b in zip(plain[2:], zero[3:]):
        assert max_abs(a, b) <= TOL_F32


def _softmax64(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


@pytest.mark.parametrize("rows,cols", [(6, 1), (5, 64), (4, 70), (9, 1024), (3, 2500)])
def test_reference_row_operators(gpu, rows, cols):
    """gpu_softmax, gpu_softmax_backward (accumulating), gpu_scale by the C ABI and their C++
    names, against float64 closed forms."""
    case(f"row operators rows={rows} cols={cols}")
    x = synth.normal((rows, cols), 800 + cols) * 3
    g = synth.normal((rows, cols), 801 + cols)
    d0 = synth.normal((rows, cols), 802 + cols)
    out = torch.empty(rows, cols, device="cuda")
    A.softmax(out, dev(x), rows, cols)
    inplace = dev(x)
    A.softmax(inplace, inplace, rows, cols)
    din = dev(d0)
    A.softmax_backward(din, dev(g), out, rows, cols)
    sc = dev(x)
    A.scale_(sc, 0.375)
    torch.cuda.synchronize()
    p = _softmax64(x)
    assert max_abs(host(out), p) <= 1e-6
    assert np.array_equal(host(inplace), host(out))
    pf = host(out).astype(np.float64)
    want = d0 + pf * (g - (g * pf).sum(-1, keepdims=True))
    assert max_abs(host(din), want) <= 1e-5
    assert np.array_equal(host(sc), (x.astype(np.float32) * np.float32(0.375)))
    # the reference-named symbol of gpu_softmax
    f = getattr(A.lib(), "_Z11gpu_softmaxPfPKfii")
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    f.restype = None
    o2 = torch.empty_like(out)
    xin = dev(x)
    torch.cuda.synchronize()
    f(o2.data_ptr(), xin.data_ptr(), rows, cols)
    torch.cuda.synchronize()
    assert np.array_equal(host(o2), host(out))


def test_causal_mask_and_fused_probs(gpu):
    """gpu_causal_mask / _zero, and the fused probability kernels against the unfused chain
    of the reference's operators (scale, mask, softmax; softmax backward, zero, scale)."""
    BH, S, scale = 3, 77, 0.2
    case(f"mask + fused probs BH={BH} S={S}")
    s = synth.normal((BH, S, S), 900) * 4
    gp = synth.normal((BH, S, S), 901)
    m = dev(s)
    A.causal_mask(m, BH, S)
    z = dev(s)
    A.causal_mask(z, BH, S, zero=True)
    torch.cuda.synchronize()
    up = np.triu(np.ones((S, S), bool), 1)
    assert np.all(host(m)[:, up] == np.float32(-1e9)) and np.array_equal(host(m)[:, ~up],
                                                                          s[:, ~up])
    assert np.all(host(z)[:, up] == 0.0) and np.array_equal(host(z)[:, ~up], s[:, ~up])
    # unfused chain on the GPU's own operators
    chain = dev(s)
    A.scale_(chain, scale)
    A.causal_mask(chain, BH, S)
    A.softmax(chain, chain, BH * S, S)
    fused = dev(s)
    A.attention_probs(fused, BH, S, scale)
    dchain = torch.zeros(BH, S, S, device="cuda")
    A.softmax_backward(dchain, dev(gp), chain, BH * S, S)
    A.causal_mask(dchain, BH, S, zero=True)
    A.scale_(dchain, scale)
    dfused = dev(gp)
    A.attention_probs_backward(dfused, dfused, fused, BH, S, scale)
    torch.cuda.synchronize()
    assert max_abs(host(fused), host(chain)) <= 1e-7
    assert max_abs(host(dfused), host(dchain)) <= 1e-6


def test_decode_probs_and_materialized_decode(gpu):
    """The length-masked decode softmax: probabilities over each sequence's first lens keys,
    zero past them; an empty cache gives a zero row."""
    n, H, L, scale = 4, 3, 300, 0.125
    case(f"decode probs n={n} H={H} max_len={L}")
    s = synth.normal((n * H, L), 950) * 5
    lens = np.array([1, 300, 0, 137], np.int32)
    p = dev(s)
    A.decode_probs(p, torch.from_numpy(lens).to("cuda"), n, H, L, scale)
    torch.cuda.synchronize()
    got = host(p)
    for r in range(n * H):
        Ls = lens[r // H]
        if Ls == 0:
            assert np.all(got[r] == 0.0)
            continue
        want = _softmax64(s[r, :Ls].astype(np.float32) * np.float32(scale))
        assert max_abs(got[r, :Ls], want) <= 1e-6
        assert np.all(got[r, Ls:] == 0.0)


def _split_np(x, B, S, H, dh):
    """[B*S, H*dh] -> [B*H, S, dh] by index arithmetic (cuda/gpu_ops.cu:426-446)."""
    return x.reshape(B, S, H, dh).transpose(0, 2, 1, 3).reshape(B * H, S, dh)


@pytest.mark.parametrize("B,S,H,dh", [(16, 1024, 12, 64), (2, 7, 3, 32), (1, 5, 4, 3),
                                      (3, 33, 12, 64)])
def test_split_merge_heads_reference_symbols(gpu, B, S, H, dh):
    """gpu_split_heads / gpu_merge_heads under their mangled reference names
    (cuda/gpu_ops.cuh:98-104), null stream: bit-exact against the numpy permutation, the
    merge inverts the split, and the C ABI on a stream gives the same bits. (1, 5, 4, 3) has
    d_head not a multiple of 4 (the one-float path); (3, 33, 12, 64) is also run from an input
    4 bytes past a 16-byte boundary (the one-float path with d_head 64)."""
    case(f"split/merge heads B={B} S={S} H={H} dh={dh}")
    L = A.lib()
    fns = {}
    for key, name in (("split", "_Z15gpu_split_headsPfPKfiiii"),
                      ("merge", "_Z15gpu_merge_headsPfPKfiiii")):
        f = getattr(L, name)
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 4
        f.restype = None
        fns[key] = f
    n = B * S * H * dh
    x = synth.normal((n,), 950 + dh)
    want = _split_np(x, B, S, H, dh)
    for off in ((0, 1) if (B, S) == (3, 33) else (0,)):
        src = torch.from_numpy(np.concatenate([np.zeros(off, np.float32), x])).to("cuda")
        xin = src[off:]
        heads = torch.full((n,), -7.0, device="cuda")
        back = torch.full((n,), -7.0, device="cuda")
        torch.cuda.synchronize()
        fns["split"](heads.data_ptr(), xin.data_ptr(), B, S, H, dh)
        fns["merge"](back.data_ptr(), heads.data_ptr(), B, S, H, dh)
        torch.cuda.synchronize()
        assert np.array_equal(host(heads).reshape(B * H, S, dh), want), off
        assert np.array_equal(host(back), x), off
    h2 = torch.empty(n, device="cuda")
    b2 = torch.empty(n, device="cuda")
    A.split_heads(h2, dev(x), B, S, H, dh)
    A.merge_heads(b2, h2, B, S, H, dh)
    torch.cuda.synchronize()
    assert np.array_equal(host(h2).reshape(B * H, S, dh), want)
    assert np.array_equal(host(b2), x)


def test_blas_stack_in_this_process(gpu):
    """The Python test process runs PyTorch's HIP 7.0 runtime under the compiled hipBLASLt: the
    pair every other GPU test here exercises, and one dadgpt_blas_create accepts."""
    v = gpt2.blas_stack_versions()
    case(f"blas stack {v}")
    assert v["supported"] and v["hip_runtime"] // 100000 == 700, v


def test_blas_stack_cxx_caller_on_rocm_runtime(gpu, tmp_path):
    """A C++ caller without PyTorch (tests/cxx/blas_stack_test.cpp): the ROCm installation's
    7.2 HIP runtime with the same hipBLASLt; the pair is accepted, a handle is created and a
    bf16 GEMM matches the CPU product."""
    case("blas stack C++ caller on the ROCm runtime")
    libdir = os.path.join(ROOT, "dadgpt_amd", "lib")
    exe = str(tmp_path / "blas_stack_test")
    subprocess.run(["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    f"-I{ROOT}/include", os.path.join(ROOT, "tests", "cxx", "blas_stack_test.cpp"),
                    f"-L{libdir}", "-ldadgpt_gen", "-ldadgpt_attn", "-L/opt/rocm/lib",
                    "-lamdhip64", f"-Wl,-rpath,{libdir}", "-Wl,-rpath,/opt/rocm/lib", "-o", exe],
                   check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout + r.stderr
