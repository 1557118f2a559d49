"""CPU tests of the C ABI boundary: the library loads, exports every symbol the headers
declare, and rejects bad arguments on the host before any HIP call (no compute calls are
made here)."""
import ctypes
import os
import re
import subprocess

import pytest

from dadgpt_amd import attention as A

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dadgpt", "gpu_attention.h")
FAKE = 0x1000  # a non-null address; every call below fails validation before using it


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(dadgpt_\w+)\s*\(", text)))


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", A.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_header_and_binding_agree():
    assert header_functions() == sorted(A.C_SYMBOLS)


def test_library_exports_every_declared_symbol():
    syms = exported_symbols()
    missing = [s for s in A.C_SYMBOLS + A.CXX_SYMBOLS if s not in syms]
    assert not missing, missing
    L = A.lib()
    for s in A.C_SYMBOLS:
        assert hasattr(L, s)


def test_version_and_status_strings():
    L = A.lib()
    assert b"gfx950" in L.dadgpt_version()
    assert L.dadgpt_status_string(0) == b"ok"
    assert L.dadgpt_status_string(2) == b"unsupported"


def test_supported_predicate():
    assert A.flash_attention_supported(32) and A.flash_attention_supported(64)
    for d in (0, 16, 48, 80, 128, -64):
        assert not A.flash_attention_supported(d)


@pytest.mark.parametrize("fn", ["dadgpt_flash_attention_forward",
                                "dadgpt_flash_attention_forward_bf16"])
def test_forward_validation(fn):
    L = A.lib()
    f = getattr(L, fn)
    extra = [None] if fn.endswith("bf16") else []
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 48, 0.125, *extra) == 2
    assert A.last_error() == "flash attention: unsupported d_head 48"
    assert f(None, FAKE, FAKE, FAKE, FAKE, 4, 64, 64, 0.125, *extra) == 1
    assert "pointer argument 0 is null" in A.last_error()
    assert f(FAKE, FAKE, FAKE, FAKE, None, 4, 64, 64, 0.125, *extra) == 1
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 64, 64, 0.125, *extra) == 1
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 0, 64, 0.125, *extra) == 1
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 4, -3, 64, 0.125, *extra) == 1
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 64, float("nan"), *extra) == 1
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 64, float("inf"), *extra) == 1


@pytest.mark.parametrize("fn", ["dadgpt_flash_attention_backward",
                                "dadgpt_flash_attention_backward_bf16"])
def test_backward_validation(fn):
    f = getattr(A.lib(), fn)
    extra = [None] if fn.endswith("bf16") else []
    ptrs = [FAKE] * 10
    assert f(*ptrs, 4, 64, 100, 0.125, *extra) == 2
    for i in range(10):
        bad = list(ptrs)
        bad[i] = None
        assert f(*bad, 4, 64, 64, 0.125, *extra) == 1
        assert f"pointer argument {i} is null" in A.last_error()


def test_backward_phase_validation():
    f = A.lib().dadgpt_flash_attention_backward_bf16_phase
    assert f(3, *[FAKE] * 10, 4, 64, 64, 0.125, None) == 1
    assert f(-1, *[FAKE] * 10, 4, 64, 64, 0.125, None) == 1
    assert f(1, *[FAKE] * 10, 4, 64, 40, 0.125, None) == 2


def _strides(n, batch=1 << 16, head=64, row=768):
    return (A.HeadStrides * n)(*[A.HeadStrides(batch, head, row) for _ in range(n)])


def test_strided_validation():
    L = A.lib()
    fwd, bwd = (L.dadgpt_flash_attention_forward_bf16_strided,
                L.dadgpt_flash_attention_backward_bf16_strided)
    ok4, ok8 = _strides(4), _strides(8)
    # shape and pointer checks as in the contiguous calls
    assert fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 12, 64, 48, 0.125, ok4, None) == 2
    assert fwd(None, FAKE, FAKE, FAKE, FAKE, 2, 12, 64, 64, 0.125, ok4, None) == 1
    assert fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 12, 64, 64, 0.125, ok4, None) == 1
    assert fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 0, 64, 64, 0.125, ok4, None) == 1
    assert fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 12, 64, 64, 0.125, None, None) == 1
    assert "strides is null" in A.last_error()
    assert bwd(*[FAKE] * 10, 2, 12, 64, 64, 0.125, None, None) == 1
    # every stride: a non-negative multiple of 8 with d_head <= row <= 2^24
    for field, value in (("batch", 12), ("head", -64), ("row", 60), ("row", 776 + 4),
                         ("row", 1 << 25)):
        for idx in range(4):
            st = _strides(4)
            setattr(st[idx], field, value)
            assert fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 12, 64, 64, 0.125, st, None) == 1
            assert ("q", "k", "v", "out")[idx] in A.last_error()
        st = _strides(8)
        setattr(st[7], field, value)
        assert bwd(*[FAKE] * 10, 2, 12, 64, 64, 0.125, st, None) == 1
        assert "strides of dv" in A.last_error()
    for i in range(10):
        bad = [FAKE] * 10
        bad[i] = None
        assert bwd(*bad, 2, 12, 64, 64, 0.125, ok8, None) == 1


def test_tokens_validation():
    L = A.lib()
    fwd, bwd = (L.dadgpt_flash_attention_forward_bf16_tokens,
                L.dadgpt_flash_attention_backward_bf16_tokens)
    # leading dimensions below H*d_head (heads would overlap) or not multiples of 8
    assert fwd(FAKE, 768, FAKE, FAKE, FAKE, FAKE, 760, 2, 12, 64, 64, 0.125, None) == 1
    assert "leading dimension 760" in A.last_error()
    assert fwd(FAKE, 700, FAKE, FAKE, FAKE, FAKE, 2304, 2, 12, 64, 64, 0.125, None) == 1
    assert fwd(FAKE, 772, FAKE, FAKE, FAKE, FAKE, 2304, 2, 12, 64, 64, 0.125, None) == 1
    assert "multiple of 8" in A.last_error()
    assert fwd(FAKE, 768, FAKE, FAKE, FAKE, FAKE, 2304, 2, 12, 64, 48, 0.125, None) == 2
    args = lambda ld_g=2304, ld_o=768, ld_in=2304, d=64: (
        [FAKE, FAKE, FAKE, ld_g, FAKE, FAKE, FAKE, ld_o, FAKE, FAKE, FAKE, FAKE, ld_in, 2, 12,
         64, d, 0.125, None])
    assert bwd(*args(ld_g=512)) == 1
    assert bwd(*args(ld_o=1 << 25)) == 1
    assert bwd(*args(d=40)) == 2


def test_dropout_validation():
    L = A.lib()
    fwd, bwd = (L.dadgpt_flash_attention_forward_bf16_dropout,
                L.dadgpt_flash_attention_backward_bf16_dropout)
    for p in (1.0, -0.01, float("nan"), float("inf"), 1.5):
        assert fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 64, 0.125, p, 7, None) == 1
        assert "dropout_p" in A.last_error()
        assert bwd(*[FAKE] * 10, 4, 64, 64, 0.125, p, 7, None) == 1
    assert fwd(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 48, 0.125, 0.1, 7, None) == 2
    assert fwd(None, FAKE, FAKE, FAKE, FAKE, 4, 64, 64, 0.125, 0.1, 7, None) == 1
    assert bwd(*[FAKE] * 10, 4, 0, 64, 0.125, 0.1, 7, None) == 1
    fwd32, bwd32 = (L.dadgpt_flash_attention_forward_dropout,
                    L.dadgpt_flash_attention_backward_dropout)
    assert fwd32(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 64, 0.125, 1.0, 7, None) == 1
    assert bwd32(*[FAKE] * 10, 4, 64, 64, 0.125, -0.5, 7, None) == 1
    assert fwd32(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 64, 40, 0.125, 0.1, 7, None) == 2


def expected_ws(n, h, max_len, d):
    """One uint32 arrival counter per (sequence, head), the region padded to 256 bytes, then
    fp32 partials (max, sum, o[d]) per chunk, when the cache needs more than one chunk. fp32
    chunks (256 keys at d=64, 512 at d=32) are the shorter ones, so their count serves both
    element types."""
    chunk = 256 if d == 64 else 512
    n_chunk = (max_len + chunk - 1) // chunk
    if n_chunk == 1:
        return 0
    return (4 * n * h + 255) // 256 * 256 + 4 * n * h * n_chunk * (d + 2)


@pytest.mark.parametrize("n,h,L,d", [(32, 12, 1024, 64), (1, 1, 1, 32), (3, 5, 257, 64),
                                     (2, 3, 256, 64), (2, 3, 512, 32), (2, 3, 513, 32),
                                     (4, 12, 4096, 64)])
def test_decode_workspace_bytes(n, h, L, d):
    assert A.decode_workspace_bytes(n, h, L, d) == expected_ws(n, h, L, d)


def test_decode_workspace_bytes_rejects_bad_shapes():
    assert A.decode_workspace_bytes(0, 12, 1024, 64) == 0
    assert A.decode_workspace_bytes(4, 12, 1024, 48) == 0


@pytest.mark.parametrize("fn", ["dadgpt_decode_attention_bf16", "dadgpt_decode_attention_f32"])
def test_decode_validation(fn):
    f = getattr(A.lib(), fn)
    need = expected_ws(4, 2, 2000, 64)
    assert need > 0
    args = lambda **kw: [kw.get("out", FAKE), FAKE, FAKE, FAKE, kw.get("lens", FAKE),
                         kw.get("n", 4), kw.get("h", 2), kw.get("L", 2000), kw.get("d", 64),
                         kw.get("scale", 0.125), kw.get("ws", FAKE), kw.get("wsb", need), None]
    assert f(*args(d=48)) == 2
    assert f(*args(out=None)) == 1
    assert f(*args(lens=None)) == 1
    assert f(*args(n=0)) == 1
    assert f(*args(L=0)) == 1
    assert f(*args(n=1 << 22)) == 1  # 2^22 x 2 heads: 2^23 caches of 512 lanes
    assert f(*args(scale=float("nan"))) == 1
    assert f(*args(ws=None)) == 4
    assert f(*args(wsb=need - 1)) == 4
    assert "needed" in A.last_error()


def test_decode_launch_limits():
    """Grid limits of the decode launch: (n_seq * n_heads) workgroups of 512 lanes must count
    fewer than 2^32 work-items, and the chunk count (256-key fp32 chunks at d_head 64) must
    fit grid.y <= 65535; both are refused on the host."""
    for fn in ("dadgpt_decode_attention_bf16", "dadgpt_decode_attention_f32"):
        f = getattr(A.lib(), fn)
        big = [FAKE, FAKE, FAKE, FAKE, FAKE]
        assert f(*big, 1 << 12, 1 << 11, 64, 64, 0.125, None, 0, None) == 1  # 2^23 caches
        assert "launch limits" in A.last_error()
        assert f(*big, 1, 1, 65535 * 256 + 1, 64, 0.125, FAKE, 1 << 40, None) == 1
        assert "launch limits" in A.last_error()


def test_attention_launch_limits():
    """Attention grids are (BH, ceil(S / 64)) at the smallest tile: S above 65535 * 64 and
    BH = 2^24 (2^32 work-items of 256-lane workgroups) are refused on the host."""
    L = A.lib()
    f = L.dadgpt_flash_attention_forward_bf16
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 1, 65535 * 64 + 1, 64, 0.125, None) == 1
    assert "exceeds" in A.last_error()
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 24, 1, 64, 0.125, None) == 1
    g = L.dadgpt_flash_attention_forward
    assert g(FAKE, FAKE, FAKE, FAKE, FAKE, 1, 65535 * 64 + 1, 64, 0.125) == 1


def test_decode_noalloc_validation():
    """The allocation-free decode checks the shape like the workspace form and refuses, before
    any HIP call, a shape whose split partials would not fit the fixed per-device scratch."""
    f = A.lib().dadgpt_decode_attention_bf16_noalloc
    args = lambda **kw: [kw.get("out", FAKE), FAKE, FAKE, FAKE, kw.get("lens", FAKE),
                         kw.get("n", 32), kw.get("h", 12), kw.get("L", 1024), kw.get("d", 64),
                         kw.get("scale", 0.125), None]
    assert f(*args(d=48)) == 2
    assert f(*args(out=None)) == 1
    assert f(*args(lens=None)) == 1
    assert f(*args(n=0)) == 1
    assert f(*args(scale=float("inf"))) == 1
    limit = A.DECODE_NOALLOC_SCRATCH_BYTES
    # the largest max_len that fits at 32 x 12 caches, d_head 64, and the next chunk beyond it
    fits = max(L for L in range(256, 20000, 256) if expected_ws(32, 12, L, 64) <= limit)
    assert expected_ws(32, 12, fits + 1, 64) > limit
    assert f(*args(L=fits + 1)) == 4
    assert "scratch" in A.last_error() and str(limit) in A.last_error()
    assert f(*args(n=1 << 12, h=1 << 11)) == 1  # launch limit before the scratch check


def test_decode_noalloc_limit_matches_header():
    text = open(HEADER).read()
    m = re.search(r"#define DADGPT_DECODE_NOALLOC_SCRATCH_BYTES \(\(size_t\)(\d+) << (\d+)\)",
                  text)
    assert m, "scratch limit macro not found"
    assert int(m.group(1)) << int(m.group(2)) == A.DECODE_NOALLOC_SCRATCH_BYTES


def test_use_fused_attention_policy():
    """The reference's choice (src/model.cpp:183-197) over every input combination:
    dropout or an unsupported d_head -> materialized; Fused / Materialized as selected; Auto
    -> fused from ctx_len 512."""
    for d in (16, 32, 48, 64, 80, 128):
        for ctx in (1, 64, 511, 512, 513, 1024, 8192):
            for drop in (False, True):
                for impl in ("auto", "fused", "materialized"):
                    want = (not drop and d in (32, 64) and
                            (impl == "fused" or (impl == "auto" and ctx >= 512)))
                    assert A.use_fused_attention(impl, d, ctx, drop) == want, (impl, d, ctx, drop)


def test_materialized_ops_validation():
    L = A.lib()
    assert L.dadgpt_softmax(None, FAKE, 4, 64, None) == 1
    assert L.dadgpt_softmax(FAKE, FAKE, 0, 64, None) == 1
    assert L.dadgpt_softmax(FAKE, FAKE, 4, 0, None) == 1
    assert L.dadgpt_softmax(FAKE + 2, FAKE, 4, 64, None) == 1
    assert "aligned" in A.last_error()
    assert L.dadgpt_softmax(FAKE, FAKE, 1 << 26, 4, None) == 1  # rows * 64 lanes >= 2^32
    assert L.dadgpt_softmax_backward(FAKE, FAKE, None, 4, 64, None) == 1
    assert L.dadgpt_causal_mask(FAKE, 0, 64, None) == 1
    assert L.dadgpt_causal_mask_zero(None, 2, 64, None) == 1
    assert L.dadgpt_scale(None, 10, 2.0, None) == 1
    assert L.dadgpt_scale(FAKE, -1, 2.0, None) == 1
    assert L.dadgpt_scale(FAKE, 0, 2.0, None) == 0  # nothing to do, no launch
    assert L.dadgpt_attention_probs(FAKE, 2, 64, float("nan"), None) == 1
    assert L.dadgpt_attention_probs(FAKE, 0, 64, 0.125, None) == 1
    assert L.dadgpt_attention_probs_backward(FAKE, FAKE, None, 2, 64, 0.125, None) == 1
    assert L.dadgpt_decode_probs(FAKE, None, 2, 12, 1024, 0.125, None) == 1
    assert L.dadgpt_decode_probs(FAKE, FAKE, 2, 0, 1024, 0.125, None) == 1
    assert L.dadgpt_attention_dropout(FAKE, FAKE, 2, 64, 1.0, 7, None) == 1
    assert L.dadgpt_attention_dropout(None, FAKE, 2, 64, 0.1, 7, None) == 1
    assert L.dadgpt_attention_probs_backward_dropout(FAKE, FAKE, FAKE, 2, 64, 0.125, -0.5, 7,
                                                     None) == 1
    assert L.dadgpt_attention_probs_backward_dropout(FAKE, FAKE, FAKE, 2, 64, float("inf"), 0.1,
                                                     7, None) == 1


def test_cxx_reference_names_link_and_throw(tmp_path):
    """A C++ caller using the reference's names/signatures links and gets the reference's
    exceptions (built with g++ here; needs no GPU)."""
    exe = tmp_path / "boundary_test"
    libdir = os.path.dirname(A.LIB_PATH)
    subprocess.run(["g++", "-std=c++20", "-O1", f"-I{ROOT}/include",
                    os.path.join(ROOT, "tests", "cxx", "boundary_test.cpp"),
                    f"-L{libdir}", "-ldadgpt_attn", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("OK")


@pytest.mark.parametrize("model_hpp_first", [True, False])
def test_cxx_header_composes_with_reference_enum(tmp_path, model_hpp_first):
    """The drop-in header only declares AttentionImpl, so a caller that also includes the
    reference's model.hpp (which defines it, src/model.hpp:81) compiles in either include order
    and links use_fused_attention (a full definition in the header would be a redefinition)."""
    exe = tmp_path / "model_hpp_order"
    libdir = os.path.dirname(A.LIB_PATH)
    flags = ["-DMODEL_HPP_FIRST"] if model_hpp_first else []
    subprocess.run(["g++", "-std=c++20", "-O1", *flags, f"-I{ROOT}/include",
                    os.path.join(ROOT, "tests", "cxx", "model_hpp_order_test.cpp"),
                    f"-L{libdir}", "-ldadgpt_attn", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "OK", r.stdout + r.stderr
