"""GPU test of the allocation-free decode entry point (dadgpt_decode_attention_bf16_noalloc).

It must return, bit for bit, what dadgpt_decode_attention_bf16 returns with a caller
workspace (both run the same kernels), on consecutive calls that share the library's fixed
scratch: a first call with split caches, then a smaller shape, then the first shape again
(the counters left by each call must be zero for the next). Sampled rows are also checked
against the CPU oracle. Everything goes through the C ABI (ctypes).
"""
import numpy as np
import pytest
import torch

import oracle
from dadgpt_amd import attention as A
from dadgpt_amd import synth


def _run_both(n, H, L, D, seed, dev):
    qn, kc, vc, lens = synth.decode_inputs(n, H, L, D, seed=seed)
    bf = torch.bfloat16
    q = torch.from_numpy(qn).to(dev).to(bf)
    k = torch.from_numpy(kc).to(dev).to(bf)
    v = torch.from_numpy(vc).to(dev).to(bf)
    ln = torch.from_numpy(lens).to(dev)
    scale = 1.0 / np.sqrt(D)
    ref = torch.empty(n, H, D, dtype=bf, device=dev)
    ws = A.decode_workspace(n, H, L, D, device=dev)
    A.decode_attention(ref, q, k, v, ln, n, H, L, D, scale, ws)
    out = torch.full((n, H, D), float("nan"), dtype=bf, device=dev)
    A.decode_attention_noalloc(out, q, k, v, ln, n, H, L, D, scale)
    torch.cuda.synchronize()
    return out, ref, (qn, kc, vc, lens, scale)


@pytest.mark.gpu
def test_noalloc_decode_matches_workspace_form(gpu):
    cases = [(32, 12, 1024, 64, synth.BASE_SEED + 4),  # cfg4: split caches (2 bf16 chunks)
             (5, 3, 700, 64, 311),                     # smaller shape, reuses the scratch
             (4, 2, 2600, 32, 312),                    # d_head 32, 3 chunks
             (32, 12, 1024, 64, synth.BASE_SEED + 4)]  # the first shape again
    for n, H, L, D, seed in cases:
        print(f"[noalloc] n={n} H={H} max_len={L} d_head={D} seed={seed}", flush=True)
        assert A.decode_workspace_bytes(n, H, L, D) <= A.DECODE_NOALLOC_SCRATCH_BYTES
        out, ref, (qn, kc, vc, lens, scale) = _run_both(n, H, L, D, seed, gpu)
        assert not torch.isnan(out.float()).any()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (n, H, L, D)
        # sampled sequences against the oracle (bf16 tolerance of the decode tests)
        pick = np.unique(np.array([0, n // 2, n - 1]))
        o_ref = oracle.decode(qn[pick], kc[pick], vc[pick], lens[pick], scale)
        err = float(np.abs(out.float().cpu().numpy()[pick] - o_ref).max())
        assert err <= 2e-2, err


@pytest.mark.gpu
def test_noalloc_decode_refuses_oversize(gpu):
    """A shape whose partials exceed the scratch fails with the workspace status and leaves
    the next valid call correct."""
    dev = gpu
    bf = torch.bfloat16
    n, H, L, D = 32, 12, 12288, 64
    assert A.decode_workspace_bytes(n, H, L, D) > A.DECODE_NOALLOC_SCRATCH_BYTES
    q = torch.zeros(n, H, D, dtype=bf, device=dev)
    k = torch.zeros(n, H, L, D, dtype=bf, device=dev)
    lens = torch.full((n,), L, dtype=torch.int32, device=dev)
    out = torch.empty(n, H, D, dtype=bf, device=dev)
    with pytest.raises(A.AttentionError) as e:
        A.decode_attention_noalloc(out, q, k, k, lens, n, H, L, D, 0.125)
    assert e.value.status == 4
    del k
    out2, ref2, _ = _run_both(6, 4, 900, 64, 313, dev)
    assert torch.equal(out2.view(torch.int16), ref2.view(torch.int16))
