"""Benchmark of the fused causal attention path on one MI355X.

Headline (BASELINE.json metric "attn fwd/bwd TFLOP/s (B16 H12 T1024 D64 bf16); KV-decode HBM
GB/s"): one step = the bf16 causal forward (saving lse) plus the backward from that lse at
B=16, H=12, T=1024, D=64, inputs N(0,1) synthetic and resident in HBM.
value = algorithmic FLOPs of the step / time per step:
  forward  4*B*H*T^2*D/2           = 25.770 GFLOP
  backward 2.5 x forward (5 GEMMs) = 64.425 GFLOP
The same line carries each kernel's time and roofline fraction, the KV-decode HBM bandwidth
(config 4: 32 ragged sequences, H12, D64, bf16 cache, timed over rotating cache copies so
the 256 MB MALL cannot hold them), the roofline of the dominant kernel, and the reference's
CPU path timed on a bounded sample on this host.

Config 5 (GPT-2 124M architecture, random init, 16 prompts of U[16,256] random tokens,
batched prefill + 128 greedy tokens) is reported under components.generate_cfg5: tokens/s,
the decode-attention time share, the comparison with fp32 attention, and the greedy gate at
the reference's precision (fp32 flash vs fp32 materialized attention, fp32 projections).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-generate]
    python bench.py --profile-sample     # each kernel --reps times + a copy of known size,
                                         # for rocprofv3 --pmc runs; prints no bench line
    python bench.py --generate-only      # the config 5 leg alone (for rocprofv3)
    python bench.py --generate-only --no-gate   # ... without the fp32 greedy-gate models
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# Before torch: the package loads its hipBLASLt ahead of PyTorch's bundled one.
import dadgpt_amd  # noqa: E402,F401

PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 4096 flop/clk/CU x 2.4 GHz, dense
PEAK_F32_TFLOPS = 157.3     # fp32 MFMA, dense
PEAK_HBM_GBPS = 8000.0
CPU_THREADS = 16            # the GPU box's CPU share for one GPU

B, H, T, D = 16, 12, 1024, 64
BH = B * H
CFG2_BH = 8 * H                          # config 2: B8 H12 T1024 D64, forward only
SCALE = 0.125
UNIT = 2.0 * BH * T * T * D / 2          # one causal S x S x D product: 12.885 GFLOP
FWD_FLOPS = 2 * UNIT                     # 25.770 GFLOP
BWD_FLOPS = 5 * UNIT                     # 64.425 GFLOP
# Algorithmic share per backward kernel: dK/dV computes S, dP, dV, dK (4 units); dQ computes
# dQ (1 unit) and recomputes S and dP (executed, not algorithmic).
KERNEL_FLOPS = {"fwd": FWD_FLOPS, "bwd_dq": UNIT, "bwd_dkdv": 4 * UNIT}

DEC_N, DEC_H, DEC_L, DEC_D = 32, 12, 1024, 64
COPY_BYTES = 256 << 20                   # calibration copy for the --pmc traffic factor

# HBM bytes per launch from the rocprofv3 --pmc runs (FETCH_SIZE + WRITE_SIZE, each scaled by
# the factor a plain copy of known size reads): lines "traffic <kernel> <bytes>".
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "pmc_traffic_cfg3_cfg4.txt")


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--reps", type=int, default=20, help="launches per kernel timing")
    p.add_argument("--decode-copies", type=int, default=8)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-slices", type=int, default=6,
                   help="cfg3 (b,h) slices for the single-thread CPU run (x16 for all cores)")
    p.add_argument("--profile-sample", action="store_true")
    p.add_argument("--no-generate", action="store_true", help="skip the config 5 leg")
    p.add_argument("--generate-only", action="store_true",
                   help="run only the config 5 leg (for profiling); prints no bench line")
    p.add_argument("--no-gate", action="store_true",
                   help="config 5 without the fp32 greedy-gate models (profiles of the "
                        "product path)")
    p.add_argument("--prewarm-seconds", type=float, default=2.0,
                   help="untimed fwd+bwd steps before the warmup, so clocks have ramped")
    return p.parse_args()


def event_time_ms(fn, reps, stream):
    """Average ms per call of fn() over `reps` back-to-back calls, HIP events on `stream`
    (the stream every kernel here is launched on)."""
    import torch
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / reps


# The sources of the profiled kernels: the traffic summary records their digest at profiling
# time, so a bench line can say whether its traffic figures describe the kernels it timed.
KERNEL_SOURCES = [os.path.join(ROOT, "dadgpt_amd", "csrc", n) for n in (
    "attn_fwd_bf16.hip", "attn_bwd_bf16.hip", "decode.hip", "tiles.hpp", "common.hpp",
    "lanes.hpp", "dropout.hpp", "kernels.hpp")]


def kernel_sources_digest():
    import hashlib

    h = hashlib.sha256()
    for path in KERNEL_SOURCES:
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def load_traffic():
    """({kernel: HBM bytes per launch}, digest of the kernel sources they were measured on)
    from the committed --pmc summary (empty / None if absent)."""
    out, digest = {}, None
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                m = re.match(r"^traffic\s+(\w+)\s+(\d+)\s*$", line)
                if m:
                    out[m.group(1)] = int(m.group(2))
                m = re.match(r"^# kernel sources digest\s+([0-9a-f]+)", line)
                if m:
                    digest = m.group(1)
    except OSError:
        pass
    return out, digest


def decode_lens():
    """Config 4's cache lengths: U[1, 1024] per sequence, seeded."""
    import numpy as np
    from dadgpt_amd import synth
    return synth.uniform_int(1, DEC_L, DEC_N, synth.BASE_SEED ^ synth.TENSOR_ID["lens"]).astype(
        np.int32)


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed(fn, reps=1):
    """Median wall time of reps calls (after one untimed warm-up when reps > 1)."""
    if reps > 1:
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline(n_slices):
    """The reference's CPU path on this host (oracle/_ref: its own tensor_ops.cpp and
    backward.cpp composed in the materialized op order; the C restatement when that is not
    built). Bounded samples, about 20 s in all:
      - cfg3 forward+backward on n_slices (b,h) slices single-threaded, and on 16 * n_slices
        slices over CPU_THREADS threads (slices are independent; ctypes releases the GIL);
        value = the all-thread rate in algorithmic TFLOP/s;
      - cfg1 (B1 H4 T64 D32) forward+backward in full, cfg4 decode (32 ragged caches) in full;
      - cfg5: per-token cost of the reference's CPU GPT-2 forward (one sequence of 16 and of 32
        tokens), extrapolated to 16 prompts + 128 greedy tokens each."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle
    from dadgpt_amd import synth

    ref = oracle.ref_available()
    kind = "reference" if ref else "port"
    fwd = oracle.ref_attn_fwd if ref else (lambda q, k, v, sc: oracle.attn_fwd_slices(
        q, k, v, sc, 0, q.shape[0]))
    bwd = oracle.ref_attn_bwd if ref else (lambda g, q, k, v, sc: oracle.attn_bwd_slices(
        g, q, k, v, sc, 0, q.shape[0]))
    per_slice = (FWD_FLOPS + BWD_FLOPS) / BH

    def run(x):
        q, k, v, g = x
        fwd(q, k, v, SCALE)
        bwd(g, q, k, v, SCALE)

    one = synth.attn_inputs(n_slices, T, D, seed=synth.BASE_SEED + 3, with_dout=True, bf16=True)
    dt1 = _timed(lambda: run(one))
    chunks = [synth.attn_inputs(n_slices, T, D, seed=synth.BASE_SEED + 30 + i, with_dout=True,
                                bf16=True) for i in range(CPU_THREADS)]
    with ThreadPoolExecutor(CPU_THREADS) as pool:
        t0 = time.perf_counter()
        list(pool.map(run, chunks))
        dtn = time.perf_counter() - t0
    tf1 = per_slice * n_slices / dt1 / 1e12
    tfn = per_slice * n_slices * CPU_THREADS / dtn / 1e12

    q1, k1, v1, g1 = synth.attn_inputs(4, 64, 32, seed=synth.BASE_SEED, with_dout=True)
    sc1 = float(np.float32(1 / np.sqrt(32)))
    cfg1_s = _timed(lambda: (fwd(q1, k1, v1, sc1), bwd(g1, q1, k1, v1, sc1)), reps=3)
    qd, kc, vc, _ = synth.decode_inputs(DEC_N, DEC_H, DEC_L, DEC_D, seed=synth.BASE_SEED + 4)
    lens = decode_lens()  # the GPU decode measurement's lengths
    dec = oracle.ref_decode if ref else oracle.decode
    cfg4_s = _timed(lambda: dec(qd, kc, vc, lens, SCALE), reps=3)
    cfg4_bytes = 2 * int(lens.sum()) * DEC_H * DEC_D * 2 + 2 * DEC_N * DEC_H * DEC_D * 2

    cfg5 = None
    if ref:
        from dadgpt_amd import gpt2
        cfg = gpt2.PRESETS["gpt2-124m"]
        host = gpt2.init_params(cfg, synth.CFG5_SEED).float().cpu().numpy()
        toks = synth.cfg5_prompts(cfg["vocab_size"])[0]
        t16 = _timed(lambda: oracle.ref_gpt2_forward(host, cfg, toks[:16]))
        t32 = _timed(lambda: oracle.ref_gpt2_forward(host, cfg, toks[:32]))
        per_tok = (t32 - t16) / 16  # the marginal cost of one more token
        prompts = synth.cfg5_prompts(cfg["vocab_size"])
        work = sum(len(p) for p in prompts) + synth.CFG5_N * synth.CFG5_NEW
        cfg5 = {"tokens_per_s_extrapolated": round(synth.CFG5_N * synth.CFG5_NEW /
                                                   (work * per_tok), 3),
                "seconds_per_token": round(per_tok, 4),
                "sample": "one sequence through the reference's CPU GPT-2 forward at 16 and 32 "
                          "tokens (fp32, single thread); the marginal per-token cost times "
                          f"{work} token forwards (16 prompts + 16 x 128 generated tokens; the "
                          "reference's CPU path has no KV cache), extrapolated"}
    return {
        "value": float(f"{tfn:.6g}"),
        "unit": "TFLOP/s",
        "cores": CPU_THREADS,
        "kind": kind,
        "sample": (f"fp32 forward+backward of {n_slices * CPU_THREADS} of {BH} (b,h) slices of "
                   f"B16 H12 T1024 D64 (bf16-rounded inputs), {n_slices} slices per thread on "
                   f"{CPU_THREADS} threads, {dtn:.2f} s; algorithmic FLOPs of those slices / "
                   f"wall time"),
        "seconds": round(dtn, 3),
        "host": {"cpu_model": _cpu_model(), "hardware_threads": os.cpu_count(),
                 "threads_available": len(os.sched_getaffinity(0))},
        "single_thread": {"value": float(f"{tf1:.6g}"), "unit": "TFLOP/s", "cores": 1,
                          "sample": f"{n_slices} slices, one thread, {dt1:.2f} s"},
        "cfg1_fwd_bwd_ms": round(cfg1_s * 1e3, 3),
        "cfg4_decode": {"ms": round(cfg4_s * 1e3, 3),
                        "gbps": round(cfg4_bytes / cfg4_s / 1e9, 3), "bytes": cfg4_bytes,
                        "cores": 1},
        "cfg5": cfg5,
    }


class Workload:
    """Device buffers of config 3 (fwd+bwd) and config 4 (decode, rotating cache copies)."""

    def __init__(self, decode_copies):
        import numpy as np
        import torch
        from dadgpt_amd import attention as A
        from dadgpt_amd import synth

        self.A = A
        dev = torch.device("cuda:0")
        gen = torch.Generator(device=dev)
        gen.manual_seed(0xDAD6B7)

        def randn(*shape):
            return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32).to(
                torch.bfloat16)

        self.q, self.k, self.v, self.g = (randn(BH, T, D) for _ in range(4))
        self.out = torch.empty_like(self.q)
        self.lse = torch.empty(BH, T, device=dev)
        self.dq, self.dk, self.dv = (torch.empty_like(self.q) for _ in range(3))
        self.delta = torch.empty(BH, T, device=dev)

        lens_h = decode_lens()
        self.lens = torch.from_numpy(lens_h.astype(np.int32)).to(dev)
        # K and V rows actually read, plus q and out
        self.dec_bytes = int(2 * lens_h.sum() * DEC_H * DEC_D * 2 + 2 * DEC_N * DEC_H * DEC_D * 2)
        self.ncopy = decode_copies
        self.kcs = [randn(DEC_N, DEC_H, DEC_L, DEC_D) for _ in range(decode_copies)]
        self.vcs = [randn(DEC_N, DEC_H, DEC_L, DEC_D) for _ in range(decode_copies)]
        self.qd = randn(DEC_N, DEC_H, DEC_D)
        self.od = torch.empty_like(self.qd)
        self.ws = A.decode_workspace(DEC_N, DEC_H, DEC_L, DEC_D)

    def fwd(self):
        self.A.flash_attention_forward_bf16(self.out, self.lse, self.q, self.k, self.v, BH, T, D,
                                            SCALE, None)

    def fwd_cfg2(self):
        """BASELINE config 2 (B8 H12 T1024 D64): the first 96 slices of the config 3 tensors."""
        self.A.flash_attention_forward_bf16(self.out, self.lse, self.q, self.k, self.v, CFG2_BH,
                                            T, D, SCALE, None)

    def fp32_paths(self):
        """The reference's precision at config 3: the fp32 flash kernels and the fp32
        materialized path (hipBLASLt strided-batched GEMMs + fused row passes, [BH, T, T]
        probabilities in HBM). Returns (flash fwd, flash bwd, materialized fwd, bwd)."""
        import torch
        from dadgpt_amd import gpt2
        A = self.A
        f = [t.float() for t in (self.q, self.k, self.v, self.g)]
        q, k, v, g = f
        out, dq, dk, dv = (torch.empty_like(q) for _ in range(4))
        lse, delta = torch.empty(BH, T, device="cuda"), torch.empty(BH, T, device="cuda")
        probs = torch.empty(BH, T, T, device="cuda")
        dsc = torch.empty(BH, T, T, device="cuda")
        blas = gpt2.Blas()
        self._fp32 = (f, out, dq, dk, dv, lse, delta, probs, dsc, blas)

        def ffwd():
            A.flash_attention_forward(out, lse, q, k, v, BH, T, D, SCALE)

        def fbwd():
            A.flash_attention_backward(dq, dk, dv, delta, g, out, lse, q, k, v, BH, T, D,
                                             SCALE)

        def mfwd():
            blas.attention_materialized_forward(out, probs, q, k, v, BH, T, D, SCALE)

        def mbwd():
            blas.attention_materialized_backward(dq, dk, dv, dsc, g, probs, q, k, v, BH, T, D,
                                                 SCALE)
        return ffwd, fbwd, mfwd, mbwd

    def bwd(self):
        self.A.flash_attention_backward_bf16(self.dq, self.dk, self.dv, self.delta, self.g,
                                             self.out, self.lse, self.q, self.k, self.v, BH, T,
                                             D, SCALE, None)

    def phase(self, p):
        def run():
            self.A.flash_attention_backward_bf16_phase(p, self.dq, self.dk, self.dv, self.delta,
                                                       self.g, self.out, self.lse, self.q,
                                                       self.k, self.v, BH, T, D, SCALE, None)
        return run

    def step(self):
        self.fwd()
        self.bwd()

    def dropout(self, p=0.1, seed=7):
        """Forward and backward with attention-probability dropout at rate p (the keep bits
        regenerated inside the kernels)."""
        A = self.A

        def fwd():
            A.flash_attention_forward_bf16_dropout(self.out, self.lse, self.q, self.k, self.v,
                                                   BH, T, D, SCALE, p, seed)

        def bwd():
            A.flash_attention_backward_bf16_dropout(self.dq, self.dk, self.dv, self.delta,
                                                    self.g, self.out, self.lse, self.q,
                                                    self.k, self.v, BH, T, D, SCALE, p, seed)
        return fwd, bwd

    def tokens(self):
        """Forward and backward over the token-major layout of a fused QKV projection
        ([B*T, 3*H*D] in, [B*T, H*D] out, gradient [B*T, 3*H*D]): the same kernels reading and
        writing rows where the projections keep them, with no split/merge passes."""
        import torch
        A, HD = self.A, H * D
        if not hasattr(self, "qkv"):
            self.qkv = torch.cat([t.view(B, H, T, D).permute(0, 2, 1, 3).reshape(B * T, HD)
                                  for t in (self.q, self.k, self.v)], dim=1).contiguous()
            self.g_tok = self.g.view(B, H, T, D).permute(0, 2, 1, 3).reshape(B * T, HD).clone()
            self.o_tok = torch.empty_like(self.g_tok)
            self.dqkv = torch.empty_like(self.qkv)
        qkv, dqkv = self.qkv, self.dqkv

        def fwd():
            A.flash_attention_forward_bf16_tokens(self.o_tok, HD, self.lse, qkv, qkv[:, HD:],
                                                  qkv[:, 2 * HD:], 3 * HD, B, H, T, D, SCALE)

        def bwd():
            A.flash_attention_backward_bf16_tokens(dqkv, dqkv[:, HD:], dqkv[:, 2 * HD:], 3 * HD,
                                                   self.delta, self.g_tok, self.o_tok, HD,
                                                   self.lse, qkv, qkv[:, HD:], qkv[:, 2 * HD:],
                                                   3 * HD, B, H, T, D, SCALE)
        return fwd, bwd

    def decode(self, i, lens=None, n_seq=DEC_N):
        self.A.decode_attention(self.od, self.qd, self.kcs[i % self.ncopy],
                                self.vcs[i % self.ncopy], self.lens if lens is None else lens,
                                n_seq, DEC_H, DEC_L, DEC_D, SCALE, self.ws, None)


def profile_sample(wl, reps):
    """Each kernel `reps` times, then a device copy of COPY_BYTES (the calibration kernel
    for FETCH_SIZE / WRITE_SIZE), for rocprofv3 runs."""
    import torch
    for _ in range(reps):
        wl.fwd()
    for p in (1, 2):
        run = wl.phase(p)
        for _ in range(reps):
            run()
    for i in range(reps):
        wl.decode(i)
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[profile-sample] {reps} launches each of fwd, bwd phases 0-2, decode, and a "
          f"{COPY_BYTES} B copy", flush=True)




def generate_cfg5(gate: bool = True):
    """Config 5: GPT-2 124M architecture, random init (the reference's init rules,
    src/model.cpp:121-166), 16 prompts of U[16,256] random tokens, batched prefill into the KV
    cache, 128 greedy tokens each; then the same with fp32 attention, and (gate) with fp32
    flash and fp32 materialized attention over fp32 projections."""
    import numpy as np
    import torch

    from dadgpt_amd import gpt2, synth

    GEN_N, GEN_NEW, GEN_SEED = synth.CFG5_N, synth.CFG5_NEW, synth.CFG5_SEED
    cfg = gpt2.PRESETS["gpt2-124m"]
    prompts = synth.cfg5_prompts(cfg["vocab_size"])
    params = gpt2.init_params(cfg, GEN_SEED)
    m16 = gpt2.GPT2(cfg, params, GEN_N, attention="bf16")
    m16.generate(prompts, 8)  # builds the hipBLASLt plans and captures the decode step
    runs = [m16.generate(prompts, GEN_NEW, timing=True) for _ in range(3)]
    best = min(runs, key=lambda r: r["timing"]["prefill_ms"] + r["timing"]["decode_ms"])
    t = best["timing"]
    # the attention launches timed one by one need the eager step (no events inside a graph)
    m16.set_graphs(False)
    eager = m16.generate(prompts, GEN_NEW, timing=True)["timing"]
    m16.close()
    m32 = gpt2.GPT2(cfg, params, GEN_N, attention="fp32")
    ref = m32.generate(prompts, GEN_NEW, timing=True)
    m32.close()
    # the greedy gate at the reference's precision: fp32 flash attention against the GPU's own
    # fp32 materialized attention, both over fp32 projections, logits kept for the comparison
    gate_runs = {}
    for name, attention in ((("flash", "fp32"), ("materialized", "fp32_materialized"))
                            if gate else ()):
        mg = gpt2.GPT2(cfg, params, GEN_N, attention=attention, projections="fp32")
        gate_runs[name] = mg.generate(prompts, GEN_NEW, logits=True)
        mg.close()
    del params
    torch.cuda.synchronize()

    def first_divergence(a, b):
        return [int(np.nonzero(ra != rb)[0][0]) if (ra != rb).any() else GEN_NEW
                for ra, rb in zip(a, b)]
    a, b = best["tokens"], ref["tokens"]
    div = first_divergence(a, b)
    div_margins = [float(ref["margins"][r, d]) for r, d in enumerate(div) if d < GEN_NEW]
    if gate:
        gf, gm = gate_runs["flash"], gate_runs["materialized"]
        gdiv = first_divergence(gf["tokens"], gm["tokens"])
        gate_dev = max(float(np.abs(gf["logits"][:min(d + 1, GEN_NEW), r] -
                                    gm["logits"][:min(d + 1, GEN_NEW), r]).max())
                       for r, d in enumerate(gdiv))
    total_ms = t["prefill_ms"] + t["decode_ms"]
    out = {
        "config": "GPT-2 124M arch (d768 L12 H12 ff3072 ctx1024 V50257), random init, 16 "
                  "prompts len U[16,256], 128 greedy tokens, bf16 attention, bf16 projections "
                  "(hipBLASLt prefill, skinny MFMA decode), fp32 residual",
        "tokens": int(GEN_N * GEN_NEW),
        "tokens_per_s": round(GEN_N * GEN_NEW / (total_ms * 1e-3), 1),
        "decode_tokens_per_s": round(GEN_N * t["decode_steps"] / (t["decode_ms"] * 1e-3), 1),
        "prefill_ms": round(t["prefill_ms"], 3),
        "decode_ms": round(t["decode_ms"], 3),
        "decode_ms_per_step": round(t["decode_ms"] / t["decode_steps"], 4),
        "decode_graph": True,
        "eager_decode_ms": round(eager["decode_ms"], 3),
        "decode_attn_ms": round(eager["decode_attn_ms"], 3),
        "attn_share_of_decode": round(eager["decode_attn_ms"] / eager["decode_ms"], 4),
        "attn_share_basis": "eager decode steps: the attention launches timed with events over "
                            "the same run's decode time (a replayed graph cannot hold events)",
        "fp32_attention": {
            "tokens_per_s": round(GEN_N * GEN_NEW / ((ref["timing"]["prefill_ms"] +
                                                      ref["timing"]["decode_ms"]) * 1e-3), 1),
            "identical_tokens": float((a == b).mean()),
            "rows_identical": int(sum(d == GEN_NEW for d in div)),
            "first_divergence_per_row": div,
            "fp32_margin_at_divergence_max": max(div_margins) if div_margins else None,
            "min_margin_fp32": float(ref["margins"].min()),
            "min_margin_bf16": float(best["margins"].min()),
        },
    }
    if gate:
        out["greedy_gate_fp32"] = {
            "what": "fp32 flash attention vs the GPU's own fp32 materialized attention, both "
                    "with fp32 projections (the reference's precision), same weights and prompts",
            "rows_identical": int(sum(d == GEN_NEW for d in gdiv)),
            "identical_tokens": float((gf["tokens"] == gm["tokens"]).mean()),
            "first_divergence_per_row": gdiv,
            "max_logit_difference_shared_history": gate_dev,
            "min_margin": float(gm["margins"].min()),
        }
    print(f"[bench] generate cfg5 {json.dumps(out)}", file=sys.stderr, flush=True)
    return out


def hip_stack():
    """The HIP runtime and hipBLASLt versions this process runs on (the generation leg's and
    materialized path's GEMMs), and whether the library accepts the pair."""
    from dadgpt_amd import gpt2

    try:
        return gpt2.blas_stack_versions()
    except Exception as e:  # the versions are a report, not a gate, here
        return {"error": str(e)}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1 "
                                   "(every (b,h) slice is independent, so the path shards "
                                   "over (b,h) with no exchange)", "n_gpus": args.gpus}),
              flush=True)
        sys.exit(2)

    import torch

    if args.generate_only:
        generate_cfg5(gate=not args.no_gate)
        return
    wl = Workload(args.decode_copies)
    wl.A.lib()
    if args.profile_sample:
        profile_sample(wl, args.reps)
        return
    stream = torch.cuda.current_stream()

    t_end = time.perf_counter() + args.prewarm_seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            wl.step()
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        wl.step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        wl.step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = start.elapsed_time(end) / args.steps
    print(f"[bench] step fwd+bwd {ms_step:.3f} ms (wall {1e3 * wall / args.steps:.3f} ms)",
          file=sys.stderr, flush=True)

    # per-kernel averages (same stream, back-to-back launches of each), in three interleaved
    # rounds with the best round kept, so every variant is timed in the same state of the box
    # (a single pass timed the later variants up to 25% slower than interleaved rounds do)
    tok_fwd, tok_bwd = wl.tokens()
    drop_fwd, drop_bwd = wl.dropout()
    f32_fwd, f32_bwd, mat_fwd, mat_bwd = wl.fp32_paths()
    for _ in range(5):  # also builds and tunes the hipBLASLt plans of the materialized path
        for fn in (tok_fwd, tok_bwd, drop_fwd, drop_bwd, f32_fwd, f32_bwd, mat_fwd, mat_bwd):
            fn()
    timed = {"fwd": wl.fwd, "bwd_dq": wl.phase(1), "bwd_dkdv": wl.phase(2), "bwd": wl.bwd,
             "fwd_cfg2": wl.fwd_cfg2, "tok_fwd": tok_fwd, "tok_bwd": tok_bwd,
             "drop_fwd": drop_fwd, "drop_bwd": drop_bwd, "f32_fwd": f32_fwd, "f32_bwd": f32_bwd,
             "mat_fwd": mat_fwd, "mat_bwd": mat_bwd}
    best = {}
    for _ in range(3):
        for name, fn in timed.items():
            best[name] = min(best.get(name, float("inf")), event_time_ms(fn, args.reps, stream))
    kern_ms = {k: best[k] for k in ("fwd", "bwd_dq", "bwd_dkdv")}
    bwd_ms = best["bwd"]
    tok_ms = (best["tok_fwd"], best["tok_bwd"])
    drop_ms = (best["drop_fwd"], best["drop_bwd"])
    wl.step()  # leave the undropped results in the buffers
    print(f"[bench] kernels {json.dumps({k: round(x, 4) for k, x in kern_ms.items()})}",
          file=sys.stderr, flush=True)

    # ---- decode (config 4): rotating cache copies, launches captured in a graph ----
    for i in range(wl.ncopy):
        wl.decode(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    per_graph = 4 * wl.ncopy
    with torch.cuda.graph(graph):
        for i in range(per_graph):
            wl.decode(i)
    graph.replay()
    torch.cuda.synchronize()
    dec_ms = event_time_ms(graph.replay, 5, torch.cuda.current_stream()) / per_graph
    dec_gbps = wl.dec_bytes / (dec_ms * 1e-3) / 1e9

    # the same kernel and cache buffers on uniform lengths, to split cfg4's time: every cache
    # one 512-key chunk (no split, no raggedness), and every cache 1024 keys (two chunks,
    # merged by the last-arriving chunk), each over ~50 MB
    def decode_case(n_seq, length):
        lens = torch.full((n_seq,), length, dtype=torch.int32, device="cuda")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(per_graph):
                wl.decode(i, lens, n_seq)
        g.replay()
        torch.cuda.synchronize()
        ms = event_time_ms(g.replay, 5, torch.cuda.current_stream()) / per_graph
        nbytes = 2 * n_seq * length * DEC_H * DEC_D * 2 + 2 * n_seq * DEC_H * DEC_D * 2
        return {"us_per_launch": round(ms * 1e3, 3), "bytes": nbytes,
                "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    dec_cases = {"one_chunk_per_cache": dict(decode_case(DEC_N, 512),
                                             config="32 seqs x 12 heads x 512 keys"),
                 "two_chunks_per_cache": dict(decode_case(DEC_N // 2, 1024),
                                              config="16 seqs x 12 heads x 1024 keys")}
    print(f"[bench] decode on uniform lengths: {json.dumps(dec_cases)}", file=sys.stderr,
          flush=True)
    # eager launches over the rotating copies (launch gaps included)
    eager_dec_ms = event_time_ms(lambda it=iter(range(10 ** 9)): wl.decode(next(it)),
                                 args.reps, stream)
    print(f"[bench] decode {dec_ms * 1e3:.2f} us/launch in graph ({dec_gbps:.0f} GB/s), eager "
          f"{eager_dec_ms * 1e3:.2f} us", file=sys.stderr, flush=True)
    # practical HBM rate: a vendor device copy of the decode's byte count (rotating sources,
    # eager like eager_dec_ms); it moves the bytes twice (read and write)
    srcs = [torch.randn(wl.dec_bytes // 2, device="cuda").to(torch.bfloat16)
            for _ in range(wl.ncopy)]
    dst = torch.empty_like(srcs[0])
    for x in srcs:
        dst.copy_(x)
    copy_ms = event_time_ms(lambda it=iter(range(10 ** 9)): dst.copy_(srcs[next(it) % wl.ncopy]),
                            args.reps, stream)
    copy_gbps = 2 * wl.dec_bytes / (copy_ms * 1e-3) / 1e9
    del srcs, dst
    print(f"[bench] device copy of the decode's bytes: {copy_ms * 1e3:.2f} us "
          f"({copy_gbps:.0f} GB/s read + write)", file=sys.stderr, flush=True)

    traffic, traffic_digest = load_traffic()
    digest_now = kernel_sources_digest()
    traffic_src = {"file": os.path.relpath(TRAFFIC_FILE, ROOT),
                   "kernel_sources_digest": traffic_digest,
                   "current_sources_digest": digest_now,
                   "current": traffic_digest == digest_now,
                   "what": "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE per dispatch (scaled by a "
                           "calibration copy), measured on the kernel sources of that digest; "
                           "stale when the digests differ"}
    comps = {}
    for name, ms in kern_ms.items():
        c = {"ms": round(ms, 5)}
        if name in KERNEL_FLOPS:
            tf = KERNEL_FLOPS[name] / (ms * 1e-3) / 1e12
            c.update({"algorithmic_gflop": round(KERNEL_FLOPS[name] / 1e9, 3),
                      "tflops": round(tf, 2), "frac_mfma_peak": round(tf / PEAK_BF16_TFLOPS, 4)})
        if name in traffic:
            c["hbm_bytes_per_launch"] = traffic[name]
        comps[name] = c
    for name, ms, fl in (("fwd_total", kern_ms["fwd"], FWD_FLOPS), ("bwd_total", bwd_ms,
                                                                     BWD_FLOPS)):
        tf = fl / (ms * 1e-3) / 1e12
        comps[name] = {"ms": round(ms, 5), "tflops": round(tf, 2),
                       "frac_mfma_peak": round(tf / PEAK_BF16_TFLOPS, 4)}
    comps["tokens_layout"] = {
        "fwd_ms": round(tok_ms[0], 5), "bwd_ms": round(tok_ms[1], 5),
        "fwd_tflops": round(FWD_FLOPS / (tok_ms[0] * 1e-3) / 1e12, 2),
        "bwd_tflops": round(BWD_FLOPS / (tok_ms[1] * 1e-3) / 1e12, 2),
        "layout": "q,k,v in one token-major [B*T, 3*H*D] buffer, out/dout [B*T, H*D], "
                  "dq,dk,dv into one [B*T, 3*H*D] buffer"}
    cfg2_tf = FWD_FLOPS * CFG2_BH / BH / (best["fwd_cfg2"] * 1e-3) / 1e12
    comps["fwd_cfg2"] = {"ms": round(best["fwd_cfg2"], 5),
                         "algorithmic_gflop": round(FWD_FLOPS * CFG2_BH / BH / 1e9, 3),
                         "tflops": round(cfg2_tf, 2),
                         "frac_mfma_peak": round(cfg2_tf / PEAK_BF16_TFLOPS, 4),
                         "config": "BASELINE config 2: B8 H12 T1024 D64 bf16 causal forward"}
    for key, (fk, bk), what in (
            ("fp32_flash", ("f32_fwd", "f32_bwd"),
             "fp32 flash kernels at fp32 accuracy, config 3 shape: every product on the "
             "bf16 MFMA as six bf16 cross terms of a three-way split (so the fractions of the "
             "fp32 MFMA peak can exceed 1; *_frac_bf16_peak_executed count the six bf16 "
             "products executed per fp32 product)"),
            ("fp32_materialized", ("mat_fwd", "mat_bwd"),
             "fp32 materialized path (hipBLASLt fp32 strided-batched GEMMs over the full "
             "T x T scores + fused row passes; executes twice the causal FLOPs), config 3 "
             "shape")):
        ftf = FWD_FLOPS / (best[fk] * 1e-3) / 1e12
        btf = BWD_FLOPS / (best[bk] * 1e-3) / 1e12
        comps[key] = {"fwd_ms": round(best[fk], 5), "bwd_ms": round(best[bk], 5),
                      "fwd_tflops": round(ftf, 2), "bwd_tflops": round(btf, 2),
                      "fwd_frac_fp32_mfma_peak": round(ftf / PEAK_F32_TFLOPS, 4),
                      "bwd_frac_fp32_mfma_peak": round(btf / PEAK_F32_TFLOPS, 4),
                      "peak_tflops": PEAK_F32_TFLOPS, "what": what}
        if key == "fp32_flash":
            comps[key]["fwd_frac_bf16_peak_executed"] = round(6 * ftf / PEAK_BF16_TFLOPS, 4)
            comps[key]["bwd_frac_bf16_peak_executed"] = round(6 * btf / PEAK_BF16_TFLOPS, 4)
    comps["dropout"] = {
        "p": 0.1, "fwd_ms": round(drop_ms[0], 5), "bwd_ms": round(drop_ms[1], 5),
        "fwd_tflops": round(FWD_FLOPS / (drop_ms[0] * 1e-3) / 1e12, 2),
        "bwd_tflops": round(BWD_FLOPS / (drop_ms[1] * 1e-3) / 1e12, 2)}
    comps["decode"] = {"us_per_launch": round(dec_ms * 1e3, 3), "bytes": wl.dec_bytes,
                       "gbps": round(dec_gbps, 1),
                       "frac_hbm_peak": round(dec_gbps / PEAK_HBM_GBPS, 4),
                       "eager_us_per_launch": round(eager_dec_ms * 1e3, 3),
                       "device_copy": {
                           "us": round(copy_ms * 1e3, 3),
                           "gbps_read_plus_write": round(copy_gbps, 1),
                           "what": "torch copy_ of a buffer of the decode's byte count (rotating "
                                   "sources, eager): the rate a vendor streaming kernel reaches "
                                   "on this box, to set gbps against"},
                       "uniform_lengths": dec_cases,
                       "cache_copies": wl.ncopy, "hbm_bytes_per_launch": traffic.get("decode"),
                       "config": "32 seqs, H12, D64, bf16 cache [32,12,1024,64], lens U[1,1024]"}

    if not args.no_generate:
        comps["generate_cfg5"] = generate_cfg5()

    dom = max(("fwd", "bwd_dq", "bwd_dkdv"), key=lambda n: kern_ms[n])
    ach = KERNEL_FLOPS[dom] / (kern_ms[dom] * 1e-3) / 1e12
    roofline = {"bound": "mfma", "kernel": dom, "achieved": round(ach, 2),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": traffic.get(dom),
                "traffic_source": traffic_src}

    value = (FWD_FLOPS + BWD_FLOPS) / (ms_step * 1e-3) / 1e12
    line = {
        "metric": "attn fwd/bwd TFLOP/s (B16 H12 T1024 D64 bf16); KV-decode HBM GB/s",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1), resident in HBM",
        "config": {"workload": "causal attention forward+backward, B16 H12 T1024 D64 "
                               "(BASELINE config 3)",
                   "B": B, "H": H, "T": T, "D": D, "scale": SCALE, "causal": True,
                   "dropout": 0.0},
        "roofline": roofline,
        "components": comps,
        "decode_gbps": round(dec_gbps, 1),
        "hip_stack": hip_stack(),
    }
    if not args.no_cpu_baseline:
        print(f"[bench] cpu baseline on {args.cpu_slices} slices ...", file=sys.stderr,
              flush=True)
        line["cpu_baseline"] = cpu_baseline(args.cpu_slices)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
