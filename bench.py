#!/usr/bin/env python3
"""Benchmark of grout's attention hot path on one MI355X.

Primary line (BASELINE.json metric): decode-attention HBM GB/s on the
Qwen3-32B-shaped decode step at 32k context (Hq=64, Hkv=8, D=128), one step =
split-K decode + LSE merge for one layer; the step rotates over 4 layer caches
(4 x 128 MiB of K+V > the 256 MB Infinity Cache) so K/V stream from HBM.
Also reported: prefill FMHA TFLOP/s (Qwen3-4B, S=2048), the 4B decode layer
and 36-layer graph step (ctx 4096), the fused QK-norm/RoPE/KV write, and the
CPU oracle baseline timed on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
# HBM bytes per split-kernel launch (Qwen3-32B, ctx 32768) by split count, measured with
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, scaled by a plain-copy calibration (x2.0, x1.0).
DECODE32B_TRAFFIC_BYTES = {32: 134.32e6 + 1.065e6}
DECODE32B_TRAFFIC_SOURCE = "profiles/attn_decode_split_qwen3-32b_ctx_sweep.md"
F16_MFMA_PEAK_TFLOPS = 2516.6  # MI355X dense fp16 MFMA, TFLOP/s
D = 128


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--only", default="",
                    help="comma list: decode32b,prefill,decode4b,shard,norm,engine4b,engine4b_q4km (gemv, qgemv, "
                         "engine4b_q5km: only when named)")
    ap.add_argument("--eager", action="store_true",
                    help="launch the timed calls from the host instead of replaying a captured "
                         "graph (for per-dispatch counter collection)")
    ap.add_argument("--decode-splits", type=int, default=None,
                    help="Qwen3-32B decode: this split count at every context instead of the "
                         "per-context sweep (1-4096)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a plain 256 MiB device copy (HBM counter calibration)")
    return ap.parse_args()


GRAPH_TIMING = True
# Untimed work before every timed region.  After idle the GPU's clocks take
# ~25 ms of continuous work to settle: S=2048 prefill FMHA measured 47.2, 43.1,
# 41.2, then 40.0-40.5 us per call over successive 200-call graph replays.
WARM_MS = 100.0


def warm_until(run_once, ms=WARM_MS):
    """Repeats run_once() (then synchronizes) until `ms` of wall time passed."""
    import torch

    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        run_once()
        torch.cuda.synchronize()


def time_launches(fn, steps, warmup, stream=None, graph=None):
    """Average device time per call of fn(i) over `steps` back-to-back calls,
    bracketed by HIP events recorded on the stream the kernels are launched on.
    With graph=True the `steps` calls are first captured into one HIP graph
    (the C ABI calls are capture-safe) so host launch overhead cannot leave the
    GPU idle between calls; the timed region is one replay of that graph.
    The `warmup` calls and at least WARM_MS of untimed repeats come first, so
    the timed region runs at settled clocks."""
    import torch

    graph = GRAPH_TIMING if graph is None else graph
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                fn(i)
        warm_until(g.replay)  # untimed replays
        s = torch.cuda.current_stream()
        start.record(s)
        g.replay()
        end.record(s)
    else:
        s = stream or torch.cuda.current_stream()
        warm_until(lambda: [fn(i) for i in range(min(steps, 50))])
        start.record(s)
        for i in range(steps):
            fn(i)
        end.record(s)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    if graph:
        del g
    return ms


def time_distribution(fn, calls=100, replays=20):
    """Spread of the per-call device time: `calls` back-to-back calls of fn(i)
    captured into one HIP graph, replayed `replays` times with a HIP event
    between consecutive replays on the replaying stream; p10 / median / p90 of
    the per-call average of each replay, in us (fn must already be warm).
    Each replay's average also carries the gap before that replay starts
    (~6.5 us on MI355X), i.e. ~0.07 us per call at 100 calls."""
    import numpy as np
    import torch

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(calls):
            fn(i)
    g.replay()  # untimed replay
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    ev[0].record(s)
    for r in range(replays):
        g.replay()
        ev[r + 1].record(s)
    torch.cuda.synchronize()
    us = np.array([ev[r].elapsed_time(ev[r + 1]) * 1e3 / calls for r in range(replays)])
    del g
    p10, med, p90 = np.percentile(us, (10, 50, 90))
    return dict(p10_us=round(float(p10), 3), median_us=round(float(med), 3),
                p90_us=round(float(p90), 3), calls_per_replay=calls, replays=replays)


class DecodeBench:
    """Decode attention over n_layers rotating layer caches [Hkv][max_ctx][128]
    (more bytes than the 256 MB Infinity Cache, so K/V stream from HBM); one
    step = one layer's split pass + merge (grout_attn_decode)."""

    def __init__(self, Hq, Hkv, max_ctx, n_layers):
        import torch

        dev = torch.device("cuda")
        g = torch.Generator(device=dev).manual_seed(1234)
        self.Hq, self.Hkv, self.max_ctx, self.n = Hq, Hkv, max_ctx, n_layers
        self.kcs = [torch.randn((Hkv, max_ctx, D), generator=g, device=dev, dtype=torch.float16)
                    for _ in range(n_layers)]
        self.vcs = [torch.randn((Hkv, max_ctx, D), generator=g, device=dev, dtype=torch.float16)
                    for _ in range(n_layers)]
        self.q = torch.randn((Hq, D), generator=g, device=dev, dtype=torch.float16)
        self.out = torch.empty_like(self.q)
        self.dev = dev

    def alg_bytes(self, ctx):
        return 2 * self.Hkv * ctx * D * 2 + 2 * self.Hq * D * 2

    def time_step(self, ctx, ns, steps, warmup, dist=False):
        import torch
        from grout_amd import ops

        pos = torch.tensor([ctx - 1], dtype=torch.int32, device=self.dev)
        ws = ops.decode_workspace(self.Hq, self.Hkv, ns, self.dev)

        def step(i=0):
            j = i % self.n
            ops.attn_decode(self.q, self.kcs[j], self.vcs[j], pos, num_splits=ns, out=self.out,
                            workspace=ws)

        ms = time_launches(step, steps, warmup)
        return (ms, time_distribution(step, calls=25 * self.n)) if dist else ms

    def time_split(self, ctx, ns, steps, warmup, dist=False):
        import ctypes as C
        import torch
        from grout_amd import ops
        from grout_amd._lib import call

        pos = torch.tensor([ctx - 1], dtype=torch.int32, device=self.dev)
        ws = ops.decode_workspace(self.Hq, self.Hkv, ns, self.dev)
        G = self.Hq // self.Hkv
        acc = ws[: self.Hkv * ns * G * D]
        ml = ws[self.Hkv * ns * G * D:]
        qp, pp = C.c_void_p(self.q.data_ptr()), C.c_void_p(pos.data_ptr())
        kps = [C.c_void_p(t.data_ptr()) for t in self.kcs]
        vps = [C.c_void_p(t.data_ptr()) for t in self.vcs]
        ap, mp = C.c_void_p(acc.data_ptr()), C.c_void_p(ml.data_ptr())

        def split_only(i=0):
            j = i % self.n
            sp = C.c_void_p(torch.cuda.current_stream().cuda_stream)  # the capture stream
            call("grout_fmha_decode_gqa_split", qp, kps[j], vps[j], ap, mp, pp, self.Hq,
                 self.Hkv, D, self.max_ctx, self.max_ctx * D, ns, 1.0 / math.sqrt(D), sp)

        ms = time_launches(split_only, steps, warmup)
        return (ms, time_distribution(split_only, calls=25 * self.n)) if dist else ms

    def close(self):
        import torch

        del self.kcs, self.vcs
        torch.cuda.empty_cache()


def bench_decode(ops, Hq, Hkv, ctx, max_ctx, n_layers, steps, warmup, num_splits=None):
    b = DecodeBench(Hq, Hkv, max_ctx, n_layers)
    ns = num_splits or ops.default_splits(max_ctx, Hq, Hkv)
    r = dict(step_ms=b.time_step(ctx, ns, steps, warmup),
             split_ms=b.time_split(ctx, ns, steps, warmup), alg_bytes=b.alg_bytes(ctx),
             num_splits=ns)
    b.close()
    return r


DECODE32B_SPLITS = (8, 16, 24, 32, 40, 48, 64)


def bench_decode32b_sweep(ops, ctxs, steps, warmup, sweep_steps=100, splits=None):
    """Config 4: Qwen3-32B decode attention (Hq=64, Hkv=8) at each context.
    The split count is swept first (sweep_steps graph-replayed steps of split
    pass + merge per candidate), as the reference tunes FMHA_NUM_KV_SPLITS per
    context (src/model.rs:135-141, benchmarks/sweep_tg_sm100.sh:32-43); the
    fastest is then timed afresh over `steps` steps, so the reported time is
    not the minimum of the sweep's samples.  splits: one count to use at every
    context instead of the sweep (e.g. under a profiler, whose per-dispatch
    overhead moves the sweep's pick)."""
    b = DecodeBench(64, 8, 32768, 4)
    out = {}
    for ctx in ctxs:
        sweep = {ns: b.time_step(ctx, ns, sweep_steps, warmup)
                 for ns in ((splits,) if splits else DECODE32B_SPLITS)}
        best = min(sweep, key=sweep.get)
        step_ms, step_dist = b.time_step(ctx, best, steps, warmup, dist=True)
        split_ms, split_dist = b.time_split(ctx, best, steps, warmup, dist=True)
        out[ctx] = dict(step_ms=step_ms, split_ms=split_ms, step_dist=step_dist,
                        split_dist=split_dist, alg_bytes=b.alg_bytes(ctx), num_splits=best,
                        default_splits=ops.default_splits(32768, 64, 8),
                        sweep_us={ns: round(ms * 1e3, 2) for ns, ms in sweep.items()})
        print(f"# decode32b ctx={ctx} best={best} {out[ctx]['sweep_us']}", file=sys.stderr,
              flush=True)
    b.close()
    return out


SHARD_KV_SPLITS = (32, 64, 128, 256)


def bench_shard(ops, steps, warmup, sweep_steps=100):
    """One GPU's share of a Qwen3-32B decode layer at 32k sharded over 8 GPUs,
    at its real shape (multi-GPU runs are outside this build).  kv-head
    sharding: each GPU holds one kv head and its 8 query heads (Hkv=1, Hq=8,
    ctx 32768, 24 rotating layer caches > the Infinity Cache), split count
    swept as for config 4.  Sequence sharding over 4 GPUs: each GPU runs the
    8192-position slice (the decode32b_sweep entry at ctx 8192, 32 splits)
    and, after the all-gather, the merge of 4 x 8 gathered partials, timed
    here alone."""
    import torch

    b = DecodeBench(8, 1, 32768, 24)
    ctx = 32768
    sweep = {ns: b.time_step(ctx, ns, sweep_steps, warmup) for ns in SHARD_KV_SPLITS}
    best = min(sweep, key=sweep.get)
    kv = dict(step_ms=b.time_step(ctx, best, steps, warmup),
              split_ms=b.time_split(ctx, best, steps, warmup), alg_bytes=b.alg_bytes(ctx),
              num_splits=best, sweep_us={ns: round(ms * 1e3, 2) for ns, ms in sweep.items()})
    b.close()
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(3)
    acc = torch.randn((8, 32, 8, D), generator=g, device=dev, dtype=torch.float32)
    ml = torch.stack([torch.randn((8, 32, 8), generator=g, device=dev),
                      torch.rand((8, 32, 8), generator=g, device=dev) + 1.0], -1)
    out = torch.empty((64, D), dtype=torch.float16, device=dev)
    merge_ms = time_launches(lambda i=0: ops.splitk_reduce_merge(acc, ml, out=out), steps, warmup)
    return dict(kv_head=kv, merge_ms=merge_ms)


def bench_decode_graph(grout_amd, Hq, Hkv, ctx, max_ctx, n_layers, steps, warmup):
    import torch
    from grout_amd.engine import AttentionConfig, AttentionEngine

    dev = torch.device("cuda")
    cfg = AttentionConfig(n_layers, Hq, Hkv, max_ctx=max_ctx)
    ones = [torch.ones(D, dtype=torch.float16, device=dev) for _ in range(n_layers)]
    eng = AttentionEngine(cfg, ones, ones, dev)
    g = torch.Generator(device=dev).manual_seed(7)
    for t in eng.k_caches + eng.v_caches:
        t.normal_(generator=g)
    graph = eng.build_decode_graph()
    for b in graph.qkv:
        b.normal_(generator=g)
    stream = torch.cuda.current_stream(dev)
    # consecutive positions centred on ctx, as a decode loop issues them: each
    # replay leaves the next position in the graph's word, so a step is one
    # hipGraphLaunch
    base = ctx - 1 - steps // 2
    ms = time_launches(lambda i=0: graph.launch_step(base + i), steps, warmup, stream, graph=False)
    graph.destroy()
    del eng
    torch.cuda.empty_cache()
    return ms


PREFILL_US_SOURCE = ("HIP events around one graph replay of the timed calls; us_dist spreads "
                     "20 replays of 100 calls, each replay's average carrying its ~6.5 us start gap")


def bench_prefill(ops, S, Hq, Hkv, steps, warmup):
    import torch

    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(99)
    q = torch.randn((S, Hq, D), generator=g, device=dev, dtype=torch.float16)
    kc = torch.randn((Hkv, S, D), generator=g, device=dev, dtype=torch.float16)
    vc = torch.randn((Hkv, S, D), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty_like(q)
    call = lambda i=0: ops.fmha_prefill(q, kc, vc, 0, out=out)
    ms = time_launches(call, steps, warmup, torch.cuda.current_stream(dev))
    flop = 4.0 * Hq * D * S * (S + 1) / 2
    return dict(ms=ms, flop=flop, dist=time_distribution(call, calls=100),
                plan=ops.prefill_plan(S, Hq, Hkv),
                library=bench_prefill_library(q, kc, vc, out, steps, warmup))


def bench_prefill_library(q, kc, vc, out, steps, warmup):
    """PyTorch's fused causal attention on the same inputs, as a vendor-library
    point of comparison: F.scaled_dot_product_attention restricted to its flash
    backend (on ROCm an AOTriton kernel), fp16, is_causal, K/V expanded to one
    copy per query head (the flash backend takes equal head counts).  Reported
    with the largest |difference| from this build's output."""
    import torch
    import torch.nn.functional as F

    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        S, Hq, _ = q.shape
        G = Hq // kc.shape[0]
        qt = q.permute(1, 0, 2).unsqueeze(0).contiguous()
        kt = kc[:, :S].repeat_interleave(G, 0).unsqueeze(0).contiguous()
        vt = vc[:, :S].repeat_interleave(G, 0).unsqueeze(0).contiguous()
        call = lambda i=0: F.scaled_dot_product_attention(qt, kt, vt, is_causal=True,
                                                          scale=D ** -0.5)
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            ref = call()
            ms = time_launches(call, steps, warmup, torch.cuda.current_stream(q.device), graph=False)
        diff = (ref[0].permute(1, 0, 2).float() - out.float()).abs().max().item()
        del qt, kt, vt, ref
        return dict(name="torch sdpa flash (AOTriton), K/V expanded to Hq heads", ms=ms,
                    max_abs_diff=diff)
    except Exception as e:  # noqa: BLE001 - reported, not fatal: a comparison only
        return dict(name="torch sdpa flash", error=f"{type(e).__name__}: {str(e)[:160]}")


def bench_norm(ops, S, Hq, Hkv, max_ctx, steps, warmup):
    import torch

    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(5)
    q = torch.randn((S, Hq, D), generator=g, device=dev, dtype=torch.float16)
    k = torch.randn((S, Hkv, D), generator=g, device=dev, dtype=torch.float16)
    v = torch.randn((S, Hkv, D), generator=g, device=dev, dtype=torch.float16)
    gam = torch.ones(D, dtype=torch.float16, device=dev)
    rope = ops.rope_tables(max_ctx, device=dev)
    kc = torch.zeros((Hkv, max_ctx, D), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    out = torch.empty_like(q)
    ms = time_launches(lambda i=0: ops.qk_norm_rope_kv_prefill(q, k, v, gam, gam, rope, kc, vc, 0,
                                                               out=out),
                       steps, warmup, torch.cuda.current_stream(dev))
    alg_bytes = 2 * S * (Hq + 2 * Hkv) * D * 2
    return dict(ms=ms, alg_bytes=alg_bytes)


def bench_fused_attention(Hq, Hkv, ctx, max_ctx, n_layers, steps, warmup):
    """Per-layer decode attention as the engine's decode graph runs it
    (grout_attn_decode_fused: norm/RoPE/KV write + split-K, then the merge),
    over n_layers rotating caches; ms per layer."""
    import torch
    from grout_amd import ops

    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(11)
    kcs = [torch.randn((Hkv, max_ctx, D), generator=g, device=dev, dtype=torch.float16)
           for _ in range(n_layers)]
    vcs = [torch.randn((Hkv, max_ctx, D), generator=g, device=dev, dtype=torch.float16)
           for _ in range(n_layers)]
    qkv = torch.randn(((Hq + 2 * Hkv) * D,), generator=g, device=dev, dtype=torch.float16)
    gam = torch.ones(D, dtype=torch.float16, device=dev)
    rope = ops.rope_tables(max_ctx, device=dev)
    pos = torch.tensor([ctx - 1], dtype=torch.int32, device=dev)
    out = torch.empty((Hq, D), dtype=torch.float16, device=dev)
    ns = ops.default_splits(max_ctx, Hq, Hkv)
    ws = ops.decode_workspace(Hq, Hkv, ns, dev)
    ms = time_launches(lambda i: ops.attn_decode_fused(qkv, gam, gam, rope, kcs[i % n_layers],
                                                       vcs[i % n_layers], pos, Hq, num_splits=ns,
                                                       out=out, workspace=ws),
                       steps, warmup)
    del kcs, vcs
    torch.cuda.empty_cache()
    return ms


def bench_engine(prompt_len=512, decode_steps=256, max_ctx=1024, cfg=None):
    """Config 5: Qwen3-4B-shaped engine (or `cfg`), random N(0, 0.02) fp16
    weights (norm weights 1), a seeded uniform prompt prefilled, then greedy
    decode steps, each one replay of the captured decode-step graph plus the
    4-byte token read-back (the public decode_greedy call, timed on the host
    clock)."""
    import numpy as np
    import torch
    from grout_amd.model import Engine, Qwen3Config, Qwen3Weights

    cfg = cfg or Qwen3Config.qwen3_4b()
    w = Qwen3Weights.random(cfg, seed=0)
    eng = Engine(cfg, w, max_ctx=max_ctx)
    prompt = np.random.default_rng(512).integers(0, cfg.vocab_size, prompt_len)
    eng.warmup()
    tok = eng.prefill_greedy(prompt)  # untimed: first rocBLAS calls pick their kernels
    for _ in range(8):
        tok = eng.decode_greedy(tok)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok = eng.prefill_greedy(prompt)
    prefill_s = time.perf_counter() - t0
    toks = [tok]
    t0 = time.perf_counter()
    for _ in range(decode_steps):
        toks.append(eng.decode_greedy(toks[-1]))
    decode_s = time.perf_counter() - t0
    eng.close()
    # whole-prompt prefill at the reference's published lengths, on an engine
    # with room for the longest (median of 3 after one untimed call each)
    eng = Engine(cfg, w, max_ctx=max(PREFILL_SWEEP_PP) + 1)
    pre_sweep = {}
    for pp in PREFILL_SWEEP_PP:
        pr = np.random.default_rng(pp).integers(0, cfg.vocab_size, pp)
        eng.prefill_greedy(pr)
        ts = []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            eng.prefill_greedy(pr)
            ts.append(time.perf_counter() - t0)
        pre_sweep[pp] = sorted(ts)[1] * 1e3
    eng.close()
    # per decode token: every fp16 weight once (the tied embedding is read as
    # the lm_head; the embedding gather is one row, so an untied embedding
    # does not count) + K and V of the live context
    embed_only = 0 if cfg.tie_word_embeddings else cfg.vocab_size * cfg.hidden_size
    weight_bytes = 2 * (cfg.num_params() - embed_only)
    mean_ctx = prompt_len + decode_steps / 2
    kv_bytes = cfg.num_layers * 2 * cfg.num_key_value_heads * mean_ctx * D * 2
    del w, eng
    torch.cuda.empty_cache()
    return dict(prefill_ms=prefill_s * 1e3, decode_ms=decode_s * 1e3 / decode_steps,
                tok_s=decode_steps / decode_s, bytes_per_token=weight_bytes + kv_bytes,
                distinct_tokens=len(set(toks)), mean_ctx=mean_ctx, prefill_sweep_ms=pre_sweep)


# Reference's published Qwen3-4B fp16 whole-prefill latency, median ms, grout
# tuned for one RTX 5090 (benchmarks/pytorch/README.md:32-38): other hardware,
# context for the sweep, not a baseline of this path.
PREFILL_SWEEP_PP = (18, 128, 512, 2048, 8192)
REFERENCE_4B_RTX5090_PREFILL_MS = {18: 6.31, 128: 7.39, 512: 14.50, 2048: 50.69, 8192: 279.12}


# Reference's published request_gen_tps for Qwen3-32B on one B200
# (benchmarks/RESULTS.md:25-59): (pp, tg) -> grout's median.  Whole-model
# figures on other hardware: context for the sweep below, not a baseline of
# this path.
REFERENCE_32B_B200 = {(18, 36): 79.6, (18, 128): 79.9, (18, 512): 80.1, (128, 36): 79.0,
                      (512, 36): 75.3, (2048, 36): 61.4, (8192, 36): 37.2}


def bench_engine32b(reps=3):
    """Qwen3-32B-shaped engine (64 layers, hidden 5120, MLP 25600, 64/8 heads,
    untied head; 65.5 GB of random N(0, 0.02) fp16 weights) driven through
    the reference's request sweep: each request prefills a seeded uniform
    prompt of pp tokens (the first generated token) and decodes tg - 1 more
    greedily; request_gen_tps = tg / end-to-end time, the reference's
    definition (benchmarks/aggregate_sweep.py:23), median of `reps` requests
    after one untimed request per prompt length."""
    import numpy as np
    import torch
    from grout_amd.model import Engine, Qwen3Config, Qwen3Weights

    cfg = Qwen3Config(64, 5120, 25600, 64, 8, 151936, tie_word_embeddings=False)
    w = Qwen3Weights.random(cfg, seed=0)
    eng = Engine(cfg, w, max_ctx=8192 + 64)
    rng = np.random.default_rng(512)
    eng.warmup()

    def request(pp, tg):
        prompt = rng.integers(0, cfg.vocab_size, pp)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tok = eng.prefill_greedy(prompt)
        t1 = time.perf_counter()
        for _ in range(tg - 1):
            tok = eng.decode_greedy(tok)
        t2 = time.perf_counter()
        return (t1 - t0) * 1e3, (t2 - t0) * 1e3

    out = []
    for pp, tg in REFERENCE_32B_B200:
        request(pp, 36 if pp > 18 else 8)  # untimed: rocBLAS picks its kernels per shape
        runs = sorted((request(pp, tg) for _ in range(reps)), key=lambda r: r[1])
        pre, e2e = runs[len(runs) // 2]
        out.append(dict(pp=pp, tg=tg, prefill_ms=round(pre, 2), e2e_ms=round(e2e, 1),
                        decode_ms_per_token=round((e2e - pre) / (tg - 1), 4),
                        request_gen_tps=round(tg * 1e3 / e2e, 1),
                        reference_b200_request_gen_tps=REFERENCE_32B_B200[(pp, tg)]))
        print(f"# engine32b {out[-1]}", file=sys.stderr, flush=True)
    eng.close()
    weight_bytes = 2 * (cfg.num_params() - cfg.vocab_size * cfg.hidden_size)
    del w, eng
    torch.cuda.empty_cache()
    return dict(requests=out, weight_bytes=weight_bytes)


def q4km_formats(n_layers, base=12):
    """Q4_K_M-style mix: attn_v and ffn_down in Q6_K for the first and last
    eighth of the layers and every third layer between, Q4_K elsewhere (base=13:
    the Q5_K_M mix, Q5_K in place of Q4_K)."""
    Q4, Q6 = base, 14

    def more_bits(l):
        return l < n_layers // 8 or l >= 7 * n_layers // 8 or (l - n_layers // 8) % 3 == 2

    def fmts(l):
        hi = Q6 if more_bits(l) else Q4
        return {"q": Q4, "k": Q4, "v": hi, "o": Q4, "gate": Q4, "up": Q4, "down": hi}
    return fmts


def bench_engine_q(prompt_len=512, decode_steps=256, max_ctx=1024, base=12):
    """Config 5 over low-bit weights: the Qwen3-4B engine with random
    GGUF-block weights in a Q4_K_M-style mix (q4km_formats; Q6_K tied
    embedding / lm_head; base=13 for the Q5_K_M mix), prompt and timing as
    bench_engine."""
    import numpy as np
    import torch
    from grout_amd.model import Engine, QuantWeights, Qwen3Config

    cfg = Qwen3Config.qwen3_4b()
    qw = QuantWeights.random(cfg, q4km_formats(cfg.num_layers, base), embed_fmt=14, seed=0)
    torch.cuda.synchronize()
    eng = Engine.from_quantized(cfg, qw, max_ctx=max_ctx)
    prompt = np.random.default_rng(512).integers(0, cfg.vocab_size, prompt_len)
    eng.warmup()
    tok = eng.prefill_greedy(prompt)
    for _ in range(8):
        tok = eng.decode_greedy(tok)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok = eng.prefill_greedy(prompt)
    prefill_s = time.perf_counter() - t0
    toks = [tok]
    t0 = time.perf_counter()
    for _ in range(decode_steps):
        toks.append(eng.decode_greedy(toks[-1]))
    decode_s = time.perf_counter() - t0
    eng.close()
    # per decode token: every repacked weight byte once (the tied table is
    # read whole by the lm_head GEMV) + K and V of the live context
    weight_bytes = qw.device_bytes()
    mean_ctx = prompt_len + decode_steps / 2
    kv_bytes = cfg.num_layers * 2 * cfg.num_key_value_heads * mean_ctx * D * 2
    del qw, eng
    torch.cuda.empty_cache()
    return dict(prefill_ms=prefill_s * 1e3, decode_ms=decode_s * 1e3 / decode_steps,
                tok_s=decode_steps / decode_s, bytes_per_token=weight_bytes + kv_bytes,
                weight_bytes=weight_bytes, distinct_tokens=len(set(toks)), mean_ctx=mean_ctx)


def bench_gemv(steps, warmup):
    """The decode step's projections on Qwen3-4B shapes, each over 8 rotating
    weight copies (> the 256 MB Infinity Cache for all but the smallest), as
    called in the decode graph (fused norm / SiLU inputs included)."""
    import ctypes as C
    import torch
    from grout_amd._lib import call

    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(3)
    H, I, QKV, Q, V = 2560, 9728, 6144, 4096, 151936
    # name: (weight rows, K, mode); gate_up_norm_silu writes I outputs
    shapes = {"qkv_norm": (QKV, H, "norm"), "o_proj": (H, Q, "plain"),
              "gate_up_norm_silu": (2 * I, H, "silu"), "down": (H, I, "plain"),
              "lm_head": (V, H, "plain")}
    out = {}
    for name, (n, k, mode) in shapes.items():
        copies = 1 if name == "lm_head" else 8
        Ws = [torch.empty((n, k), dtype=torch.float16, device=dev).normal_(0, 0.02, generator=g)
              for _ in range(copies)]
        x = torch.randn(2 * k, dtype=torch.float16, device=dev, generator=g)
        r = torch.randn(k, dtype=torch.float16, device=dev, generator=g)
        gam = torch.ones(k, dtype=torch.float16, device=dev)
        ro = torch.empty(k, dtype=torch.float16, device=dev)
        y = torch.empty(n, dtype=torch.float16, device=dev)
        P = lambda t: C.c_void_p(t.data_ptr())

        def fn(i, Ws=Ws, x=x, r=r, gam=gam, ro=ro, y=y, n=n, k=k, mode=mode):
            s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
            W = P(Ws[i % len(Ws)])
            if mode == "plain":
                call("grout_gemv", W, P(x), P(y), n, k, s)
            elif mode == "norm":
                call("grout_gemv_rms_norm", W, P(r), P(x), P(gam), P(ro), P(y), n, k,
                     C.c_float(1e-6), s)
            else:
                call("grout_gemv_rms_norm_silu_mul", W, P(r), P(x), P(gam), P(ro), P(y), n // 2,
                     k, C.c_float(1e-6), s)

        ms = time_launches(fn, steps, warmup)
        out[name] = dict(us=round(ms * 1e3, 2), gbs=round(n * k * 2 / (ms * 1e-3) / 1e9, 1))
        del Ws
        torch.cuda.empty_cache()
    return out


def bench_qgemv(steps, warmup):
    """The low-bit GEMVs (Q8_0 / Q4_K / Q5_K / Q6_K) on the Qwen3-4B decode shapes:
    random ggml payloads (block scales set to 0.01) repacked once, then timed
    over enough rotating copies that more than 600 MB of weights cycle (past
    the 256 MB Infinity Cache).  GB/s counts the repacked weight bytes read
    per launch plus the f16 input and output."""
    import ctypes as C
    import torch
    from grout_amd._lib import call, lib

    L = lib()
    dev = torch.device("cuda")
    H, I, QKV, Q, V = 2560, 9728, 6144, 4096, 151936
    shapes = {"qkv": (QKV, H, False), "o_proj": (H, Q, False), "gate_up_silu": (2 * I, H, True),
              "down": (H, I, False), "lm_head": (V, H, False)}
    fmts = {"Q8_0": (8, 32, 34, 0), "Q4_K": (12, 256, 144, 0), "Q5_K": (13, 256, 176, 0),
            "Q6_K": (14, 256, 210, 208)}
    P = lambda t: C.c_void_p(t.data_ptr())
    d_bytes = torch.tensor([0.01], dtype=torch.float16).view(torch.uint8).to(dev)
    out = {}
    for fname, (fmt, be, bb, d_off) in fmts.items():
        res = {}
        for name, (n, k, silu) in shapes.items():
            nbytes = L.grout_qweight_bytes(fmt, n, k)
            copies = max(1, min(8, -(-600_000_000 // nbytes)))
            Ws = []
            for c in range(copies):
                raw = torch.randint(0, 256, (n * k // be, bb), dtype=torch.uint8, device=dev)
                raw[:, d_off:d_off + 2] = d_bytes
                if fmt in (12, 13):
                    raw[:, 2:4] = d_bytes
                w = torch.empty(nbytes, dtype=torch.uint8, device=dev)
                call("grout_qweight_repack", fmt, P(raw), n, k, P(w), None)
                Ws.append(w)
                del raw
            x = (torch.randn(k, device=dev) * 0.1).to(torch.float16)
            y = torch.empty(n, dtype=torch.float16, device=dev)

            def fn(i, Ws=Ws, x=x, y=y, n=n, k=k, silu=silu, fmt=fmt):
                s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
                if silu:
                    call("grout_gemv_q_silu_mul", fmt, P(Ws[i % len(Ws)]), P(x), P(y), n // 2, k, s)
                else:
                    call("grout_gemv_q", fmt, P(Ws[i % len(Ws)]), P(x), P(y), n, k, s)

            ms = time_launches(fn, steps, warmup)
            moved = nbytes + 2 * k + 2 * (n // 2 if silu else n)
            res[name] = dict(us=round(ms * 1e3, 2), gbs=round(moved / (ms * 1e-3) / 1e9, 1),
                             weight_bytes=nbytes)
            del Ws
            torch.cuda.empty_cache()
        res["step_weight_us"] = round(36 * sum(res[s]["us"] for s in ("qkv", "o_proj", "gate_up_silu",
                                                                       "down")) + res["lm_head"]["us"], 1)
        out[fname] = res
    return out


def host_cpu():
    """CPU model name, logical CPU count and the CPUs this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return model, os.cpu_count() or 1, usable


def cpu_threads(limit):
    """All-core thread count: the CPUs this process may use, capped by
    OMP_NUM_THREADS when set (the GPU box's CPU share) and by `limit`."""
    _, _, usable = host_cpu()
    n = usable
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, min(n, limit))


def _timed(fn, min_s, max_reps=1000):
    t0 = time.perf_counter()
    reps = 0
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_s or reps >= max_reps:
            return dt / reps, reps


def cpu_baseline(Hq=64, Hkv=8, ctx=32768, S=2048, pHq=32, pHkv=8):
    """The scalar fp32 oracle (oracle/grout_oracle.c, gcc -O2, no fast-math)
    timed on this host's cores on the same workloads as the GPU lines:
    * decode: one full Qwen3-32B layer (Hq=64, Hkv=8) at ctx 32768, single
      thread and all-core (threads over query heads); GB/s of the same
      algorithmic bytes as the GPU line;
    * prefill: Qwen3-4B causal attention at S=2048 on sampled rows (every 32nd
      row, all 32 heads), all-core; TFLOP/s over those rows' exact
      4*Hq*128*(row+1) FLOP."""
    import numpy as np

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle as O

    model, ncpu, usable = host_cpu()
    nthr = cpu_threads(Hq)
    q = O.fill_normal_f16(O.seed_for("bq"), (Hq, D))
    kc = O.fill_normal_f16(O.seed_for("bk"), (Hkv, ctx, D))
    vc = O.fill_normal_f16(O.seed_for("bv"), (Hkv, ctx, D))
    alg = 2 * Hkv * ctx * D * 2 + 2 * Hq * D * 2
    t1, r1 = _timed(lambda: O.attention_decode(q, kc, vc, ctx - 1, nthreads=1), 4.0)
    tn, rn = _timed(lambda: O.attention_decode(q, kc, vc, ctx - 1, nthreads=nthr), 4.0)
    del kc, vc
    pq = O.fill_normal_f16(O.seed_for("pbq"), (S, pHq, D))
    pk = O.fill_normal_f16(O.seed_for("pbk"), (pHkv, S, D))
    pv = O.fill_normal_f16(O.seed_for("pbv"), (pHkv, S, D))
    rows = np.arange(31, S, 32, dtype=np.int32)
    pflop = float(sum(4.0 * pHq * D * (int(r) + 1) for r in rows))
    pthr = cpu_threads(pHq)
    tp, rp = _timed(lambda: O.attention_prefill_rows(pq, pk, pv, 0, rows=rows, nthreads=pthr),
                    3.0)
    tp1, rp1 = _timed(lambda: O.attention_prefill_rows(pq, pk, pv, 0, rows=rows[::8],
                                                       nthreads=1), 2.0)
    pflop1 = float(sum(4.0 * pHq * D * (int(r) + 1) for r in rows[::8]))
    return dict(
        value=alg / tn / 1e9, unit="GB/s", cores=nthr, kind="port",
        sample=f"oracle/grout_oracle.c go_attention_decode, one full Qwen3-32B decode layer "
               f"(Hq={Hq}, Hkv={Hkv}, ctx {ctx}), {nthr} threads over query heads, "
               f"{rn} reps of {tn * 1e3:.1f} ms",
        cpu_model=model, cpu_count=ncpu, cpus_usable=usable,
        layer_ms=tn * 1e3,
        single_thread={"value": alg / t1 / 1e9, "unit": "GB/s", "cores": 1,
                       "layer_ms": t1 * 1e3, "reps": r1},
        prefill={"workload": f"qwen3-4b causal prefill attention S={S} Hq={pHq} Hkv={pHkv}, "
                             f"{len(rows)} sampled rows (every 32nd), all heads",
                 "tflops": pflop / tp / 1e12, "cores": pthr, "ms": tp * 1e3, "reps": rp,
                 "single_thread_tflops": pflop1 / tp1 / 1e12,
                 "single_thread_rows": int(len(rows[::8]))})


def guarded(fn):
    """Runs one secondary bench section.  A Python-level failure (out of
    memory, an argument error) is printed to stderr and returned as
    {"error": ...}, which the JSON line carries, so the headline measurement
    still reaches the line.  The headline section itself is not guarded."""
    import traceback

    import torch

    try:
        return fn()
    except Exception as ex:  # noqa: BLE001 - recorded in the line
        traceback.print_exc()
        torch.cuda.empty_cache()
        return {"error": f"{type(ex).__name__}: {ex}"[:400]}


def assemble_line(res, steps, warmup, cpu=None):
    """The one JSON line from the measured sections in `res` (each as its
    bench function returns it, or {"error": ...}) and the CPU baseline."""
    line = {"metric": "decode-attn HBM GB/s (% of peak) + prefill FMHA TFLOP/s (% MFMA peak)",
            "n_gpus": 1, "steps": steps, "warmup": warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic"}
    if "decode32b" in res:
        r = res["decode32b"]
        gbs = r["alg_bytes"] / (r["step_ms"] * 1e-3) / 1e9
        # the roofline's kernel time: median per-call time over 20 graph
        # replays of 100 split-kernel launches each (robust against one
        # replay's clock or queueing outlier)
        split_med_us = r["split_dist"]["median_us"]
        split_gbs = r["alg_bytes"] / (split_med_us * 1e-6) / 1e9
        line.update(value=round(gbs, 1), unit="GB/s", ms_per_step=round(r["step_ms"], 5))
        line["config"] = {"workload": "qwen3-32b decode attention (split-K + LSE merge), Hq=64 "
                                      "Hkv=8 D=128, ctx 32768, batch 1, 4 rotating layer caches",
                          "num_splits": r["num_splits"], "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                          "step_us_dist": r["step_dist"]}
        traffic = DECODE32B_TRAFFIC_BYTES.get(r["num_splits"])
        line["roofline"] = {"bound": "hbm", "kernel": "attn_decode_split_kernel",
                            "achieved": round(split_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(split_gbs / HBM_PEAK_GBS, 4),
                            "traffic": traffic,
                            "traffic_source": DECODE32B_TRAFFIC_SOURCE if traffic else None,
                            "kernel_us": split_med_us,
                            "kernel_us_source": "median_us of kernel_us_dist (per-call average "
                                                "of each of 20 graph replays x 100 launches)",
                            "kernel_us_dist": r["split_dist"],
                            "alg_bytes_per_launch": r["alg_bytes"]}
        sweep = {}
        for ctx, rr in res["decode32b_sweep"].items():
            g = rr["alg_bytes"] / (rr["step_ms"] * 1e-3) / 1e9
            sg = rr["alg_bytes"] / (rr["split_ms"] * 1e-3) / 1e9
            sweep[str(ctx)] = {"num_splits": rr["num_splits"], "step_us": round(rr["step_ms"] * 1e3, 2),
                               "step_gbs": round(g, 1), "step_hbm_frac": round(g / HBM_PEAK_GBS, 4),
                               "split_us": round(rr["split_ms"] * 1e3, 2),
                               "split_gbs": round(sg, 1), "split_hbm_frac": round(sg / HBM_PEAK_GBS, 4),
                               "step_us_dist": rr["step_dist"], "split_us_dist": rr["split_dist"],
                               "alg_bytes": rr["alg_bytes"], "splits_swept_us": rr["sweep_us"]}
        line["decode32b_sweep"] = sweep
    def ok(key):
        return key in res and "error" not in res[key]

    if ok("prefill"):
        r = res["prefill"]
        tf = r["flop"] / (r["ms"] * 1e-3) / 1e12
        line["prefill"] = {"workload": "qwen3-4b causal prefill FMHA S=2048 Hq=32 Hkv=8 D=128",
                           "us": round(r["ms"] * 1e3, 2), "tflops": round(tf, 1),
                           "mfma_frac": round(tf / F16_MFMA_PEAK_TFLOPS, 4),
                           "flop": r["flop"], "us_source": PREFILL_US_SOURCE, "us_dist": r["dist"],
                           "work_split": r["plan"]}
        sweep = {}
        for S, rr in res["prefill_sweep"].items():
            t = rr["flop"] / (rr["ms"] * 1e-3) / 1e12
            sweep[str(S)] = {"us": round(rr["ms"] * 1e3, 2), "tflops": round(t, 1),
                             "mfma_frac": round(t / F16_MFMA_PEAK_TFLOPS, 4), "flop": rr["flop"],
                             "us_dist": rr["dist"], "work_split": rr["plan"]}
            lib = rr.get("library") or {}
            if "ms" in lib:
                lt = rr["flop"] / (lib["ms"] * 1e-3) / 1e12
                sweep[str(S)]["library"] = {"name": lib["name"], "us": round(lib["ms"] * 1e3, 2),
                                            "tflops": round(lt, 1),
                                            "max_abs_diff": round(lib["max_abs_diff"], 6)}
            elif lib:
                sweep[str(S)]["library"] = lib
        line["prefill_sweep"] = sweep
    if ok("decode4b"):
        r = res["decode4b"]
        gbs = r["alg_bytes"] / (r["step_ms"] * 1e-3) / 1e9
        line["decode4b"] = {"workload": "qwen3-4b decode attention Hq=32 Hkv=8 ctx 4096, 36 layer caches",
                            "us_per_layer": round(r["step_ms"] * 1e3, 2), "gbs": round(gbs, 1),
                            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "num_splits": r["num_splits"],
                            "graph_36_layers_us": round(r["graph_ms"] * 1e3, 1)}
    if ok("shard"):
        r = res["shard"]
        kv = r["kv_head"]
        gbs = kv["alg_bytes"] / (kv["step_ms"] * 1e-3) / 1e9
        sgbs = kv["alg_bytes"] / (kv["split_ms"] * 1e-3) / 1e9
        seq = line.get("decode32b_sweep", {}).get("8192", {})
        line["shard"] = {
            "workload": "one GPU's share of a qwen3-32b decode layer at ctx 32768 sharded over "
                        "GPUs (design only: no multi-GPU run in this build)",
            "kv_head_8way": {"shape": "Hq=8 Hkv=1 ctx 32768, 24 layer caches",
                             "num_splits": kv["num_splits"],
                             "step_us": round(kv["step_ms"] * 1e3, 2),
                             "step_gbs": round(gbs, 1), "step_hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                             "split_us": round(kv["split_ms"] * 1e3, 2),
                             "split_hbm_frac": round(sgbs / HBM_PEAK_GBS, 4),
                             "splits_swept_us": kv["sweep_us"]},
            "sequence_4way": {"slice": "Hq=64 Hkv=8, 8192 positions per GPU, 32 splits: the "
                                       "decode32b_sweep entry at ctx 8192",
                              "slice_split_us": seq.get("split_us"),
                              "merge_of_4x8_gathered_partials_us": round(r["merge_ms"] * 1e3, 2)}}
    if ok("norm"):
        r = res["norm"]
        gbs = r["alg_bytes"] / (r["ms"] * 1e-3) / 1e9
        line["qk_norm_rope_kv"] = {"workload": "fused QK-norm/RoPE/KV write S=2048 Hq=32 Hkv=8",
                                   "us": round(r["ms"] * 1e3, 2), "gbs": round(gbs, 1),
                                   "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if "gemv" in res:
        line["gemv"] = res["gemv"]
    if "qgemv" in res:
        line["qgemv"] = res["qgemv"]
    if ok("engine4b"):
        r = res["engine4b"]
        gbs = r["bytes_per_token"] * r["tok_s"] / 1e9
        line["engine4b"] = {
            "workload": "qwen3-4b engine, random N(0,0.02) fp16 weights, 512-token prompt, "
                        "256 greedy decode steps (decode-step hipGraph)",
            "decode_tok_s": round(r["tok_s"], 1), "decode_ms_per_token": round(r["decode_ms"], 4),
            "prefill_512_ms": round(r["prefill_ms"], 2),
            "prefill_sweep": {str(pp): {"ms": round(ms, 2), "tok_s": round(pp / ms * 1e3, 1),
                                        "reference_rtx5090_ms": REFERENCE_4B_RTX5090_PREFILL_MS[pp]}
                              for pp, ms in r["prefill_sweep_ms"].items()},
            "prefill_sweep_context": "whole-prompt prefill (embedding to last-token logits, "
                                     "median of 3); reference_rtx5090_ms: grout's published "
                                     "medians on one RTX 5090 (benchmarks/pytorch/README.md:"
                                     "32-38; other hardware)",
            "weight_stream_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "attention_share": round(r["attn_graph_ms"] / r["decode_ms"], 4),
            "attention_us_per_token": round(r["attn_graph_ms"] * 1e3, 1)}
    if ok("engine32b"):
        r = res["engine32b"]
        head = next(q for q in r["requests"] if (q["pp"], q["tg"]) == (18, 128))
        gbs = r["weight_bytes"] / (head["decode_ms_per_token"] * 1e-3) / 1e9
        line["engine32b"] = {
            "workload": "qwen3-32b engine, random N(0,0.02) fp16 weights (untied head); requests "
                        "of pp prompt tokens + tg generated (greedy, decode-step hipGraph)",
            "decode_tok_s": round(1e3 / head["decode_ms_per_token"], 1),
            "decode_ms_per_token": head["decode_ms_per_token"],
            "weight_stream_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "requests": r["requests"],
            "reference_context": "reference_b200_request_gen_tps: grout's published medians on "
                                 "one B200 (benchmarks/RESULTS.md:25-59; whole model, other "
                                 "hardware)"}
    if ok("engine4b_q4km"):
        r = res["engine4b_q4km"]
        gbs = r["bytes_per_token"] * r["tok_s"] / 1e9
        line["engine4b_q4km"] = {
            "workload": "qwen3-4b engine, random GGUF-block weights in a Q4_K_M-style mix "
                        "(Q4_K; attn_v / ffn_down Q6_K in 18 of 36 layers; Q6_K tied embedding), "
                        "512-token prompt, 256 greedy decode steps (decode-step hipGraph)",
            "decode_tok_s": round(r["tok_s"], 1), "decode_ms_per_token": round(r["decode_ms"], 4),
            "prefill_512_ms": round(r["prefill_ms"], 2),
            "weight_bytes": r["weight_bytes"],
            "weight_stream_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    if ok("engine4b_q5km"):
        r = res["engine4b_q5km"]
        gbs = r["bytes_per_token"] * r["tok_s"] / 1e9
        line["engine4b_q5km"] = {
            "workload": "qwen3-4b engine, random GGUF-block weights in a Q5_K_M-style mix "
                        "(Q5_K; attn_v / ffn_down Q6_K in 18 of 36 layers; Q6_K tied embedding), "
                        "512-token prompt, 256 greedy decode steps (decode-step hipGraph)",
            "decode_tok_s": round(r["tok_s"], 1), "decode_ms_per_token": round(r["decode_ms"], 4),
            "prefill_512_ms": round(r["prefill_ms"], 2),
            "weight_bytes": r["weight_bytes"],
            "weight_stream_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
    # sections that failed carry their error instead of numbers
    names = {"prefill_error": "prefill", "norm": "qk_norm_rope_kv"}
    for key, v in res.items():
        if isinstance(v, dict) and "error" in v:
            line[names.get(key, key)] = v
    if cpu is not None:
        def rnd(v):
            if isinstance(v, float):
                return round(v, 4)
            if isinstance(v, dict):
                return {k: rnd(x) for k, x in v.items()}
            return v
        line["cpu_baseline"] = rnd(cpu)
    return line


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(requested --gpus {a.gpus}); run with --gpus 1", file=sys.stderr)
        return 2
    if a.decode_splits is not None and not 1 <= a.decode_splits <= 4096:
        print(f"--decode-splits {a.decode_splits}: the split count must be in [1, 4096]",
              file=sys.stderr)
        return 2
    import torch
    import grout_amd
    from grout_amd import ops

    global GRAPH_TIMING
    GRAPH_TIMING = not a.eager
    grout_amd.lib()
    if a.copy_calib:
        src = torch.ones(128 << 20, dtype=torch.float16, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"# copy_calib: 3 copies of {src.numel() * 2} bytes", file=sys.stderr, flush=True)
        del src, dst
    only = set(filter(None, a.only.split(",")))
    want = lambda k: not only or k in only
    res = {}
    if want("decode32b"):
        res["decode32b_sweep"] = bench_decode32b_sweep(ops, (8192, 16384, 32768), a.steps,
                                                       a.warmup, splits=a.decode_splits)
        res["decode32b"] = res["decode32b_sweep"][32768]
        print(f"# decode32b {res['decode32b']}", file=sys.stderr, flush=True)
    if want("prefill"):
        sweep = guarded(lambda: {S: bench_prefill(ops, S, 32, 8,
                                                  max(a.steps // (4 if S < 8192 else 10), 10),
                                                  a.warmup)
                                 for S in (512, 2048, 8192)})
        if "error" in sweep:
            res["prefill_error"] = sweep
        else:
            res["prefill_sweep"] = sweep
            res["prefill"] = sweep[2048]
        print(f"# prefill {sweep}", file=sys.stderr, flush=True)
    if want("decode4b"):
        def decode4b():
            r = bench_decode(ops, 32, 8, 4096, 32768, 36, a.steps, a.warmup)
            r["graph_ms"] = bench_decode_graph(grout_amd, 32, 8, 4096, 32768, 36,
                                               max(a.steps // 4, 10), a.warmup)
            return r
        res["decode4b"] = guarded(decode4b)
        print(f"# decode4b {res['decode4b']}", file=sys.stderr, flush=True)
    if want("shard"):
        res["shard"] = guarded(lambda: bench_shard(ops, a.steps, a.warmup))
        print(f"# shard {res['shard']}", file=sys.stderr, flush=True)
    if want("norm"):
        res["norm"] = guarded(lambda: bench_norm(ops, 2048, 32, 8, 32768, a.steps, a.warmup))
        print(f"# norm {res['norm']}", file=sys.stderr, flush=True)
    if "gemv" in only:
        res["gemv"] = bench_gemv(a.steps, a.warmup)
        print(f"# gemv {res['gemv']}", file=sys.stderr, flush=True)
    if "qgemv" in only:
        res["qgemv"] = bench_qgemv(a.steps, a.warmup)
        print(f"# qgemv {res['qgemv']}", file=sys.stderr, flush=True)
    if want("engine4b"):
        def engine4b():
            r = bench_engine()
            # attention part of one decode step at the mean context of the run:
            # 36 layers of the fused norm/RoPE/KV write + split-K + merge
            r["attn_graph_ms"] = 36 * bench_fused_attention(
                32, 8, int(r["mean_ctx"]), 1024, 36, a.steps, a.warmup)
            return r
        res["engine4b"] = guarded(engine4b)
        print(f"# engine4b {res['engine4b']}", file=sys.stderr, flush=True)
    if want("engine32b"):
        res["engine32b"] = guarded(bench_engine32b)
    if want("engine4b_q4km"):
        res["engine4b_q4km"] = guarded(bench_engine_q)
        print(f"# engine4b_q4km {res['engine4b_q4km']}", file=sys.stderr, flush=True)
    if "engine4b_q5km" in only:
        res["engine4b_q5km"] = guarded(lambda: bench_engine_q(base=13))
        print(f"# engine4b_q5km {res['engine4b_q5km']}", file=sys.stderr, flush=True)

    cb = guarded(cpu_baseline) if not a.no_cpu and "decode32b" in res else None
    print(json.dumps(assemble_line(res, a.steps, a.warmup, cb)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
