"""GPU parity of the gfx950 kernels (through the C ABI) against the CPU oracle.

Inputs come from the oracle's seeded SplitMix64/Box-Muller generator.  Bars:
K/V cache rows and indexing bit-exact; attention outputs within max-abs 1e-2
and mean-abs 1e-3 of the fp32 oracle."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import D, assert_close, dev, gamma, host, host_f32, normal

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


# ------------------------------------------------------------------ layout


def test_mfma_layout_probe(gpu):
    out = gpu.ops.diag_mfma_layout().cpu().numpy()
    for l in range(64):
        for j in range(4):
            m, n = 4 * (l // 16) + j, l % 16  # C fragment: col l%16, rows 4*(l/16)+j
            # A row m, k-slot n//8 is held by lane m + 16*(n//8) at element n%8
            assert out[l, j] == (m + 16 * (n // 8)) * 8 + n % 8, (l, j, out[l, j])


# ------------------------------------------------- fused norm / RoPE / KV write


@pytest.mark.parametrize("S,Hq,Hkv,pos0,max_ctx", [
    (1, 16, 8, 0, 64), (37, 32, 8, 100, 256), (64, 40, 8, 5, 128), (2048, 32, 8, 0, 32768)])
def test_qk_norm_rope_kv_prefill_bit_exact(gpu, S, Hq, Hkv, pos0, max_ctx):
    _say("norm_rope_prefill", S, Hq, Hkv, pos0, max_ctx)
    q, k, v = normal("nq", (S, Hq, D)), normal("nk", (S, Hkv, D)), normal("nv", (S, Hkv, D))
    gq, gk = gamma("gq"), gamma("gk")
    cos, sin = O.rope_table(max_ctx, D, 1e6)
    kc = np.full((Hkv, max_ctx, D), 0x7BFF, np.uint16)  # canary in every slot
    vc = kc.copy()
    kc_ref, vc_ref = kc.copy(), vc.copy()
    q_ref = O.qk_norm_rope_kv_prefill(q, k, v, gq, gk, cos, sin, kc_ref, vc_ref, pos0, 1e-6)

    rope = gpu.ops.rope_tables(max_ctx)
    kc_d, vc_d = dev(kc), dev(vc)
    q_out = gpu.ops.qk_norm_rope_kv_prefill(dev(q), dev(k), dev(v), dev(gq), dev(gk), rope, kc_d,
                                            vc_d, pos0)
    torch.cuda.synchronize()
    assert np.array_equal(host(q_out), q_ref), "rotated q differs"
    assert np.array_equal(host(kc_d), kc_ref), "k cache differs (incl. untouched canary slots)"
    assert np.array_equal(host(vc_d), vc_ref), "v cache differs (incl. untouched canary slots)"


@pytest.mark.parametrize("Hq,Hkv,pos,max_ctx", [(16, 8, 512, 1024), (64, 8, 32767, 32768), (32, 8, 0, 64)])
def test_qk_norm_rope_kv_decode_bit_exact(gpu, Hq, Hkv, pos, max_ctx):
    _say("norm_rope_decode", Hq, Hkv, pos, max_ctx)
    qkv = normal("dqkv", ((Hq + 2 * Hkv) * D,))
    gq, gk = gamma("gq"), gamma("gk")
    cos, sin = O.rope_table(max_ctx, D, 1e6)
    kc = normal("dkc", (Hkv, max_ctx, D))
    vc = normal("dvc", (Hkv, max_ctx, D))
    kc_ref, vc_ref = kc.copy(), vc.copy()
    q_ref = O.qk_norm_rope_kv_decode(qkv, gq, gk, cos, sin, kc_ref, vc_ref, pos, Hq, Hkv, 1e-6)
    rope = gpu.ops.rope_tables(max_ctx)
    kc_d, vc_d = dev(kc), dev(vc)
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    q_out = gpu.ops.qk_norm_rope_kv_decode(dev(qkv), dev(gq), dev(gk), rope, kc_d, vc_d, p, Hq)
    torch.cuda.synchronize()
    assert np.array_equal(host(q_out), q_ref)
    assert np.array_equal(host(kc_d), kc_ref)
    assert np.array_equal(host(vc_d), vc_ref)


def test_qk_norm_rope_kv_decode_out_of_range_position_writes_nothing(gpu):
    Hq, Hkv, max_ctx = 16, 8, 64
    qkv = normal("oqkv", ((Hq + 2 * Hkv) * D,))
    rope = gpu.ops.rope_tables(max_ctx)
    kc_d = torch.zeros((Hkv, max_ctx, D), dtype=torch.float16, device="cuda")
    vc_d = torch.zeros_like(kc_d)
    p = torch.tensor([max_ctx], dtype=torch.int32, device="cuda")
    gq = dev(gamma("gq"))
    gpu.ops.qk_norm_rope_kv_decode(dev(qkv), gq, gq, rope, kc_d, vc_d, p, Hq)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(kc_d)) == 0 and int(torch.count_nonzero(vc_d)) == 0


# ------------------------------------------------------------ decode attention


def _decode_case(gpu, Hq, Hkv, ctx, max_ctx, num_splits, tag):
    _say("decode", Hq, Hkv, ctx, max_ctx, num_splits)
    q = normal(tag + "q", (Hq, D))
    kc = normal(tag + "k", (Hkv, max_ctx, D))
    vc = normal(tag + "v", (Hkv, max_ctx, D))
    ref = O.attention_decode(q, kc, vc, ctx - 1, nthreads=16)
    p = torch.tensor([ctx - 1], dtype=torch.int32, device="cuda")
    out = gpu.ops.attn_decode(dev(q), dev(kc), dev(vc), p, num_splits=num_splits)
    torch.cuda.synchronize()
    assert_close(host_f32(out), ref, f"decode Hq={Hq} Hkv={Hkv} ctx={ctx} splits={num_splits}")


@pytest.mark.parametrize("Hq,Hkv,ctx,max_ctx,splits", [
    (16, 8, 513, 1024, None),     # config 1 shape (0.6B)
    (32, 8, 4096, 32768, None),   # config 2 (4B)
    (32, 8, 4096, 32768, 1),
    (32, 8, 4096, 32768, 7),
    (32, 8, 4096, 32768, 200),    # more splits than tiles: empty splits
    (64, 8, 8192, 32768, None),   # config 4 (32B)
    (64, 8, 16384, 32768, None),
    (64, 8, 32768, 32768, None),
    (8, 8, 1, 64, None),          # ctx = 1, G = 1
    (32, 2, 100, 160, 3),         # ragged ctx, G = 16
    (40, 8, 777, 1000, None),     # G = 5
    (16, 1, 1500, 2048, None),    # one kv head (G = 16)
    (28, 4, 900, 1024, 5),        # Hkv = 4, G = 7
    (32, 32, 600, 640, None),     # 32 kv heads (G = 1): a wide first grid dimension
    (26, 2, 1000, 1024, 9),       # G = 13
    (32, 16, 2000, 2048, None),   # Hkv = 16, G = 2
    (12, 3, 2000, 2048, None),    # odd kv head counts: Hkv = 3, 5, 6
    (80, 5, 777, 1024, 9),        # Hkv = 5, G = 16
    (48, 6, 3001, 4096, None),    # Hkv = 6, G = 8, ragged
    (64, 8, 131072, 131072, 4096),  # GROUT_MAX_SPLITS: one 32-position tile per split, G = 8
    (16, 8, 3000, 4096, 4096),    # GROUT_MAX_SPLITS, 94 tiles: all but 94 splits empty
])
def test_decode_attention_vs_oracle(gpu, Hq, Hkv, ctx, max_ctx, splits):
    _decode_case(gpu, Hq, Hkv, ctx, max_ctx, splits, f"dec{Hq}_{ctx}")


def _random_decode_cases(n=12, seed=2024):
    """Seeded shapes beyond the hand-picked ones: any G <= 16 the decode
    kernels take, 1-8 kv heads, ragged contexts, caches longer than the
    context, default or explicit split counts (some above the tile count)."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        Hkv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.integers(1, 17))
        ctx = int(rng.integers(1, 3001))
        max_ctx = ctx + int(rng.integers(0, 65))
        splits = None if rng.random() < 0.4 else int(rng.integers(1, 65))
        cases.append((G * Hkv, Hkv, ctx, max_ctx, splits))
    return cases


@pytest.mark.parametrize("Hq,Hkv,ctx,max_ctx,splits", _random_decode_cases())
def test_decode_random_shapes_vs_oracle(gpu, Hq, Hkv, ctx, max_ctx, splits):
    _decode_case(gpu, Hq, Hkv, ctx, max_ctx, splits, f"rdec{Hq}_{Hkv}_{ctx}")


@pytest.mark.parametrize("Hq,Hkv,pos,max_ctx,splits", [
    (32, 8, 640, 1024, 1),        # engine shape, one split (direct output)
    (32, 8, 640, 1024, None),     # default splits + merge
    (32, 8, 4095, 4096, 1),
    (64, 8, 8191, 32768, None),   # 32B, G = 8
    (64, 8, 16383, 32768, None),  # config 4 at ctx 16384
    (32, 2, 100, 160, 3),         # G = 16, ragged
    (32, 2, 100, 160, 1),         # G = 16, one split: a group also takes row 16
    (40, 8, 16, 64, 1),           # G = 5, the new row opens a tile
    (8, 8, 0, 64, 1),             # first position
    (16, 8, 47, 64, 7),           # more splits than tiles
    (16, 1, 300, 512, None),      # one kv head
    (28, 4, 200, 256, 3),         # Hkv = 4, G = 7
    (32, 8, 4095, 4096, 4096),    # GROUT_MAX_SPLITS: the new row's split among 4000 empty ones
    (24, 3, 300, 512, None),      # Hkv = 3, G = 8
])
def test_fused_decode_step_vs_oracle(gpu, Hq, Hkv, pos, max_ctx, splits):
    """Norm/RoPE/KV write fused into the decode attention: cache rows
    bit-exact against the oracle's norm/RoPE/KV write, output within the
    attention tolerance of the oracle's attention on the oracle's q rows.
    Cache rows past pos hold NaN: the tile loads clamp to row pos, which the
    kernel patches with the new row, so they never reach the output."""
    _say("fused_decode", Hq, Hkv, pos, max_ctx, splits)
    qkv = normal("fqkv", ((Hq + 2 * Hkv) * D,))
    gq, gk = gamma("fgq"), gamma("fgk")
    cos, sin = O.rope_table(max_ctx, D, 1e6)
    kc = normal("fkc", (Hkv, max_ctx, D))
    vc = normal("fvc", (Hkv, max_ctx, D))
    kc[:, pos:, :] = 0x7E00  # NaN: the cache's old row pos and everything after it
    vc[:, pos:, :] = 0x7E00
    kc_ref, vc_ref = kc.copy(), vc.copy()
    q_ref = O.qk_norm_rope_kv_decode(qkv, gq, gk, cos, sin, kc_ref, vc_ref, pos, Hq, Hkv, 1e-6)
    ref = O.attention_decode(q_ref, kc_ref, vc_ref, pos, nthreads=8)
    rope = gpu.ops.rope_tables(max_ctx)
    kc_d, vc_d = dev(kc), dev(vc)
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    out = gpu.ops.attn_decode_fused(dev(qkv), dev(gq), dev(gk), rope, kc_d, vc_d, p, Hq,
                                    num_splits=splits)
    torch.cuda.synchronize()
    assert np.array_equal(host(kc_d), kc_ref)
    assert np.array_equal(host(vc_d), vc_ref)
    assert_close(host_f32(out), ref, f"fused decode Hq={Hq} pos={pos} splits={splits}")


@pytest.mark.parametrize("pos,splits", [(64, None), (64, 1), (1000, 3)])
def test_fused_decode_position_past_cache_writes_nothing(gpu, pos, splits):
    """A position at or past max_ctx (a graph replayed one step too far) must
    not write the cache: both caches stay bit-identical, and the output is the
    attention of the q rows rotated at the last table row over all max_ctx
    cached positions."""
    Hq, Hkv, max_ctx = 16, 8, 64
    _say("fused_decode_past", Hq, Hkv, pos, max_ctx, splits)
    qkv = normal("pqkv", ((Hq + 2 * Hkv) * D,))
    gq, gk = gamma("pgq"), gamma("pgk")
    cos, sin = O.rope_table(max_ctx, D, 1e6)
    kc = normal("pkc", (Hkv, max_ctx, D))
    vc = normal("pvc", (Hkv, max_ctx, D))
    q_ref = O.qk_norm_rope_kv_decode(qkv, gq, gk, cos, sin, kc.copy(), vc.copy(), max_ctx - 1,
                                     Hq, Hkv, 1e-6)
    ref = O.attention_decode(q_ref, kc, vc, max_ctx - 1, nthreads=8)
    rope = gpu.ops.rope_tables(max_ctx)
    kc_d, vc_d = dev(kc), dev(vc)
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    out = gpu.ops.attn_decode_fused(dev(qkv), dev(gq), dev(gk), rope, kc_d, vc_d, p, Hq,
                                    num_splits=splits)
    torch.cuda.synchronize()
    assert np.array_equal(host(kc_d), kc)
    assert np.array_equal(host(vc_d), vc)
    assert_close(host_f32(out), ref, f"fused decode past the cache pos={pos} splits={splits}")


def test_decode_split_then_merge_matches_fused_call(gpu):
    Hq, Hkv, ctx, max_ctx, ns = 32, 8, 3000, 4096, 11
    q, kc, vc = normal("sq", (Hq, D)), normal("sk", (Hkv, max_ctx, D)), normal("sv", (Hkv, max_ctx, D))
    p = torch.tensor([ctx - 1], dtype=torch.int32, device="cuda")
    qd, kd, vd = dev(q), dev(kc), dev(vc)
    acc, ml = gpu.ops.fmha_decode_gqa_split(qd, kd, vd, p, ns)
    merged = gpu.ops.splitk_reduce_merge(acc, ml)
    fused = gpu.ops.attn_decode(qd, kd, vd, p, num_splits=ns)
    torch.cuda.synchronize()
    assert torch.equal(merged, fused)
    assert_close(host_f32(merged), O.attention_decode(q, kc, vc, ctx - 1, nthreads=8), "two-kernel path")
    # partial statistics: sum over splits of l * 2^(m - M) equals the full softmax denominator
    ml = ml.cpu().double()
    M = ml[..., 0].max(1, keepdim=True).values
    L = (ml[..., 1] * torch.exp2(ml[..., 0] - M)).sum(1)
    qf = q.view(np.float16).astype(np.float64).reshape(Hkv, Hq // Hkv, D)
    kf = kc[:, :ctx].view(np.float16).astype(np.float64)
    s = np.einsum("hgd,hnd->hgn", qf, kf) / np.sqrt(D) * np.log2(np.e)
    ref_L = np.exp2(s - M.numpy()[..., None][:, 0]).sum(-1)
    assert np.allclose(L.numpy(), ref_L, rtol=2e-3)


def test_sharded_decode_layer_matches_the_whole_layer(gpu):
    """The two ways one Qwen3-32B decode layer at 32k would be spread over
    GPUs, run as each GPU's share on this one: (1) by kv head, one kv head and
    its 8 q heads per GPU (Hkv=1 slices of the cache); (2) by sequence, each
    GPU running the split pass on its slice of the context and the slices'
    partials gathered ([Hkv][P x splits][G][...], what an all-gather delivers)
    into one merge.  Each result is checked against the oracle on the whole
    layer and against the unsharded call."""
    from grout_amd._lib import call

    Hq, Hkv, max_ctx = 64, 8, 32768
    G = Hq // Hkv
    ctx = max_ctx
    _say("sharded decode", Hq, Hkv, ctx)
    q = normal("shq", (Hq, D))
    kc, vc = normal("shk", (Hkv, max_ctx, D)), normal("shv", (Hkv, max_ctx, D))
    ref = O.attention_decode(q, kc, vc, ctx - 1, nthreads=8)
    qd, kd, vd = dev(q), dev(kc), dev(vc)
    p = torch.tensor([ctx - 1], dtype=torch.int32, device="cuda")
    whole = gpu.ops.attn_decode(qd, kd, vd, p, num_splits=32)
    # (1) kv-head shards
    by_head = torch.cat([gpu.ops.attn_decode(qd[h * G:(h + 1) * G], kd[h:h + 1], vd[h:h + 1], p,
                                             num_splits=32) for h in range(Hkv)])
    # (2) sequence shards: 4 aligned slices x 8 splits, and 3 ragged slices
    def by_sequence(bounds, ns):
        accs, mls = [], []
        for a, b in zip(bounds[:-1], bounds[1:]):
            acc = torch.empty((Hkv, ns, G, D), dtype=torch.float32, device="cuda")
            ml = torch.empty((Hkv, ns, G, 2), dtype=torch.float32, device="cuda")
            pl = torch.tensor([b - a - 1], dtype=torch.int32, device="cuda")
            call("grout_fmha_decode_gqa_split", qd.data_ptr(), kd.data_ptr() + a * D * 2,
                 vd.data_ptr() + a * D * 2, acc.data_ptr(), ml.data_ptr(), pl.data_ptr(), Hq, Hkv,
                 D, b - a, max_ctx * D, ns, D ** -0.5, torch.cuda.current_stream().cuda_stream)
            accs.append(acc)
            mls.append(ml)
            torch.cuda.synchronize()  # pl lives until the pass has read it
        return gpu.ops.splitk_reduce_merge(torch.cat(accs, 1).contiguous(),
                                           torch.cat(mls, 1).contiguous())
    by_seq4 = by_sequence([0, 8192, 16384, 24576, 32768], 8)
    by_seq3 = by_sequence([0, 10000, 22000, 32768], 8)
    torch.cuda.synchronize()
    w = host_f32(whole)
    for name, out in (("kv-head shards", by_head), ("4 sequence shards", by_seq4),
                      ("3 ragged sequence shards", by_seq3)):
        got = host_f32(out)
        assert_close(got, ref, f"{name} vs oracle")
        # same math, other accumulation orders: within a few f16 ulps of the whole call
        assert np.abs(got - w).max() <= 4 * 2.0 ** -11 * max(1.0, np.abs(w).max()), name


def test_decode_reuses_workspace_across_calls(gpu):
    """Consecutive decodes on one workspace (as the decode graph does)."""
    Hq, Hkv, max_ctx, ns = 64, 8, 4096, 24
    q, kc, vc = normal("wq", (Hq, D)), normal("wk", (Hkv, max_ctx, D)), normal("wv", (Hkv, max_ctx, D))
    qd, kd, vd = dev(q), dev(kc), dev(vc)
    ws = gpu.ops.decode_workspace(Hq, Hkv, ns, "cuda")
    outs = []
    for ctx in (4096, 1, 33, 2500, 4096, 700):
        p = torch.tensor([ctx - 1], dtype=torch.int32, device="cuda")
        outs.append((ctx, gpu.ops.attn_decode(qd, kd, vd, p, num_splits=ns, workspace=ws).clone()))
    torch.cuda.synchronize()
    for ctx, out in outs:
        assert_close(host_f32(out), O.attention_decode(q, kc, vc, ctx - 1, nthreads=8), f"reuse ctx={ctx}")


# ----------------------------------------------------------- prefill attention


@pytest.mark.parametrize("S,Hq,Hkv,pos0", [
    (1, 32, 8, 0), (17, 32, 8, 0), (64, 16, 8, 3), (200, 32, 8, 77), (130, 64, 8, 0),
    (96, 8, 8, 10), (77, 40, 8, 9), (33, 16, 1, 0), (150, 48, 8, 5), (111, 56, 8, 0),
    (1, 32, 8, 4095), (3, 64, 8, 1000),  # a one-token extend, a short chunk after a long prefix
    (100, 24, 3, 5), (70, 80, 5, 0), (300, 36, 6, 17),  # Hkv = 3, 5, 6 (G = 8, 16, 6)
    (60, 40, 40, 3), (50, 26, 2, 0), (90, 39, 3, 11)])  # Hkv = 40 (G = 1); G = 13 (13 one-head
                                                       # sub-groups per kv head, both Hkv = 2, 3)
def test_prefill_attention_vs_oracle(gpu, S, Hq, Hkv, pos0):
    _say("prefill", S, Hq, Hkv, pos0)
    max_ctx = pos0 + S + 5
    q = normal(f"pq{S}", (S, Hq, D))
    kc, vc = normal(f"pk{S}", (Hkv, max_ctx, D)), normal(f"pv{S}", (Hkv, max_ctx, D))
    ref = O.attention_prefill_rows(q, kc, vc, pos0, nthreads=8)
    out = gpu.ops.fmha_prefill(dev(q), dev(kc), dev(vc), pos0)
    torch.cuda.synchronize()
    assert_close(host_f32(out), ref, f"prefill S={S} Hq={Hq} Hkv={Hkv} pos0={pos0}")


def _random_prefill_cases(n=10, seed=4048):
    """Seeded prefill shapes: any G up to 16 (head groups of the largest
    divisor of G that is <= 8), 1-8 kv heads, ragged lengths, and a start
    position pos0 > 0 in most cases (rows below it come from the cache)."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        Hkv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.integers(1, 17))
        S = int(rng.integers(1, 301))
        pos0 = 0 if rng.random() < 0.3 else int(rng.integers(1, 201))
        cases.append((S, G * Hkv, Hkv, pos0))
    return cases


@pytest.mark.parametrize("form", ["default", "rows32", "shared"])
@pytest.mark.parametrize("S,Hq,Hkv,pos0", _random_prefill_cases())
def test_prefill_random_shapes_vs_oracle(gpu, monkeypatch, form, S, Hq, Hkv, pos0):
    """Default work split (64-row blocks at these lengths), 128-row blocks
    forced, and the shared K/V stream forced."""
    if form == "rows32":
        monkeypatch.setenv("GROUT_FMHA_PREFILL_WAVE_ROWS", "32")
    if form == "shared":
        monkeypatch.setenv("GROUT_FMHA_PREFILL_SHARED", "1")
    _say("prefill random", form, S, Hq, Hkv, pos0)
    max_ctx = pos0 + S + 3
    q = normal(f"rpq{S}_{Hq}", (S, Hq, D))
    kc, vc = normal(f"rpk{S}_{Hkv}", (Hkv, max_ctx, D)), normal(f"rpv{S}_{Hkv}", (Hkv, max_ctx, D))
    ref = O.attention_prefill_rows(q, kc, vc, pos0, nthreads=8)
    out = gpu.ops.fmha_prefill(dev(q), dev(kc), dev(vc), pos0)
    torch.cuda.synchronize()
    assert_close(host_f32(out), ref, f"prefill S={S} Hq={Hq} Hkv={Hkv} pos0={pos0}")


@pytest.mark.parametrize("mode", ["single", "paired", "single64", "paired64", "shared",
                                  "shared_single"])
@pytest.mark.parametrize("S,Hq,Hkv,pos0", [
    (1, 32, 8, 0), (17, 32, 8, 0), (130, 64, 8, 0), (200, 32, 8, 77), (77, 40, 8, 9),
    (33, 16, 1, 0), (700, 32, 8, 100), (1000, 16, 4, 0), (2048, 24, 8, 0), (600, 56, 8, 7),
    (3000, 32, 8, 0), (523, 8, 8, 300), (300, 48, 8, 20), (400, 16, 8, 0), (260, 64, 2, 31)])
def test_prefill_work_splits_vs_oracle(gpu, monkeypatch, mode, S, Hq, Hkv, pos0):
    """Every work split of the prefill FMHA, forced through
    GROUT_FMHA_PREFILL_SHARED / _PAIRED / _WAVE_ROWS: per-team K/V staging
    with one q block per workgroup (its tiles split over the two 4-wave teams)
    or complementary q-block pairs (team B taking the light block and the
    tail of the heavy one), each with 128-row blocks (32 rows per wave) or
    64-row blocks (16 rows per wave), and the shared K/V stream (256-row
    blocks, both teams on one staged tile stream, pairs run back to back or
    one block per workgroup).
    Odd block counts, a kv prefix (pos0 > 0), a single kv head, HG = 3 (rows
    that fall outside a 126- or 63-row block), HG = 5, 6 and 7 (60-63 of 64
    rows used), HG = 2 and HG = 1 (one head per kv group), and G = 32 (four
    8-head q blocks per kv group)."""
    monkeypatch.setenv("GROUT_FMHA_PREFILL_SHARED", "1" if mode.startswith("shared") else "0")
    monkeypatch.setenv("GROUT_FMHA_PREFILL_PAIRED",
                       "1" if mode.startswith("paired") or mode == "shared" else "0")
    monkeypatch.setenv("GROUT_FMHA_PREFILL_WAVE_ROWS", "16" if mode.endswith("64") else "32")
    _say("prefill_split", mode, S, Hq, Hkv, pos0)
    max_ctx = pos0 + S + 3
    q = normal(f"wq{S}", (S, Hq, D))
    kc, vc = normal(f"wk{S}", (Hkv, max_ctx, D)), normal(f"wv{S}", (Hkv, max_ctx, D))
    rows = None if S <= 1000 else np.r_[0:64, 700:764, 1333:1397, S - 64:S]
    ref = O.attention_prefill_rows(q, kc, vc, pos0, rows=rows, nthreads=16)
    out = gpu.ops.fmha_prefill(dev(q), dev(kc), dev(vc), pos0)
    torch.cuda.synchronize()
    got = host_f32(out) if rows is None else host_f32(out)[rows]
    assert_close(got, ref, f"prefill {mode} S={S} Hq={Hq} Hkv={Hkv} pos0={pos0}")


@pytest.mark.parametrize("form", ["rows16", "rows32", "shared"])
@pytest.mark.parametrize("S,pos0", [(77, 0), (130, 61), (1000, 24)])
def test_prefill_ignores_cache_rows_past_kv_len(gpu, monkeypatch, form, S, pos0):
    """Cache rows at and past kv_len = pos0 + S hold NaN: the last kv tile
    reads them as zeros (bounded loads) and masks them, so outputs stay equal
    to the oracle's, which never reads them (per-team staging with 64- and
    128-row blocks, shared staging)."""
    monkeypatch.setenv("GROUT_FMHA_PREFILL_SHARED", "1" if form == "shared" else "0")
    monkeypatch.setenv("GROUT_FMHA_PREFILL_WAVE_ROWS", "32" if form == "rows32" else "16")
    _say("prefill_nan_tail", form, S, pos0)
    Hq, Hkv, max_ctx = 32, 8, pos0 + S + 70
    q = normal(f"nt{S}", (S, Hq, D))
    kc, vc = normal(f"ntk{S}", (Hkv, max_ctx, D)), normal(f"ntv{S}", (Hkv, max_ctx, D))
    nan16 = np.uint16(0x7E00)
    kc[:, pos0 + S:] = nan16
    vc[:, pos0 + S:] = nan16
    ref = O.attention_prefill_rows(q, kc, vc, pos0, nthreads=16)
    out = gpu.ops.fmha_prefill(dev(q), dev(kc), dev(vc), pos0)
    torch.cuda.synchronize()
    assert_close(host_f32(out), ref, f"prefill nan tail {form} S={S} pos0={pos0}")


# ------------------------------------------------------- configs end to end


def test_config1_decode_step_pipeline(gpu):
    """Qwen3-0.6B-shaped decode step: 512 cached positions, new token's q,k,v
    through QK-RMSNorm + RoPE (pos 512, theta 1e6, eps 1e-6), KV write at slot
    512, attention over 513 positions with scale 1/sqrt(128)."""
    Hq, Hkv, pos, max_ctx = 16, 8, 512, 1024
    kc = normal("c1k", (Hkv, max_ctx, D))
    vc = normal("c1v", (Hkv, max_ctx, D))
    kc[:, pos + 1:] = 0
    vc[:, pos + 1:] = 0
    qkv = normal("c1qkv", ((Hq + 2 * Hkv) * D,))
    gq, gk = gamma("c1gq"), gamma("c1gk")
    cos, sin = O.rope_table(max_ctx, D, 1e6)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    q_ref = O.qk_norm_rope_kv_decode(qkv, gq, gk, cos, sin, kc_ref, vc_ref, pos, Hq, Hkv, 1e-6)
    out_ref = O.attention_decode(q_ref, kc_ref, vc_ref, pos)

    rope = gpu.ops.rope_tables(max_ctx)
    kd, vd = dev(kc), dev(vc)
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    q_rope = gpu.ops.qk_norm_rope_kv_decode(dev(qkv), dev(gq), dev(gk), rope, kd, vd, p, Hq)
    out = gpu.ops.attention(q_rope.view(1, Hq, D), kd, vd, p)
    torch.cuda.synchronize()
    assert np.array_equal(host(kd), kc_ref) and np.array_equal(host(vd), vc_ref)
    assert_close(host_f32(out).reshape(Hq, D), out_ref, "config1 decode step")


@pytest.mark.parametrize("S", [512, 2048, 8192])
def test_config3_prefill_pipeline(gpu, S):
    """Qwen3-4B-shaped prefill: fused QK-norm/RoPE/KV write at positions
    0..S-1, then causal FMHA.  S=512 checked in full; S=2048 and S=8192 on
    rows 0..63, the last 64 rows and 64 seeded random rows (every head of
    each row); rotated q and the K/V cache rows in full, bit for bit."""
    _say("config3", S)
    Hq, Hkv, max_ctx = 32, 8, 32768
    q, k, v = normal(f"c3q{S}", (S, Hq, D)), normal(f"c3k{S}", (S, Hkv, D)), normal(f"c3v{S}", (S, Hkv, D))
    gq, gk = gamma("c3gq"), gamma("c3gk")
    cos, sin = O.rope_table(max_ctx, D, 1e6)
    kc_ref = np.zeros((Hkv, max_ctx, D), np.uint16)
    vc_ref = kc_ref.copy()
    q_ref = O.qk_norm_rope_kv_prefill(q, k, v, gq, gk, cos, sin, kc_ref, vc_ref, 0, 1e-6)
    rows = np.arange(S) if S <= 512 else np.unique(np.concatenate([
        np.arange(64), np.arange(S - 64, S), np.random.default_rng(S).integers(0, S, 64)]))
    ref = O.attention_prefill_rows(q_ref, kc_ref, vc_ref, 0, rows=rows, nthreads=16)

    rope = gpu.ops.rope_tables(max_ctx)
    kd = torch.zeros((Hkv, max_ctx, D), dtype=torch.float16, device="cuda")
    vd = torch.zeros_like(kd)
    q_rope = gpu.ops.qk_norm_rope_kv_prefill(dev(q), dev(k), dev(v), dev(gq), dev(gk), rope, kd, vd, 0)
    out = gpu.ops.attention(q_rope, kd, vd, 0)
    torch.cuda.synchronize()
    assert np.array_equal(host(q_rope), q_ref)
    assert np.array_equal(host(kd[:, :S]), kc_ref[:, :S]) and np.array_equal(host(vd[:, :S]), vc_ref[:, :S])
    assert_close(host_f32(out)[rows], ref, f"config3 prefill S={S}")


def test_prefill_row_equals_decode_at_same_position(gpu):
    """Prefill row m and a decode step at position m read the same cache: equal within tolerance."""
    S, Hq, Hkv, max_ctx = 300, 32, 8, 512
    q = normal("xq", (S, Hq, D))
    kd, vd = dev(normal("xk", (Hkv, max_ctx, D))), dev(normal("xv", (Hkv, max_ctx, D)))
    qd = dev(q)
    pre = gpu.ops.fmha_prefill(qd, kd, vd, 0)
    for m in (0, 31, 32, 255, 299):
        p = torch.tensor([m], dtype=torch.int32, device="cuda")
        dec = gpu.ops.attn_decode(qd[m], kd, vd, p)
        torch.cuda.synchronize()
        assert_close(host_f32(dec), host_f32(pre[m]), f"prefill row {m} vs decode")


# ------------------------------------------------------------- decode graph


def test_ops_run_on_the_callers_stream(gpu):
    """Every call works on the stream it is given: the fused prefill write,
    the prefill FMHA, split-K decode and the fused decode layer issued on a
    side stream (default priority), each behind a host-visible dependency on
    that stream only, equal the same calls on the default stream bit for
    bit."""
    Hq, Hkv, S, max_ctx = 32, 8, 300, 1024
    _say("side stream")
    q, k, v = normal("ssq", (S, Hq, D)), normal("ssk", (S, Hkv, D)), normal("ssv", (S, Hkv, D))
    gq, gk = dev(gamma("ssgq")), dev(gamma("ssgk"))
    qkv = dev(normal("ssqkv", ((Hq + 2 * Hkv) * D,)))
    rope = gpu.ops.rope_tables(max_ctx)
    qd, kd, vd = dev(q), dev(k), dev(v)

    def run():
        kc = torch.zeros((Hkv, max_ctx, D), dtype=torch.float16, device="cuda")
        vc = torch.zeros_like(kc)
        qr = gpu.ops.qk_norm_rope_kv_prefill(qd, kd, vd, gq, gk, rope, kc, vc, 0)
        pre = gpu.ops.fmha_prefill(qr, kc, vc, 0)
        p = torch.tensor([S], dtype=torch.int32, device="cuda")
        fused = gpu.ops.attn_decode_fused(qkv, gq, gk, rope, kc, vc, p, Hq)
        dec = gpu.ops.attn_decode(pre[-1], kc, vc, p, num_splits=7)
        return [pre, fused, dec, kc, vc]

    ref = run()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        torch.cuda._sleep(1 << 20)  # the side stream is busy first: a call on the
        got = run()                 # default stream instead would read unfinished inputs
    side.synchronize()
    for i, (a, b) in enumerate(zip(ref, got)):
        assert torch.equal(a, b), f"output {i} differs on the side stream"


def test_ops_captured_by_the_caller_replay_like_eager_calls(gpu):
    """The calls are capture-safe: the fused decode layer, split-K decode and
    the prefill FMHA captured into a caller's HIP graph (torch), replayed
    several times with the program's own eager work (new inputs, a new
    position) and host synchronizations between the replays, match eager
    calls on the same inputs bit for bit at every replay."""
    Hq, Hkv, S, max_ctx = 32, 8, 200, 1024
    _say("caller graph")
    gq, gk = dev(gamma("cggq")), dev(gamma("cggk"))
    rope = gpu.ops.rope_tables(max_ctx)
    kc = dev(normal("cgk", (Hkv, max_ctx, D)))
    vc = dev(normal("cgv", (Hkv, max_ctx, D)))
    qkv = torch.empty(((Hq + 2 * Hkv) * D,), dtype=torch.float16, device="cuda")
    qp = torch.empty((S, Hq, D), dtype=torch.float16, device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = gpu.ops.decode_workspace(Hq, Hkv, 16, "cuda")
    ws2 = gpu.ops.decode_workspace(Hq, Hkv, 5, "cuda")
    outs = [torch.empty((Hq, D), dtype=torch.float16, device="cuda") for _ in range(2)]
    pre = torch.empty_like(qp)

    def body(kc_, vc_, o0, o1, pr):
        gpu.ops.attn_decode_fused(qkv, gq, gk, rope, kc_, vc_, pos, Hq, num_splits=16, out=o0,
                                  workspace=ws)
        gpu.ops.attn_decode(qkv[:Hq * D].view(Hq, D), kc_, vc_, pos, num_splits=5, out=o1,
                            workspace=ws2)
        gpu.ops.fmha_prefill(qp, kc_, vc_, 0, out=pr)

    qkv.copy_(dev(normal("cgqkv0", ((Hq + 2 * Hkv) * D,))))
    qp.copy_(dev(normal("cgq0", (S, Hq, D))))
    body(kc.clone(), vc.clone(), *[torch.empty_like(o) for o in outs], torch.empty_like(pre))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    kg, vg = kc.clone(), vc.clone()
    with torch.cuda.graph(g):
        body(kg, vg, outs[0], outs[1], pre)
    for rep, p in enumerate([300, 301, 57, 900]):
        qkv.copy_(dev(normal(f"cgqkv{rep}", ((Hq + 2 * Hkv) * D,))))
        qp.copy_(dev(normal(f"cgq{rep}", (S, Hq, D))))
        pos.fill_(p)
        ke, ve = kg.clone(), vg.clone()  # eager reference from the same cache state
        torch.cuda.synchronize()
        g.replay()
        eo = [torch.empty_like(o) for o in outs]
        ep = torch.empty_like(pre)
        body(ke, ve, eo[0], eo[1], ep)
        torch.cuda.synchronize()
        assert torch.equal(kg, ke) and torch.equal(vg, ve), f"replay {rep}: caches"
        assert torch.equal(outs[0], eo[0]) and torch.equal(outs[1], eo[1]), f"replay {rep}: decode"
        assert torch.equal(pre, ep), f"replay {rep}: prefill"
    del g


def test_decode_graph_replays_match_eager_ops(gpu):
    from grout_amd.engine import AttentionConfig, AttentionEngine

    cfg = AttentionConfig(num_layers=3, num_attention_heads=32, num_key_value_heads=8, max_ctx=2048)
    qn = [dev(gamma(f"gq{i}")) for i in range(3)]
    kn = [dev(gamma(f"gk{i}")) for i in range(3)]
    eng = AttentionEngine(cfg, qn, kn)
    for i in range(3):  # prior context
        eng.k_caches[i].copy_(dev(normal(f"gk_c{i}", (8, 2048, D))))
        eng.v_caches[i].copy_(dev(normal(f"gv_c{i}", (8, 2048, D))))
    graph = eng.build_decode_graph()
    eager_k = [t.clone() for t in eng.k_caches]
    eager_v = [t.clone() for t in eng.v_caches]
    for step, pos in enumerate([700, 701, 1500, 2047]):
        _say("graph replay", step, pos)
        for i in range(3):
            graph.qkv[i].copy_(dev(normal(f"gqkv{step}_{i}", ((32 + 16) * D,))))
        graph.launch_step(pos)
        torch.cuda.synchronize()
        p = torch.tensor([pos], dtype=torch.int32, device="cuda")
        for i in range(3):
            qr = gpu.ops.qk_norm_rope_kv_decode(graph.qkv[i], qn[i], kn[i], eng.rope, eager_k[i],
                                                eager_v[i], p, 32)
            ref = gpu.ops.attn_decode(qr, eager_k[i], eager_v[i], p, num_splits=graph.num_splits)
            torch.cuda.synchronize()
            assert torch.equal(eng.k_caches[i], eager_k[i]) and torch.equal(eng.v_caches[i], eager_v[i])
            assert torch.equal(graph.attn_out[i], ref), f"layer {i} step {step}"
        torch.cuda.synchronize()
    # Consecutive positions queued back to back with no host wait: every
    # launch after the first finds the position word moved on by the previous
    # replay's last merge (no write of its own), then a jump back to an
    # earlier position is written again.
    seq = [1200, 1201, 1202, 1203, 900]
    qkvs = [[dev(normal(f"gqq{pos}_{i}", ((32 + 16) * D,))) for i in range(3)] for pos in seq]
    for pos, qs in zip(seq, qkvs):
        _say("queued graph replay", pos)
        for i in range(3):
            graph.qkv[i].copy_(qs[i])
        graph.launch_step(pos)
    import ctypes as C
    from grout_amd._lib import lib

    torch.cuda.synchronize()
    word = C.c_uint32(0)
    wp = lib().grout_decode_graph_position_ptr(graph._h)
    hip = C.CDLL("libamdhip64.so")
    assert hip.hipMemcpy(C.byref(word), C.c_void_p(wp), C.c_size_t(4), 2) == 0  # D2H
    assert word.value == seq[-1] + 1, word.value
    for pos, qs in zip(seq, qkvs):
        p = torch.tensor([pos], dtype=torch.int32, device="cuda")
        for i in range(3):
            qr = gpu.ops.qk_norm_rope_kv_decode(qs[i], qn[i], kn[i], eng.rope, eager_k[i],
                                                eager_v[i], p, 32)
            ref = gpu.ops.attn_decode(qr, eager_k[i], eager_v[i], p, num_splits=graph.num_splits)
    torch.cuda.synchronize()
    for i in range(3):
        assert torch.equal(eng.k_caches[i], eager_k[i]) and torch.equal(eng.v_caches[i], eager_v[i])
    assert torch.equal(graph.attn_out[2], ref), "last queued step"
    graph.destroy()
    with pytest.raises(ValueError):
        AttentionEngine(AttentionConfig(1, 32, 8, head_dim=64), qn[:1], kn[:1])
