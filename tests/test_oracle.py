"""Pins the CPU oracle against checks that do not restate its own formulas:
published PRNG vectors, numpy's IEEE conversions, torch float64 library routines,
closed forms, invariants and brute force on tiny shapes."""
import math

import numpy as np
import pytest
import torch

import oracle as O

D = 128


# ----------------------------------------------------------------- fp16 + PRNG


def test_h2f_exhaustive_matches_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    ours = O.h2f(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f2h_roundtrip_and_numpy_rne():
    bits = np.arange(65536, dtype=np.uint16)
    f = bits.view(np.float16).astype(np.float32)
    ok = ~np.isnan(f)
    assert np.array_equal(O.f2h(f[ok]), bits[ok])
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-8, 5, 200000),
        # exact ties between neighbouring halves, normals and subnormals
        ((f[1:30000].astype(np.float64) + f[2:30001].astype(np.float64)) / 2).astype(np.float32),
        np.array([65504, 65519.99, 65520, 70000, 1e-8, 3e-8, 2.9802322e-08, -0.0], np.float32),
    ])
    x = x.astype(np.float32)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f2h(x), ref)


def test_splitmix64_published_vectors():
    # SplitMix64 seeded with 0 (Steele, Lea, Flood 2014; the sequence used by xoshiro seeding).
    assert [O.splitmix64_at(0, k) for k in range(1, 5)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]


def test_normal_stream_moments_and_single_rounding():
    x = O.fill_normal_f64(O.seed_for("moments"), 400000)
    assert abs(x.mean()) < 0.01 and abs(x.var() - 1.0) < 0.01
    assert abs(np.mean(x**4) - 3.0) < 0.05  # Gaussian kurtosis
    h = O.fill_normal_f16(O.seed_for("moments"), 400000)
    # numpy converts float64 -> float16 directly with one RNE rounding
    assert np.array_equal(h, x.astype(np.float16).view(np.uint16))


def test_uniform_range():
    g = O.h2f(O.fill_uniform_f16(O.seed_for("gamma"), 0.8, 1.2, 100000))
    assert g.min() >= 0.8 - 1e-3 and g.max() <= 1.2 + 1e-3
    assert abs(g.mean() - 1.0) < 0.01


# ----------------------------------------------------------------- RoPE tables


def test_inv_freq_and_rope_table_vs_numpy_float64():
    theta = 1e6
    inv = O.inv_freq(D, theta)
    exact = 1.0 / theta ** (np.arange(0, D, 2, dtype=np.float64) / D)
    assert np.allclose(inv, exact, rtol=3e-7, atol=0)
    c, s = O.rope_table(4096, D, theta)
    ang = np.arange(4096, dtype=np.float32)[:, None] * inv[None, :]  # f32 angle, like the reference
    assert np.max(np.abs(c - np.cos(ang.astype(np.float64)))) < 1e-7
    assert np.max(np.abs(s - np.sin(ang.astype(np.float64)))) < 1e-7
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    assert np.max(np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1)) < 3e-7


def test_rope_rows_equal_the_table_and_float64_at_the_largest_cache():
    """rope_rows(p0, n) is rows p0.. of rope_table, bit for bit, and at the
    last rows of a 2^22-position cache still cos/sin of the f32 angle."""
    theta = 1e6
    c, s = O.rope_table(3000, D, theta)
    for p0, n in ((0, 1), (0, 3000), (1, 7), (2047, 100), (2999, 1)):
        cr, sr = O.rope_rows(p0, n, D, theta)
        assert np.array_equal(cr, c[p0:p0 + n]) and np.array_equal(sr, s[p0:p0 + n]), (p0, n)
    top = (1 << 22) - 64
    cr, sr = O.rope_rows(top, 64, D, theta)
    ang = np.arange(top, top + 64).astype(np.float32)[:, None] * O.inv_freq(D, theta)[None, :]
    assert np.max(np.abs(cr - np.cos(ang.astype(np.float64)))) < 1e-7
    assert np.max(np.abs(sr - np.sin(ang.astype(np.float64)))) < 1e-7


# --------------------------------------------------------- QK-RMSNorm + RoPE


def _torch_norm_rope(x16, g16, pos, theta=1e6, eps=1e-6):
    """float64: torch rms_norm, then NeoX RoPE as complex multiplication."""
    x = torch.from_numpy(x16.view(np.float16).astype(np.float64))
    g = torch.from_numpy(g16.view(np.float16).astype(np.float64))
    n = torch.nn.functional.rms_norm(x, (D,), weight=g, eps=eps)
    inv = torch.from_numpy(O.inv_freq(D, theta).astype(np.float64))
    ang = torch.tensor(np.float32(pos) * O.inv_freq(D, theta), dtype=torch.float64)
    z = torch.complex(n[..., : D // 2], n[..., D // 2:]) * torch.polar(torch.ones_like(ang), ang)
    del inv
    return torch.cat([z.real, z.imag], -1).numpy()


@pytest.mark.parametrize("pos", [0, 1, 511, 4097, 32767])
def test_norm_rope_row_vs_torch_float64(pos):
    x = O.fill_normal_f16(O.seed_for("nrx") + pos, (64, D))
    g = O.fill_uniform_f16(O.seed_for("nrg"), 0.8, 1.2, D)
    c, s = O.rope_table(pos + 1, D, 1e6)
    ours = np.stack([O.h2f(O.qk_norm_rope_row(x[r], g, c[pos], s[pos], 1e-6)) for r in range(64)])
    ref = _torch_norm_rope(x, g, pos)
    # one f16 rounding (<= 2^-11 relative) plus fp32 arithmetic
    assert np.all(np.abs(ours - ref) <= np.abs(ref) * 2.0**-10 + 1e-6)


def test_norm_scale_invariance_and_unit_rms():
    x = O.fill_normal_f16(O.seed_for("inv"), D)
    ones = O.f2h(np.ones(D, np.float32))
    c, s = O.rope_table(1, D, 1e6)
    y = O.h2f(O.qk_norm_rope_row(x, ones, c[0], s[0], 0.0))
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1.0) < 1e-3  # gamma=1, pos 0 -> unit RMS
    x2 = O.f2h(O.h2f(x) * 4.0)  # exact power-of-two scaling in f16
    assert np.array_equal(O.qk_norm_rope_row(x2, ones, c[0], s[0], 0.0), O.qk_norm_rope_row(x, ones, c[0], s[0], 0.0))


def test_rope_pair_norm_and_relative_position():
    g = O.f2h(np.ones(D, np.float32))
    q = O.fill_normal_f16(O.seed_for("rq"), D)
    k = O.fill_normal_f16(O.seed_for("rk"), D)
    c, s = O.rope_table(2000, D, 1e6)
    def rot(x, p):
        return O.h2f(O.qk_norm_rope_row(x, g, c[p], s[p], 1e-6)).astype(np.float64)
    base = rot(q, 0)
    for p in (3, 100, 1999):
        r = rot(q, p)
        n0 = base[:64] ** 2 + base[64:] ** 2
        n1 = r[:64] ** 2 + r[64:] ** 2
        assert np.allclose(n0, n1, rtol=3e-3, atol=1e-4)
    d1 = rot(q, 700) @ rot(k, 650)
    d2 = rot(q, 1350) @ rot(k, 1300)
    assert abs(d1 - d2) < 2e-2 * max(1.0, abs(d1))


def test_sumsq_tree_matches_float64_sum():
    x = O.fill_normal_f16(O.seed_for("ss"), (32, D))
    for r in range(32):
        ref = np.sum(x[r].view(np.float16).astype(np.float64) ** 2)
        assert abs(O.sumsq_row128(x[r]) - ref) <= 1e-6 * ref


def test_rsqrt_det_correctly_rounded_on_sample():
    rng = np.random.default_rng(3)
    v = (10.0 ** rng.uniform(-7, 6, 20000)).astype(np.float32)
    ours = np.array([O.rsqrt_det(float(a)) for a in v], np.float32)
    exact = 1.0 / np.sqrt(v.astype(np.float64))
    # within half an ulp of f32 (correct rounding), allowing for the rare near-tie
    ulp = np.spacing(ours.astype(np.float32)).astype(np.float64)
    assert np.mean(np.abs(ours - exact) <= 0.5 * ulp + 1e-30) > 0.9999
    assert np.all(np.abs(ours - exact) <= ulp)


def test_prefill_kv_write_touches_only_its_slots():
    Hq, Hkv, S, pos0, max_ctx = 4, 2, 5, 7, 16
    q = O.fill_normal_f16(1, (S, Hq, D))
    k = O.fill_normal_f16(2, (S, Hkv, D))
    v = O.fill_normal_f16(3, (S, Hkv, D))
    gq = O.fill_uniform_f16(4, 0.8, 1.2, D)
    gk = O.fill_uniform_f16(5, 0.8, 1.2, D)
    c, s = O.rope_table(max_ctx, D, 1e6)
    kc = np.full((Hkv, max_ctx, D), 0x7BFF, np.uint16)  # canary
    vc = np.full((Hkv, max_ctx, D), 0x7BFF, np.uint16)
    q_out = O.qk_norm_rope_kv_prefill(q, k, v, gq, gk, c, s, kc, vc, pos0, 1e-6)
    written = np.zeros(max_ctx, bool)
    written[pos0:pos0 + S] = True
    assert np.all(kc[:, ~written] == 0x7BFF) and np.all(vc[:, ~written] == 0x7BFF)
    assert np.array_equal(vc[:, written], v.transpose(1, 0, 2))
    for si in range(S):
        for h in range(Hkv):
            assert np.array_equal(kc[h, pos0 + si], O.qk_norm_rope_row(k[si, h], gk, c[pos0 + si], s[pos0 + si], 1e-6))
        for h in range(Hq):
            assert np.array_equal(q_out[si, h], O.qk_norm_rope_row(q[si, h], gq, c[pos0 + si], s[pos0 + si], 1e-6))


# ----------------------------------------------------------------- attention


def _sdpa64(q16, k16, v16, pos0):
    """torch float64 SDPA, GQA, causal with absolute query positions pos0+s."""
    S, Hq, _ = q16.shape
    Hkv, n_kv, _ = k16.shape
    q = torch.from_numpy(q16.view(np.float16).astype(np.float64)).permute(1, 0, 2)[None]
    k = torch.from_numpy(k16[:, :n_kv].view(np.float16).astype(np.float64))[None]
    v = torch.from_numpy(v16[:, :n_kv].view(np.float16).astype(np.float64))[None]
    mask = (torch.arange(n_kv)[None, :] <= (pos0 + torch.arange(S))[:, None])
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)
    return o[0].permute(1, 0, 2).numpy()


@pytest.mark.parametrize("S,pos0,Hq,Hkv", [(1, 0, 2, 1), (17, 0, 8, 2), (33, 40, 16, 8), (64, 5, 4, 4)])
def test_prefill_vs_torch_sdpa_float64(S, pos0, Hq, Hkv):
    max_ctx = pos0 + S + 3
    q = O.fill_normal_f16(O.seed_for("pq") + S, (S, Hq, D))
    kc = O.fill_normal_f16(O.seed_for("pk") + S, (Hkv, max_ctx, D))
    vc = O.fill_normal_f16(O.seed_for("pv") + S, (Hkv, max_ctx, D))
    ours = O.attention_prefill_rows(q, kc, vc, pos0)
    ref = _sdpa64(q, kc[:, :pos0 + S], vc[:, :pos0 + S], pos0)
    assert np.max(np.abs(ours - ref)) < 2e-5


def test_prefill_bruteforce_float64_tiny():
    S, Hq, Hkv, pos0 = 6, 4, 2, 2
    q = O.fill_normal_f16(11, (S, Hq, D))
    kc = O.fill_normal_f16(12, (Hkv, pos0 + S, D))
    vc = O.fill_normal_f16(13, (Hkv, pos0 + S, D))
    ours = O.attention_prefill_rows(q, kc, vc, pos0)
    qf, kf, vf = (a.view(np.float16).astype(np.float64) for a in (q, kc, vc))
    for s in range(S):
        for h in range(Hq):
            kv = h // (Hq // Hkv)
            sc = np.array([qf[s, h] @ kf[kv, n] for n in range(pos0 + s + 1)]) / math.sqrt(D)
            w = np.exp(sc - sc.max())
            w /= w.sum()
            ref = w @ vf[kv, : pos0 + s + 1]
            assert np.max(np.abs(ours[s, h] - ref)) < 1e-5


def test_decode_vs_torch_and_closed_forms():
    Hq, Hkv, pos, max_ctx = 16, 8, 512, 600
    q = O.fill_normal_f16(O.seed_for("dq"), (Hq, D))
    kc = O.fill_normal_f16(O.seed_for("dk"), (Hkv, max_ctx, D))
    vc = O.fill_normal_f16(O.seed_for("dv"), (Hkv, max_ctx, D))
    ours = O.attention_decode(q, kc, vc, pos)
    ref = _sdpa64(q[None], kc[:, :pos + 1], vc[:, :pos + 1], pos)[0]
    assert np.max(np.abs(ours - ref)) < 2e-5
    # V constant -> output equals the constant
    vconst = np.full_like(vc, O.f2h(np.float32(0.375)))
    assert np.allclose(O.attention_decode(q, kc, vconst, pos), 0.375, atol=1e-6)
    # K constant -> uniform weights -> mean of V over the valid positions
    kconst = np.full_like(kc, O.f2h(np.float32(0.5)))
    mean_v = vc[:, : pos + 1].view(np.float16).astype(np.float64).mean(1)
    got = O.attention_decode(q, kconst, vc, pos)
    assert np.max(np.abs(got - np.repeat(mean_v, Hq // Hkv, 0))) < 1e-5
    # ctx = 1 -> v_0
    got = O.attention_decode(q, kc, vc, 0)
    assert np.allclose(got, np.repeat(vc[:, 0].view(np.float16).astype(np.float32), Hq // Hkv, 0), atol=1e-6)
    # q = lambda * k_j -> attention collapses on position j
    j = 123
    qj = O.f2h(np.repeat(kc[:, j].view(np.float16).astype(np.float32), Hq // Hkv, 0) * 8.0)
    got = O.attention_decode(qj, kc, vc, pos)
    assert np.max(np.abs(got - np.repeat(vc[:, j].view(np.float16).astype(np.float32), Hq // Hkv, 0))) < 1e-3


def test_decode_long_context_dominant_key_vs_float64():
    """2^19 cached positions, one key 16 units of score above an N(0,1)
    background placed first: every background weight is then ~1e-7 of the
    softmax sum, about one fp32 ulp of it, where sequential fp32 sums lose
    percents.  The oracle must still match a float64 softmax."""
    n, Hq = 1 << 19, 2
    g = torch.Generator().manual_seed(5)
    k = torch.randn((1, n, D), generator=g).half()
    v = torch.randn((1, n, D), generator=g).half()
    qf = torch.randn((Hq, D), generator=g, dtype=torch.float64)
    qf = qf / qf.norm(dim=1, keepdim=True) * math.sqrt(D)
    q = qf.half()
    k[0, 0] = (q[0].double() / math.sqrt(D) * 16.0).half()  # score 16 for head 0
    v[0, 0] = (4.0 * torch.randn(D, generator=g)).half()
    ours = O.attention_decode(q.numpy().view(np.uint16), k.numpy().view(np.uint16),
                              v.numpy().view(np.uint16), n - 1, nthreads=2)
    s = (k[0].double() @ q.double().T) / math.sqrt(D)
    ref = (torch.softmax(s, 0).T @ v[0].double()).numpy()
    assert np.max(np.abs(ours - ref)) < 1e-4


def test_gqa_equals_mha_with_repeated_kv():
    Hq, Hkv, pos = 8, 2, 77
    q = O.fill_normal_f16(21, (Hq, D))
    kc = O.fill_normal_f16(22, (Hkv, 80, D))
    vc = O.fill_normal_f16(23, (Hkv, 80, D))
    gqa = O.attention_decode(q, kc, vc, pos)
    mha = O.attention_decode(q, np.repeat(kc, Hq // Hkv, 0), np.repeat(vc, Hq // Hkv, 0), pos)
    assert np.array_equal(gqa, mha)


@pytest.mark.parametrize("BN,NKS", [(32, 1), (32, 2), (32, 7), (16, 16), (32, 64), (64, 5)])
@pytest.mark.parametrize("pos", [0, 31, 200])
def test_split_merge_equals_full_decode(BN, NKS, pos):
    Hq, Hkv = 8, 2
    q = O.fill_normal_f16(31, (Hq, D))
    kc = O.fill_normal_f16(32, (Hkv, 256, D))
    vc = O.fill_normal_f16(33, (Hkv, 256, D))
    att, lse = O.decode_split(q, kc, vc, pos, BN, NKS)
    merged = O.splitk_merge(att, lse, Hq)
    full = O.attention_decode(q, kc, vc, pos)
    assert np.max(np.abs(merged - full)) < 2e-6
