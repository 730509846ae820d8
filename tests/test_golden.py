"""The oracle against the committed golden fixtures (tests/golden/
attention_golden.npz, written by tests/golden/make_golden.py in torch
float64 from the same seeded inputs): the benchmark configurations at their
full shapes.  Rotated q / k within one f16 ulp of the float64 values plus
what the reference's f32 RoPE angle can miss (the fixtures' angles are
exact), the V row
bit-exact, attention within 1e-4 (the oracle's scores and exponentials are
fp32)."""
import importlib.util
import os

import numpy as np

import oracle as O

D = 128
HERE = os.path.dirname(os.path.abspath(__file__))
_spec = importlib.util.spec_from_file_location("make_golden",
                                               os.path.join(HERE, "golden", "make_golden.py"))
G = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(G)
GOLD = np.load(os.path.join(HERE, "golden", "attention_golden.npz"))


def within_rope(bits, want, pos, what):
    """Rotated f16 values against float64 `want` [..., rows, 128] at query
    positions `pos` [rows]: one f16 ulp plus the rotation the reference's f32
    angle (pos * inv_freq in f32) can miss, pos * 2^-22 radians at most,
    times the norm of each element's (i, i+64) pair."""
    got = bits.view(np.float16).astype(np.float64)
    want = want.astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -14))) - 10)
    pair = np.sqrt(want[..., :D // 2] ** 2 + want[..., D // 2:] ** 2)
    slack = np.concatenate([pair, pair], -1) * (np.asarray(pos, np.float64)[:, None] * 2.0 ** -22)
    err = np.abs(got - want)
    assert np.all(err <= ulp + slack), (what, float((err / (ulp + slack)).max()))


def close(got, want, tol, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert err.max() <= tol, (what, float(err.max()))


def c1_inputs(max_ctx):
    """Config 1 inputs as the fixture script draws them, in a max_ctx cache."""
    Hq, Hkv, pos = 16, 8, 512
    kc = np.zeros((Hkv, max_ctx, D), np.uint16)
    vc = np.zeros_like(kc)
    kc[:, :pos], vc[:, :pos] = G.normal("g1k", (Hkv, pos, D)), G.normal("g1v", (Hkv, pos, D))
    qkv = G.normal("g1qkv", ((Hq + 2 * Hkv) * D,))
    gq = O.fill_uniform_f16(O.seed_for("g1gq"), 0.8, 1.2, D)
    gk = O.fill_uniform_f16(O.seed_for("g1gk"), 0.8, 1.2, D)
    return Hq, Hkv, pos, kc, vc, qkv, gq, gk


def c3_inputs():
    S, Hq, Hkv = 2048, 32, 8
    q, k, v = G.normal("g3q", (S, Hq, D)), G.normal("g3k", (S, Hkv, D)), G.normal("g3v", (S, Hkv, D))
    gq = O.fill_uniform_f16(O.seed_for("g3gq"), 0.8, 1.2, D)
    gk = O.fill_uniform_f16(O.seed_for("g3gk"), 0.8, 1.2, D)
    return S, Hq, Hkv, q, k, v, gq, gk


def decode_inputs(tag, Hq, Hkv, ctx):
    return (G.normal(tag + "q", (Hq, D)), G.normal(tag + "k", (Hkv, ctx, D)),
            G.normal(tag + "v", (Hkv, ctx, D)))


def test_config1_oracle_vs_golden():
    Hq, Hkv, pos, kc, vc, qkv, gq, gk = c1_inputs(1024)
    cos, sin = O.rope_table(1024, D, 1e6)
    q_rot = O.qk_norm_rope_kv_decode(qkv, gq, gk, cos, sin, kc, vc, pos, Hq, Hkv, 1e-6)
    within_rope(q_rot, GOLD["c1_q_rot"], [pos], "q")
    within_rope(kc[:, pos], GOLD["c1_k_rot"], [pos], "k row")
    assert np.array_equal(vc[:, pos], qkv[(Hq + Hkv) * D:].reshape(Hkv, D))
    close(O.attention_decode(q_rot, kc, vc, pos, nthreads=8), GOLD["c1_out"], 1e-4, "out")


def test_decode_configs_oracle_vs_golden():
    for tag, Hq, Hkv, ctx, key in [("g2", 32, 8, 4096, "c2_out")] + [
            (f"g4{c}", 64, 8, c, f"c4_out_{c}") for c in (8192, 16384, 32768)]:
        q, kc, vc = decode_inputs(tag, Hq, Hkv, ctx)
        close(O.attention_decode(q, kc, vc, ctx - 1, nthreads=8), GOLD[key], 1e-4, key)


def test_config3_oracle_vs_golden():
    S, Hq, Hkv, q, k, v, gq, gk = c3_inputs()
    cos, sin = O.rope_table(S, D, 1e6)
    kc = np.zeros((Hkv, S, D), np.uint16)
    vc = np.zeros_like(kc)
    q_rot = O.qk_norm_rope_kv_prefill(q, k, v, gq, gk, cos, sin, kc, vc, 0, 1e-6)
    rows = GOLD["c3_rows"]
    # [rows, heads, 128] -> [heads, rows, 128] so the row positions line up
    within_rope(q_rot[rows].transpose(1, 0, 2), GOLD["c3_q_rot"].transpose(1, 0, 2), rows, "q rows")
    within_rope(kc[:, rows], GOLD["c3_k_rot"].transpose(1, 0, 2), rows, "k rows")
    out = O.attention_prefill_rows(q_rot, kc, vc, 0, rows=rows, nthreads=8)
    close(out, GOLD["c3_out"], 1e-4, "rows")
