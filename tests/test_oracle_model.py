"""CPU pins of the Qwen3 forward oracle (oracle/qwen3.py).

Each step is checked against torch's own fp64 routines (rms_norm, silu,
linear, scaled_dot_product_attention), the whole forward against a
torch-library fp64 forward written in the standard pre-norm form (residual
adds explicit, not fused into the next norm), and invariants that a
plausible mistake breaks: zero o_proj/down weights reduce the network to
final-norm -> lm_head in closed form; a prefill row equals a decode step at
that position; argmax ties resolve to the smallest index.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from grout_amd.model import Qwen3Config
from oracle import qwen3 as Q

TINY = Qwen3Config(num_layers=2, hidden_size=256, intermediate_size=512, num_attention_heads=4,
                   num_key_value_heads=2, vocab_size=300)
TINY_G8 = Qwen3Config(num_layers=1, hidden_size=128, intermediate_size=256,
                      num_attention_heads=8, num_key_value_heads=1, vocab_size=77)


def t64(bits):
    return torch.from_numpy(O.h2f(bits).astype(np.float64))


def f16_ulp(x):
    """Spacing of fp16 numbers at |x| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - 10)


def test_rms_norm_matches_torch_fp64():
    x = O.fill_normal_f16(O.seed_for("mx"), (7, 2560))
    r = O.fill_normal_f16(O.seed_for("mr"), (7, 2560))
    w = O.fill_uniform_f16(O.seed_for("mw"), 0.8, 1.2, (2560,))
    got = O.h2f(Q.rms_norm(x, w, 1e-6))
    ref = F.rms_norm(t64(x), (2560,), t64(w), 1e-6).numpy()
    assert np.all(np.abs(got - ref) <= f16_ulp(ref))
    out, res = Q.add_rms_norm(r, x, w, 1e-6)
    c = t64(r) + t64(x)
    assert np.array_equal(res, Q.f16_bits(c.numpy()))
    ref = F.rms_norm(c, (2560,), t64(w), 1e-6).numpy()
    assert np.all(np.abs(O.h2f(out) - ref) <= 1.01 * f16_ulp(ref))
    # scale invariance: norm(a x) == norm(x) for a power of two
    assert np.array_equal(Q.rms_norm(Q.f16_bits(O.h2f(x) * 4), w, 1e-12), Q.rms_norm(x, w, 1e-12))


def test_silu_mul_matches_torch_and_gate_order():
    gu = O.fill_normal_f16(O.seed_for("gu"), (3, 2 * 64))
    got = O.h2f(Q.silu_mul(gu, 64))
    g, u = t64(gu)[:, :64], t64(gu)[:, 64:]
    ref = (F.silu(g) * u).numpy()
    assert np.all(np.abs(got - ref) <= f16_ulp(ref) / 2 + 1e-12)
    # silu applies to the first half: gate = -20 gives ~0 whatever up is,
    # gate = +20 passes up through scaled by 20.
    row = Q.f16_bits(np.r_[[-20.0] * 8, [5.0] * 8])
    assert np.all(np.abs(O.h2f(Q.silu_mul(row, 8))) < 1e-6)
    row = Q.f16_bits(np.r_[[20.0] * 8, [5.0] * 8])
    assert np.allclose(O.h2f(Q.silu_mul(row, 8)), 100.0)


def test_linear_matches_torch_fp64():
    x = O.fill_normal_f16(O.seed_for("lx"), (5, 256))
    w = O.fill_normal_f16(O.seed_for("lw"), (40, 256))
    ref = F.linear(t64(x), t64(w)).numpy()
    got = O.h2f(Q.linear(x, w))
    assert np.all(np.abs(got - ref) <= f16_ulp(ref) / 2 + 1e-9)


def test_argmax_ties_to_smallest_index():
    v = Q.f16_bits(np.array([0.0, 3.0, -1.0, 3.0, 2.0]))
    assert Q.argmax(v) == 1
    v = Q.f16_bits(np.full(5000, -7.0))
    assert Q.argmax(v) == 0


def rope64(x, pos, theta):
    """NeoX RoPE in fp64: x [S, H, 128], rotate_half form."""
    inv = 1.0 / theta ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128)
    ang = torch.outer(torch.as_tensor(pos, dtype=torch.float64), inv)
    cos = torch.cat([ang.cos(), ang.cos()], -1)[:, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[:, None, :]
    rot = torch.cat([-x[..., 64:], x[..., :64]], -1)
    return x * cos + rot * sin


def torch_forward(cfg, host, tokens):
    """Standard pre-norm Qwen3 forward from torch library ops, fp64, no
    intermediate fp16 rounding.  Returns logits of every position."""
    eps, H = cfg.rms_norm_eps, cfg.hidden_size
    Hq, Hkv, I = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.intermediate_size
    qd, kd = Hq * 128, Hkv * 128
    S = len(tokens)
    ids = torch.as_tensor(np.asarray(tokens, np.int64))
    x = F.embedding(ids, t64(host["embed_tokens"]))
    pos = np.arange(S)
    for L in host["layers"]:
        h = F.rms_norm(x, (H,), t64(L["input_layernorm"]), eps)
        W = t64(L["qkv_proj"])
        q = F.linear(h, W[:qd]).view(S, Hq, 128)
        k = F.linear(h, W[qd:qd + kd]).view(S, Hkv, 128)
        v = F.linear(h, W[qd + kd:]).view(S, Hkv, 128)
        q = rope64(F.rms_norm(q, (128,), t64(L["q_norm"]), eps), pos, cfg.rope_theta)
        k = rope64(F.rms_norm(k, (128,), t64(L["k_norm"]), eps), pos, cfg.rope_theta)
        G = Hq // Hkv
        kk = k.repeat_interleave(G, dim=1).transpose(0, 1)
        vv = v.repeat_interleave(G, dim=1).transpose(0, 1)
        a = F.scaled_dot_product_attention(q.transpose(0, 1), kk, vv, is_causal=True)
        x = x + F.linear(a.transpose(0, 1).reshape(S, qd), t64(L["o_proj"]))
        h2 = F.rms_norm(x, (H,), t64(L["post_attention_layernorm"]), eps)
        gu = F.linear(h2, t64(L["gate_up_proj"]))
        x = x + F.linear(F.silu(gu[:, :I]) * gu[:, I:], t64(L["down_proj"]))
    head = host["lm_head"] if host.get("lm_head") is not None else host["embed_tokens"]
    return F.linear(F.rms_norm(x, (H,), t64(host["norm"]), eps), t64(head)).numpy()


@pytest.mark.parametrize("cfg", [TINY, TINY_G8], ids=["g2", "g8"])
def test_forward_matches_torch_library_forward(cfg):
    host = Q.random_host_weights(cfg, seed=11, std=0.05)
    rng = np.random.default_rng(5)
    tokens = rng.integers(0, cfg.vocab_size, 23)
    orc = Q.Qwen3Oracle(cfg, host, max_ctx=64)
    logits, tok = orc.prefill(tokens)
    ref = torch_forward(cfg, host, tokens)[-1]
    err = np.abs(logits - ref)
    scale = np.abs(ref).max()
    print(f"logit scale {scale:.3f} max_abs {err.max():.2e}")
    # fp16 storage of every intermediate (~5e-4 relative each) vs none.
    assert err.max() <= 2e-3 * max(1.0, scale) + 2e-3
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > 4 * err.max():
        assert tok == int(np.argmax(ref))


def test_prefill_row_equals_decode_step():
    cfg = TINY
    host = Q.random_host_weights(cfg, seed=3)
    tokens = np.random.default_rng(1).integers(0, cfg.vocab_size, 12)
    a = Q.Qwen3Oracle(cfg, host, max_ctx=32)
    full, _ = a.prefill(tokens)
    b = Q.Qwen3Oracle(cfg, host, max_ctx=32)
    b.prefill(tokens[:-1])
    step, _ = b.decode(int(tokens[-1]))
    assert np.all(np.abs(step - full) <= f16_ulp(full))
    for l in range(cfg.num_layers):
        assert np.array_equal(a.k[l], b.k[l]) and np.array_equal(a.v[l], b.v[l])


def test_zero_blocks_reduce_to_norm_and_head():
    cfg = TINY
    host = Q.random_host_weights(cfg, seed=9)
    for L in host["layers"]:
        L["o_proj"][:] = 0
        L["down_proj"][:] = 0
    tokens = [5, 17, 200, 42]
    logits, _ = Q.Qwen3Oracle(cfg, host, max_ctx=16).prefill(tokens)
    e = t64(host["embed_tokens"][tokens[-1]])
    normed = F.rms_norm(e, (cfg.hidden_size,), t64(host["norm"]), cfg.rms_norm_eps)
    # the engine stores the normed row as fp16 before the lm_head product
    normed = t64(Q.f16_bits(normed.numpy()))
    ref = F.linear(normed, t64(host["embed_tokens"])).numpy()
    # half an ulp for the logit's rounding, plus a few normed elements whose
    # fp32-vs-fp64 norm rounds the other way (2^-11 * |E| ~ 1e-5 each)
    assert np.all(np.abs(logits - ref) <= f16_ulp(ref) / 2 + 5e-5)
