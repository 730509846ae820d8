"""Writes tests/golden/attention_golden.npz: expected outputs of the attention
hot path at the benchmark configurations, computed in float64 with torch from
the same seeded inputs the tests generate.

Inputs come from the oracle's seeded generator (SplitMix64 + Box-Muller,
rounded once to f16; its first values are pinned by tests/test_oracle.py).
Everything downstream is torch float64 and independent of the oracle's C
code: RMSNorm (x / sqrt(mean(x^2) + eps) * gamma), NeoX RoPE with exact
angles pos * theta^(-i/64), rounding of the rotated q / k to f16 where the
kernels store f16, then scaled_dot_product_attention (GQA, causal).

  python tests/golden/make_golden.py        # rewrites the .npz (a few seconds)

Cases (the benchmark configurations at their single-GPU shapes):
  c1: Qwen3-0.6B decode step: 512 cached positions, the new token's q, k, v
      through QK-norm + RoPE at position 512, attention over 513 positions;
  c2: Qwen3-4B decode attention, ctx 4096 (q given post-RoPE);
  c4: Qwen3-32B decode attention, ctx 8192 / 16384 / 32768;
  c3: Qwen3-4B prefill S=2048: QK-norm + RoPE of every row, then causal
      attention on sampled rows.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402  (the seeded input generator only)

D, THETA, EPS = 128, 1e6, 1e-6
OUT = os.path.join(HERE, "attention_golden.npz")


def f16(a16):
    return torch.from_numpy(a16.view(np.float16).astype(np.float64))


def round16(x):
    return x.to(torch.float16).to(torch.float64)


def norm_rope(x, gamma, pos):
    """x [..., n, 128] float64 at positions pos [n] -> rotated, float64."""
    n = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + EPS) * gamma
    ang = pos.to(torch.float64)[:, None] * THETA ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    c, s = torch.cos(ang), torch.sin(ang)
    lo, hi = n[..., :D // 2], n[..., D // 2:]
    return torch.cat([lo * c - hi * s, lo * s + hi * c], -1)


def sdpa(q, k, v, q_pos):
    """q [S, Hq, D], k/v [Hkv, n, D] float64; query s at position q_pos[s]."""
    n = k.shape[1]
    mask = torch.arange(n)[None, :] <= q_pos[:, None]
    o = torch.nn.functional.scaled_dot_product_attention(
        q.permute(1, 0, 2)[None], k[None], v[None], attn_mask=mask, enable_gqa=True)
    return o[0].permute(1, 0, 2)


def normal(tag, shape):
    return O.fill_normal_f16(O.seed_for(tag), shape)


def gamma(tag):
    return f16(O.fill_uniform_f16(O.seed_for(tag), 0.8, 1.2, D))


def case1():
    Hq, Hkv, pos = 16, 8, 512
    kc, vc = f16(normal("g1k", (Hkv, pos, D))), f16(normal("g1v", (Hkv, pos, D)))
    qkv = f16(normal("g1qkv", ((Hq + 2 * Hkv) * D,)))
    gq, gk = gamma("g1gq"), gamma("g1gk")
    p = torch.tensor([pos])
    q_rot = norm_rope(qkv[:Hq * D].view(Hq, 1, D), gq, p)[:, 0]
    k_rot = norm_rope(qkv[Hq * D:(Hq + Hkv) * D].view(Hkv, 1, D), gk, p)[:, 0]
    v_new = qkv[(Hq + Hkv) * D:].view(Hkv, D)
    k_all = torch.cat([kc, round16(k_rot)[:, None]], 1)
    v_all = torch.cat([vc, v_new[:, None]], 1)
    out = sdpa(round16(q_rot)[None], k_all, v_all, p)[0]
    return {"c1_q_rot": q_rot, "c1_k_rot": k_rot, "c1_out": out}


def decode_case(tag, Hq, Hkv, ctx):
    q = f16(normal(tag + "q", (Hq, D)))
    kc, vc = f16(normal(tag + "k", (Hkv, ctx, D))), f16(normal(tag + "v", (Hkv, ctx, D)))
    return sdpa(q[None], kc, vc, torch.tensor([ctx - 1]))[0]


C3_ROWS = np.array([0, 1, 63, 64, 1000, 1024, 2046, 2047])


def case3():
    S, Hq, Hkv = 2048, 32, 8
    q, k, v = f16(normal("g3q", (S, Hq, D))), f16(normal("g3k", (S, Hkv, D))), f16(normal("g3v", (S, Hkv, D)))
    gq, gk = gamma("g3gq"), gamma("g3gk")
    pos = torch.arange(S)
    q_rot = norm_rope(q.permute(1, 0, 2), gq, pos).permute(1, 0, 2)      # [S, Hq, D]
    k_rot = norm_rope(k.permute(1, 0, 2), gk, pos)                        # [Hkv, S, D]
    rows = torch.from_numpy(C3_ROWS)
    out = sdpa(round16(q_rot[rows]), round16(k_rot), v.permute(1, 0, 2), rows)
    return {"c3_rows": C3_ROWS, "c3_q_rot": q_rot[rows], "c3_k_rot": k_rot[:, rows].permute(1, 0, 2),
            "c3_out": out}


def main():
    g = {}
    g.update(case1())
    g["c2_out"] = decode_case("g2", 32, 8, 4096)
    for ctx in (8192, 16384, 32768):
        g[f"c4_out_{ctx}"] = decode_case(f"g4{ctx}", 64, 8, ctx)
    g.update(case3())
    # float32 storage: 1e-7 relative, far inside every tolerance it is checked with
    arrays = {k: (v.numpy().astype(np.float32) if torch.is_tensor(v) else v) for k, v in g.items()}
    np.savez_compressed(OUT, **arrays)
    print(OUT, {k: a.shape for k, a in arrays.items()})


if __name__ == "__main__":
    main()
