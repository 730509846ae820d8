"""CPU restatement of the Qwen3 forward pass the engine runs (test
infrastructure only: tests/, __graft_entry__.smoke() and bench.py's CPU
baseline use it as the checker; the product never calls it).

Follows the reference's decode step (build_decode_graph_scope,
src/model.rs:2631-4006) and prefill layer sequence (src/model.rs:4031-4678):

    hidden = embed_tokens[token]                          (src/kernels.rs:1893-1938)
    per layer l:
      normed = l == 0 ? rms_norm(hidden)                  (src/kernels.rs:1530-1569)
                      : add_rms_norm(hidden_after_attn, ff_down) -> (normed, hidden)
                                                          (src/kernels.rs:4518-4657)
      [q | k | v] = normed @ qkv_proj^T                   (src/model.rs:3466-3474)
      q_rope, K/V cache rows = qk_norm_rope_kv(q, k, v)   (src/kernels.rs:4837-5452)
      attn = causal GQA attention, scale 1/sqrt(128)      (src/kernels.rs:2559-4304)
      ff_normed, hidden_after_attn = add_rms_norm(hidden, attn @ o_proj^T)
                                                          (src/model.rs:3808-3836)
      ff = silu(gate) * up, [gate | up] = ff_normed @ gate_up_proj^T
                                                          (src/kernels.rs:1493-1522)
      ff_down = ff @ down_proj^T                          (src/model.rs:3882-3892)
    normed = add_rms_norm(hidden_after_attn, ff_down, norm)  (src/model.rs:3896-3910)
    logits = normed @ lm_head^T; token = argmax, ties to the smallest index
                                                          (src/kernels.rs:1571-1740)

Every tensor the engine stores as fp16 is rounded to fp16 here at the same
point.  Norm math is fp32 (as in the kernels); products are accumulated in
fp64 and rounded once, so the GPU's fp32 accumulation differs from this by
rounding only.  The fused norm/RoPE/KV write and the attention come from the
C oracle (grout_oracle.c).

Pinned by tests/test_oracle_model.py: each step against torch's library
routines in fp64 (rms_norm, silu, linear, scaled_dot_product_attention), the
whole forward against a torch-library fp64 forward, and invariants (zero
o_proj/down reduce the network to norm -> lm_head in closed form; a prefill
row equals a decode step at that position; argmax ties).
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import numpy as np

from . import oracle as O

D = 128


def _f(a: np.ndarray) -> np.ndarray:
    """fp16 bit patterns -> fp32 (exact widening)."""
    return np.ascontiguousarray(a, np.uint16).view(np.float16).astype(np.float32)


def f16_bits(x: np.ndarray) -> np.ndarray:
    """fp32/fp64 values -> fp16 bit patterns (round to nearest even)."""
    return np.ascontiguousarray(np.asarray(x, np.float64).astype(np.float16)).view(np.uint16)


def rms_norm(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """rows of f16 -> f16(x * (1/sqrt(sum(x^2)/H + eps)) * w), fp32 math."""
    x = _f(x_bits).astype(np.float32)
    return _norm_rows(x, w_bits, eps)


def add_rms_norm(res_bits, x_bits, w_bits, eps: float):
    """c = residual + x (fp32); returns (f16(norm(c) * w), f16(c))."""
    c = (_f(res_bits).astype(np.float32) + _f(x_bits).astype(np.float32)).astype(np.float32)
    return _norm_rows(c, w_bits, eps), f16_bits(c)


def _norm_rows(c: np.ndarray, w_bits, eps: float) -> np.ndarray:
    H = c.shape[-1]
    ss = np.sum(c.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    inv = (np.float32(1.0) / np.sqrt(ss / np.float32(H) + np.float32(eps))).astype(np.float32)
    w = _f(w_bits).astype(np.float32)
    return f16_bits((c * inv).astype(np.float32) * w)


def silu_mul(gate_up_bits: np.ndarray, inter: int) -> np.ndarray:
    """gate_up rows [gate | up] -> f16(gate * sigmoid(gate) * up)."""
    gu = _f(gate_up_bits).astype(np.float64)
    g, u = gu[..., :inter], gu[..., inter:]
    return f16_bits(g / (1.0 + np.exp(-g)) * u)


def linear(x_bits: np.ndarray, w_bits: np.ndarray, w64: Optional[np.ndarray] = None) -> np.ndarray:
    """f16(x @ W^T), W row-major [n][k], accumulated in fp64 (w64: W already
    widened to fp64)."""
    x = _f(x_bits).astype(np.float64)
    w = _f(w_bits).astype(np.float64) if w64 is None else w64
    return f16_bits(x @ w.T)


def argmax(logits_bits: np.ndarray) -> int:
    """Largest fp16 logit, ties to the smallest index (np.argmax's rule)."""
    return int(np.argmax(_f(logits_bits)))


class Qwen3Oracle:
    """Host weights (fp16 bit patterns) + per-layer KV caches [Hkv][max_ctx][128].

    decode_w64 (low-bit weights): {key: fp64 matrix} for keys (l, "qkv_proj"),
    (l, "o_proj"), (l, "gate_up_proj"), (l, "down_proj") and "lm_head".  A
    decode step multiplies by these (the decode GEMVs compute with the fp32
    dequantized weights), and so does the head after a prefill (one row,
    the GEMV); prefill and extend rows multiply by the fp16 matrices in
    `host` (the dequantized weights rounded to f16 for the GEMM)."""

    def __init__(self, cfg, host: Dict, max_ctx: int, decode_w64: Optional[Dict] = None):
        self.cfg = cfg
        self.w = host
        self.max_ctx = max_ctx
        self.decode_w64 = decode_w64 or {}
        Hkv = cfg.num_key_value_heads
        self.k = [np.zeros((Hkv, max_ctx, D), np.uint16) for _ in range(cfg.num_layers)]
        self.v = [np.zeros((Hkv, max_ctx, D), np.uint16) for _ in range(cfg.num_layers)]
        self.cos, self.sin = O.rope_table(max_ctx, D, cfg.rope_theta)
        self.next_pos = 0
        self._w64: Dict = {}

    def _lin(self, x_bits, key, w_bits, decode: bool = False):
        """linear() with the fp64 copy of each weight made once."""
        if decode and key in self.decode_w64:
            return linear(x_bits, w_bits, self.decode_w64[key])
        if key not in self._w64:
            self._w64[key] = np.ascontiguousarray(w_bits, np.uint16).view(np.float16).astype(
                np.float64)
        return linear(x_bits, w_bits, self._w64[key])

    def reset(self) -> None:
        for a in self.k + self.v:
            a[:] = 0
        self.next_pos = 0

    def head_weight(self) -> np.ndarray:
        return self.w["lm_head"] if self.w.get("lm_head") is not None else self.w["embed_tokens"]

    def forward(self, tokens: Sequence[int], pos0: int, nthreads: int = 1, decode: bool = False):
        """Runs len(tokens) tokens at positions pos0.. and returns (f16 logits
        of the last one as fp32, greedy token); decode: the one-token decode
        step (its projections use decode_w64)."""
        c = self.cfg
        ids = np.asarray(tokens, np.int64)
        S = ids.size
        Hq, Hkv, I, eps = c.num_attention_heads, c.num_key_value_heads, c.intermediate_size, \
            c.rms_norm_eps
        qd, kd = Hq * D, Hkv * D
        hidden = self.w["embed_tokens"][ids]
        hidden_after_attn = ff_down = None
        for l, L in enumerate(self.w["layers"]):
            if l == 0:
                normed = rms_norm(hidden, L["input_layernorm"], eps)
            else:
                normed, hidden = add_rms_norm(hidden_after_attn, ff_down, L["input_layernorm"], eps)
            qkv = self._lin(normed, (l, "qkv_proj"), L["qkv_proj"], decode)
            q = np.ascontiguousarray(qkv[:, :qd]).reshape(S, Hq, D)
            k = np.ascontiguousarray(qkv[:, qd:qd + kd]).reshape(S, Hkv, D)
            v = np.ascontiguousarray(qkv[:, qd + kd:]).reshape(S, Hkv, D)
            q_rope = O.qk_norm_rope_kv_prefill(q, k, v, L["q_norm"], L["k_norm"], self.cos,
                                               self.sin, self.k[l], self.v[l], pos0, eps)
            attn = O.attention_prefill_rows(q_rope, self.k[l], self.v[l], pos0, nthreads=nthreads)
            attn_bits = f16_bits(attn.reshape(S, qd))
            attn_proj = self._lin(attn_bits, (l, "o_proj"), L["o_proj"], decode)
            ff_normed, hidden_after_attn = add_rms_norm(hidden, attn_proj,
                                                        L["post_attention_layernorm"], eps)
            ff = silu_mul(self._lin(ff_normed, (l, "gate_up_proj"), L["gate_up_proj"], decode), I)
            ff_down = self._lin(ff, (l, "down_proj"), L["down_proj"], decode)
        normed, _ = add_rms_norm(hidden_after_attn[-1:], ff_down[-1:], self.w["norm"], eps)
        logits = self._lin(normed, "lm_head", self.head_weight(), True)[0]
        self.next_pos = pos0 + S
        return _f(logits).astype(np.float32), argmax(logits)

    def prefill(self, tokens: Sequence[int], nthreads: int = 1):
        return self.forward(tokens, 0, nthreads)

    def decode(self, token: int, nthreads: int = 1):
        return self.forward([token], self.next_pos, nthreads, decode=True)


def random_host_weights(cfg, seed: int, std: float = 0.02, norm_lo: float = 0.8,
                        norm_hi: float = 1.2) -> Dict:
    """Seeded fp16 weights (bit patterns): matrices ~ N(0, std), norm weights
    ~ U(norm_lo, norm_hi), from numpy's PCG64 generator (fast enough for the
    Qwen3-4B layer shapes)."""
    H = cfg.hidden_size
    rng = np.random.default_rng(seed)

    def mat(shape):
        a = rng.standard_normal(shape, dtype=np.float32)
        a *= np.float32(std)
        return a.astype(np.float16).view(np.uint16)

    def vec(n):
        return rng.uniform(norm_lo, norm_hi, n).astype(np.float16).view(np.uint16)

    layers: List[Dict[str, np.ndarray]] = []
    shapes = cfg.layer_shapes()
    for _ in range(cfg.num_layers):
        layers.append({name: vec(shp[0]) if len(shp) == 1 else mat(shp)
                       for name, shp in shapes.items()})
    out = {"embed_tokens": mat((cfg.vocab_size, H)), "norm": vec(H), "layers": layers,
           "lm_head": None}
    if not cfg.tie_word_embeddings:
        out["lm_head"] = mat((cfg.vocab_size, H))
    return out
