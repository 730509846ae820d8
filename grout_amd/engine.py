"""Attention state of grout's engine: per-layer KV caches, RoPE tables, the two
StepGraph attention ops, and the decode-step HIP graph runner.

Mirrors src/model.rs: KV caches allocated as zeros [Hkv, max_ctx, D]
(1587-1599) and zeroed in place on reset so graph pointers stay valid
(536-565, 2044-2068); GraphOp::QkNormRopeKvPrefill / GraphOp::Attention
execution (4515-4560 -> 4753-4910); DecodeCudaGraphRunner (408-596).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from typing import Optional, Sequence, Union

import torch

from . import ops
from ._lib import DecodeLayer, call, lib

HEAD_DIM = 128


@dataclass(frozen=True)
class AttentionConfig:
    """The Qwen3Config fields the attention path reads (src/config.rs:7-33)."""
    num_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int = HEAD_DIM
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_ctx: int = 32768

    def validate(self) -> None:
        if self.head_dim != HEAD_DIM:
            raise ValueError(f"expected head_dim={HEAD_DIM}, got {self.head_dim}")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("num_attention_heads must be a multiple of num_key_value_heads")
        if not (math.isfinite(self.rms_norm_eps) and self.rms_norm_eps > 0):
            raise ValueError(f"rms_norm_eps={self.rms_norm_eps} must be a positive finite float")
        if not (math.isfinite(self.rope_theta) and self.rope_theta > 0):
            raise ValueError(f"rope_theta={self.rope_theta} must be a positive finite float")

    @property
    def num_kv_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads


class AttentionEngine:
    """Owns the KV caches and executes the attention ops of every layer."""

    def __init__(self, cfg: AttentionConfig, q_norm: Sequence[torch.Tensor],
                 k_norm: Sequence[torch.Tensor], device: Union[str, torch.device] = "cuda"):
        cfg.validate()
        if len(q_norm) != cfg.num_layers or len(k_norm) != cfg.num_layers:
            raise ValueError("one q_norm and one k_norm weight per layer are required")
        self.cfg = cfg
        self.device = torch.device(device)
        shape = (cfg.num_key_value_heads, cfg.max_ctx, cfg.head_dim)
        self.k_caches = [torch.zeros(shape, dtype=torch.float16, device=self.device)
                         for _ in range(cfg.num_layers)]
        self.v_caches = [torch.zeros(shape, dtype=torch.float16, device=self.device)
                         for _ in range(cfg.num_layers)]
        self.q_norm = [w.to(self.device, torch.float16).contiguous() for w in q_norm]
        self.k_norm = [w.to(self.device, torch.float16).contiguous() for w in k_norm]
        self.rope = ops.rope_tables(cfg.max_ctx, cfg.head_dim, cfg.rope_theta, self.device)

    # -- StepGraph ops --------------------------------------------------------
    def execute_qk_norm_rope_kv_prefill_op(self, layer_idx: int, q, k, v, position_start: int,
                                           out: Optional[torch.Tensor] = None) -> torch.Tensor:
        S = q.shape[0]
        if position_start + S > self.cfg.max_ctx:
            raise ValueError(f"fused qk/rope/kv range [{position_start}..{position_start + S}) "
                             f"exceeds max_seq_len {self.cfg.max_ctx}")
        return ops.qk_norm_rope_kv_prefill(q, k, v, self.q_norm[layer_idx], self.k_norm[layer_idx],
                                           self.rope, self.k_caches[layer_idx],
                                           self.v_caches[layer_idx], position_start,
                                           self.cfg.rms_norm_eps, out)

    def execute_attention_op(self, layer_idx: int, q, position: Union[int, torch.Tensor],
                             out: Optional[torch.Tensor] = None) -> torch.Tensor:
        return ops.attention(q, self.k_caches[layer_idx], self.v_caches[layer_idx], position, out)

    def reset(self) -> None:
        """Zero every cache in place (device pointers unchanged, graphs stay valid)."""
        for t in self.k_caches + self.v_caches:
            t.zero_()

    def build_decode_graph(self, num_splits: Optional[int] = None) -> "DecodeGraph":
        return DecodeGraph(self, num_splits)


class DecodeGraph:
    """HIP graph of the attention part of one decode step over all layers:
    per layer the fused norm/RoPE/KV write + split-K pass, then the merge
    (grout_attn_decode_fused).  Callers write each layer's QKV projection
    into `qkv[layer]` and read `attn_out[layer]`."""

    def __init__(self, eng: AttentionEngine, num_splits: Optional[int] = None):
        cfg = eng.cfg
        dev = eng.device
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        self.eng = eng
        self.num_splits = num_splits or ops.default_splits(cfg.max_ctx, Hq, Hkv)
        self.qkv = [torch.zeros((Hq + 2 * Hkv) * D, dtype=torch.float16, device=dev)
                    for _ in range(cfg.num_layers)]
        self.attn_out = [torch.zeros((Hq, D), dtype=torch.float16, device=dev)
                         for _ in range(cfg.num_layers)]
        self.workspace = ops.decode_workspace(Hq, Hkv, self.num_splits, dev)
        layers = (DecodeLayer * cfg.num_layers)()
        for i in range(cfg.num_layers):
            layers[i] = DecodeLayer(self.qkv[i].data_ptr(), eng.q_norm[i].data_ptr(),
                                    eng.k_norm[i].data_ptr(), None,
                                    eng.k_caches[i].data_ptr(), eng.v_caches[i].data_ptr(),
                                    self.attn_out[i].data_ptr())
        handle = C.c_void_p()
        torch.cuda.synchronize(dev)
        cos, sin = eng.rope
        call("grout_decode_graph_create", layers, cfg.num_layers, C.c_void_p(cos.data_ptr()),
             C.c_void_p(sin.data_ptr()), C.c_void_p(self.workspace.data_ptr()),
             self.workspace.numel() * 4, Hq, Hkv, D, cfg.max_ctx, self.num_splits,
             cfg.rms_norm_eps, 1.0 / math.sqrt(D),
             C.c_void_p(torch.cuda.current_stream(dev).cuda_stream), C.byref(handle))
        self._h = handle

    def launch_step(self, position: int) -> None:
        """Replay the graph for `position` on the current stream (async); a
        position one past the previous launch's needs no upload (the graph's
        last merge leaves it in the position word)."""
        if self._h is None:
            raise RuntimeError("decode graph destroyed")
        call("grout_decode_graph_launch", self._h, position,
             C.c_void_p(torch.cuda.current_stream(self.eng.device).cuda_stream))

    def destroy(self) -> None:
        if self._h is not None:
            lib().grout_decode_graph_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass
