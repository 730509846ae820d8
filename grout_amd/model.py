"""Qwen3 engine on one MI355X: the Python face of include/grout_engine.h.

Mirrors the reference's public API `grout::Engine` (src/api.rs:11-183):
token-based and blocking; `prefill` starts a new session and returns the last
token's logits, `decode` / `decode_greedy` advance it one token through the
captured decode-step HIP graph, `reset` clears the KV state.  Weights are
fp16 device tensors in the reference's fused layouts (qkv_proj rows
[Q | K | V], gate_up_proj rows [gate | up]); the engine borrows them, so this
object keeps references to them for its lifetime.

All compute runs in grout_amd/libgrout_attn.so; nothing here falls back to
PyTorch math.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np
import torch

from ._lib import ModelInfo as _CModelInfo
from ._lib import Qwen3Config as _CConfig
from ._lib import Qwen3Layer as _CLayer
from ._lib import Qwen3QLayer as _CQLayer
from ._lib import Qwen3QWeights as _CQWeights
from ._lib import Qwen3Weights as _CWeights
from ._lib import WPart as _CWPart
from ._lib import call, lib

HEAD_DIM = 128
LAYER_KEYS = ("input_layernorm", "qkv_proj", "q_norm", "k_norm", "o_proj",
              "post_attention_layernorm", "gate_up_proj", "down_proj")


@dataclass(frozen=True)
class Qwen3Config:
    """The Qwen3Config fields the engine reads (src/config.rs:7-33)."""
    num_layers: int
    hidden_size: int
    intermediate_size: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    head_dim: int = HEAD_DIM
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    tie_word_embeddings: bool = True
    eos_token_ids: tuple = (151645, 151643)

    @staticmethod
    def qwen3_4b() -> "Qwen3Config":
        """Qwen3-4B: 36 layers, hidden 2560, inter 9728, 32/8 heads, vocab 151936."""
        return Qwen3Config(36, 2560, 9728, 32, 8, 151936)

    @property
    def q_dim(self) -> int:
        return self.num_attention_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_key_value_heads * self.head_dim

    def layer_shapes(self) -> Dict[str, tuple]:
        H, I = self.hidden_size, self.intermediate_size
        return {
            "input_layernorm": (H,),
            "qkv_proj": (self.q_dim + 2 * self.kv_dim, H),
            "q_norm": (self.head_dim,),
            "k_norm": (self.head_dim,),
            "o_proj": (H, self.q_dim),
            "post_attention_layernorm": (H,),
            "gate_up_proj": (2 * I, H),
            "down_proj": (H, I),
        }

    def num_params(self) -> int:
        per_layer = sum(math.prod(s) for s in self.layer_shapes().values())
        embed = self.vocab_size * self.hidden_size
        head = 0 if self.tie_word_embeddings else embed
        return self.num_layers * per_layer + embed + head + self.hidden_size


@dataclass
class Qwen3Weights:
    """fp16 device tensors: embed_tokens [V][H], norm [H], lm_head (the
    embedding when tied) and one dict of LAYER_KEYS tensors per layer."""
    embed_tokens: torch.Tensor
    norm: torch.Tensor
    layers: List[Dict[str, torch.Tensor]]
    lm_head: Optional[torch.Tensor] = None

    def head(self) -> torch.Tensor:
        return self.embed_tokens if self.lm_head is None else self.lm_head

    @staticmethod
    def random(cfg: Qwen3Config, seed: int = 0, device="cuda", std: float = 0.02,
               norm_value: float = 1.0) -> "Qwen3Weights":
        """Matrices ~ N(0, std) drawn on the device, norm weights = norm_value."""
        g = torch.Generator(device=device)
        g.manual_seed(seed)

        def mat(shape):
            t = torch.empty(shape, dtype=torch.float16, device=device)
            t.normal_(0.0, std, generator=g)
            return t

        def vec(n):
            return torch.full((n,), norm_value, dtype=torch.float16, device=device)

        layers = []
        for _ in range(cfg.num_layers):
            layer = {}
            for k, shp in cfg.layer_shapes().items():
                layer[k] = vec(shp[0]) if len(shp) == 1 else mat(shp)
            layers.append(layer)
        embed = mat((cfg.vocab_size, cfg.hidden_size))
        head = None if cfg.tie_word_embeddings else mat((cfg.vocab_size, cfg.hidden_size))
        return Qwen3Weights(embed, vec(cfg.hidden_size), layers, head)

    @staticmethod
    def from_host(host: dict, device="cuda") -> "Qwen3Weights":
        """From numpy fp16 bit patterns (uint16) in the same structure."""
        def dev(a):
            return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(device)

        layers = [{k: dev(v) for k, v in L.items()} for L in host["layers"]]
        head = host.get("lm_head")
        return Qwen3Weights(dev(host["embed_tokens"]), dev(host["norm"]), layers,
                            None if head is None else dev(head))

    def check(self, cfg: Qwen3Config) -> None:
        def need(t, shape, what):
            if tuple(t.shape) != tuple(shape) or t.dtype != torch.float16 or not t.is_cuda \
                    or not t.is_contiguous():
                raise ValueError(f"{what}: expected contiguous fp16 cuda {shape}, got "
                                 f"{t.dtype} {tuple(t.shape)} on {t.device}")

        need(self.embed_tokens, (cfg.vocab_size, cfg.hidden_size), "embed_tokens")
        need(self.norm, (cfg.hidden_size,), "norm")
        need(self.head(), (cfg.vocab_size, cfg.hidden_size), "lm_head")
        if len(self.layers) != cfg.num_layers:
            raise ValueError(f"{len(self.layers)} layers, config has {cfg.num_layers}")
        for i, L in enumerate(self.layers):
            for k, shp in cfg.layer_shapes().items():
                need(L[k], shp, f"layer {i} {k}")


# Weight formats (ggml type ids for the low-bit ones; include/grout_engine.h).
F16, Q8_0, Q4_K, Q5_K, Q6_K = 0, 8, 12, 13, 14
QBLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
          Q6_K: (256, 210)}  # (weights, bytes) per block
QLAYER_VECS = ("input_layernorm", "q_norm", "k_norm", "post_attention_layernorm")
QLAYER_MATS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


class QuantWeights:
    """Mixed-format weights on the device for grout_engine_create_q, as a
    GGUF file holds them (the reference's Weight / MatrixWeight,
    src/weights.rs:7-56).

    Every matrix is (fmt, data): fmt F16 with data an fp16 [rows][k] array
    (numpy fp16 or uint16 bit patterns), or Q8_0 / Q4_K / Q5_K / Q6_K with data the
    tensor's ggml blocks (uint8, rows contiguous).  q|k|v and gate|up runs of
    one low-bit format are concatenated and repacked as one part (one GEMV in
    the decode step); a format change starts a new part.  The norm vectors
    are fp16.  lm_head None ties the head to embed_tokens (one device copy)."""

    def __init__(self, cfg: Qwen3Config, embed_tokens, norm, layers: List[Dict],
                 lm_head=None, device="cuda"):
        self.cfg = cfg
        self._keep: List[torch.Tensor] = []
        self._device = device
        H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
        qd, kd = cfg.q_dim, cfg.kv_dim
        if len(layers) != cfg.num_layers:
            raise ValueError(f"{len(layers)} layers, config has {cfg.num_layers}")
        self.embed = self._group([(embed_tokens, V)], H, "embed_tokens")[0]
        self.lm_head = self.embed if lm_head is None else \
            self._group([(lm_head, V)], H, "lm_head")[0]
        self.norm = self._vec(norm, H, "norm")
        self.layers = []
        for i, L in enumerate(layers):
            d = {k: self._vec(L[k], HEAD_DIM if k in ("q_norm", "k_norm") else H,
                              f"layer {i} {k}") for k in QLAYER_VECS}
            d["qkv"] = self._group([(L["q_proj"], qd), (L["k_proj"], kd), (L["v_proj"], kd)], H,
                                   f"layer {i} qkv")
            d["gate_up"] = self._group([(L["gate_proj"], I), (L["up_proj"], I)], H,
                                       f"layer {i} gate_up")
            d["o_proj"] = self._group([(L["o_proj"], H)], qd, f"layer {i} o_proj")[0]
            d["down_proj"] = self._group([(L["down_proj"], H)], I, f"layer {i} down_proj")[0]
            self.layers.append(d)

    def _vec(self, a, n, what) -> int:
        if isinstance(a, torch.Tensor):
            t = a.to(device=self._device, dtype=torch.float16).reshape(-1).contiguous()
        else:
            t = torch.from_numpy(np.ascontiguousarray(a).view(np.float16).reshape(-1)).to(
                self._device)
        if t.numel() != n:
            raise ValueError(f"{what}: {t.numel()} values, expected {n}")
        self._keep.append(t)
        return t.data_ptr()

    def _group(self, mats, k: int, what: str):
        """[(fmt, rows, device pointer)] for matrices [((fmt, data), rows)] in row order."""
        parts, i = [], 0
        while i < len(mats):
            fmt = int(mats[i][0][0])
            j = i
            while j + 1 < len(mats) and int(mats[j + 1][0][0]) == fmt:
                j += 1
            rows = sum(r for _, r in mats[i:j + 1])
            dev = isinstance(mats[i][0][1], torch.Tensor)  # blocks already on the device
            if fmt == F16:
                if dev:
                    t = torch.cat([m[1].to(self._device, torch.float16).reshape(r, k)
                                   for m, r in mats[i:j + 1]]).contiguous()
                else:
                    a = np.concatenate([np.ascontiguousarray(m[1]).view(np.uint16).reshape(r, k)
                                        for m, r in mats[i:j + 1]])
                    t = torch.from_numpy(a.view(np.float16)).to(self._device)
            elif fmt in QBLOCK:
                be, bb = QBLOCK[fmt]
                if k % be:
                    raise ValueError(f"{what}: k={k} is not a multiple of {be}")
                if dev:
                    raw = torch.cat([m[1].to(self._device).reshape(r, k // be * bb)
                                     for m, r in mats[i:j + 1]]).reshape(-1)
                else:
                    a = np.concatenate([np.ascontiguousarray(m[1], np.uint8).reshape(
                        r, k // be * bb) for m, r in mats[i:j + 1]])
                    raw = torch.from_numpy(a.reshape(-1)).to(self._device)
                nbytes = lib().grout_qweight_bytes(fmt, rows, k)
                if nbytes == 0:
                    raise ValueError(f"{what}: format {fmt} does not fit k={k}")
                t = torch.empty(nbytes, dtype=torch.uint8, device=self._device)
                call("grout_qweight_repack", fmt, C.c_void_p(raw.data_ptr()), rows, k,
                     C.c_void_p(t.data_ptr()), None)
                torch.cuda.synchronize()
                del raw
            else:
                raise ValueError(f"{what}: unsupported format {fmt}")
            self._keep.append(t)
            parts.append((fmt, rows, t.data_ptr()))
            i = j + 1
        return parts

    def device_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self._keep)

    @staticmethod
    def random_blocks(fmt: int, rows: int, k: int, std: float, gen: torch.Generator,
                      device="cuda") -> torch.Tensor:
        """Seeded random ggml blocks on the device: random payload and 6-bit
        scale bytes, block scales d (and dmin) set so the weights spread about
        std (Q4_K: centred by dmin = 7.5 d).  For timing and smoke runs."""
        if fmt == F16:
            return torch.empty((rows, k), dtype=torch.float16, device=device).normal_(
                0.0, std, generator=gen)
        be, bb = QBLOCK[fmt]
        b = torch.randint(0, 256, (rows * (k // be), bb), dtype=torch.uint8, device=device,
                          generator=gen)

        def f16(v):
            return torch.tensor([v], dtype=torch.float16).view(torch.uint8).to(device)

        if fmt == Q8_0:      # int8 uniform: std ~74 units
            b[:, 0:2] = f16(std / 74.0)
        elif fmt == Q4_K:    # q uniform 0..15, 6-bit scales uniform 0..63
            d = std / (32.0 * 4.6)
            b[:, 0:2] = f16(d)
            b[:, 2:4] = f16(7.5 * d)
        elif fmt == Q5_K:    # q uniform 0..31: centred by dmin = 15.5 d
            d = std / (32.0 * 9.2)
            b[:, 0:2] = f16(d)
            b[:, 2:4] = f16(15.5 * d)
        else:                # Q6_K: (q - 32) std ~18.5, int8 scales |sc| ~64
            b[:, 208:210] = f16(std / (74.0 * 18.5))
        return b.reshape(rows, -1)

    @classmethod
    def random(cls, cfg: Qwen3Config, layer_formats, embed_fmt: int, head_fmt=None,
               seed: int = 0, std: float = 0.02, device="cuda") -> "QuantWeights":
        """Random weights in the given formats: layer_formats(l) -> {"q", "k",
        "v", "o", "gate", "up", "down": fmt}; head_fmt None = tied head."""
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        H, I, V, qd, kd = (cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.q_dim,
                           cfg.kv_dim)

        def vec(n):
            return torch.ones(n, dtype=torch.float16, device=device)

        def mat(fmt, rows, k):
            return (fmt, cls.random_blocks(fmt, rows, k, std, g, device))

        layers = []
        for l in range(cfg.num_layers):
            f = layer_formats(l)
            layers.append({"input_layernorm": vec(H), "q_norm": vec(HEAD_DIM),
                           "k_norm": vec(HEAD_DIM), "post_attention_layernorm": vec(H),
                           "q_proj": mat(f["q"], qd, H), "k_proj": mat(f["k"], kd, H),
                           "v_proj": mat(f["v"], kd, H), "o_proj": mat(f["o"], H, qd),
                           "gate_proj": mat(f["gate"], I, H), "up_proj": mat(f["up"], I, H),
                           "down_proj": mat(f["down"], H, I)})
        head = None if head_fmt is None else mat(head_fmt, V, H)
        return cls(cfg, mat(embed_fmt, V, H), vec(H), layers, head, device)

    def c_struct(self):
        """(grout_qwen3_qweights, the layer array it points to)."""
        def wp(p):
            return _CWPart(p[0], p[1], p[2])

        layers = (_CQLayer * len(self.layers))()
        for i, d in enumerate(self.layers):
            L = layers[i]
            for k in QLAYER_VECS:
                setattr(L, k, d[k])
            L.num_qkv_parts = len(d["qkv"])
            for j, p in enumerate(d["qkv"]):
                L.qkv[j] = wp(p)
            L.num_gate_up_parts = len(d["gate_up"])
            for j, p in enumerate(d["gate_up"]):
                L.gate_up[j] = wp(p)
            L.o_proj = wp(d["o_proj"])
            L.down_proj = wp(d["down_proj"])
        return _CQWeights(wp(self.embed), self.norm, wp(self.lm_head), layers), layers


def _config_from_info(info) -> "tuple[Qwen3Config, int]":
    c = info.config
    eos = tuple(int(info.eos_token_ids[i]) for i in range(info.num_eos))
    cfg = Qwen3Config(c.num_layers, c.hidden_size, c.intermediate_size, c.num_q_heads,
                      c.num_kv_heads, c.vocab_size, c.head_dim, float(c.rms_norm_eps),
                      float(c.rope_theta), bool(info.tie_word_embeddings), eos)
    return cfg, int(c.max_ctx)


def inspect(model_dir: str) -> Dict:
    """Host-only check of a Qwen3 safetensors directory (grout_model_inspect):
    returns the config, max_position_embeddings and the fp16 weight bytes."""
    info = _CModelInfo()
    call("grout_model_inspect", str(model_dir).encode(), C.byref(info))
    cfg, max_pos = _config_from_info(info)
    return {"config": cfg, "max_position_embeddings": max_pos,
            "weight_bytes": int(info.weight_bytes)}


@dataclass
class Logits:
    """Last-token logits copied to the host as f32 (src/api.rs:39-44)."""
    values: np.ndarray


@dataclass(frozen=True)
class ModelMeta:
    """src/api.rs:46-57."""
    vocab_size: int
    eos_token_ids: tuple
    arch: str
    max_ctx: int


class Engine:
    """Synchronous Qwen3 engine (src/api.rs:11-183) over the C ABI."""

    def __init__(self, cfg: Qwen3Config, weights: Qwen3Weights, max_ctx: int = 4096,
                 device_ord: int = 0):
        if max_ctx <= 0:
            raise ValueError("max_ctx must be positive")
        weights.check(cfg)
        self.cfg = cfg
        self.weights = weights  # borrowed by the engine: keep alive
        self._meta = ModelMeta(cfg.vocab_size, tuple(cfg.eos_token_ids), "qwen3", max_ctx)
        c = _CConfig(cfg.num_layers, cfg.hidden_size, cfg.intermediate_size,
                     cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                     cfg.vocab_size, cfg.rms_norm_eps, cfg.rope_theta, max_ctx)
        self._layers = (_CLayer * cfg.num_layers)()
        for i, L in enumerate(weights.layers):
            for k in LAYER_KEYS:
                setattr(self._layers[i], k, L[k].data_ptr())
        w = _CWeights(weights.embed_tokens.data_ptr(), weights.norm.data_ptr(),
                      weights.head().data_ptr(), self._layers)
        self._h = C.c_void_p()
        call("grout_engine_create", C.byref(c), C.byref(w), device_ord, C.byref(self._h))
        self._logits = np.empty(cfg.vocab_size, np.float32)

    @classmethod
    def from_quantized(cls, cfg: Qwen3Config, weights: QuantWeights, max_ctx: int = 4096,
                       device_ord: int = 0) -> "Engine":
        """Engine over mixed-format (GGUF block) weights (grout_engine_create_q);
        the weights are borrowed: this object keeps them alive."""
        if max_ctx <= 0:
            raise ValueError("max_ctx must be positive")
        self = cls.__new__(cls)
        self._h = C.c_void_p()
        self.cfg = cfg
        self.weights = weights
        self._meta = ModelMeta(cfg.vocab_size, tuple(cfg.eos_token_ids), "qwen3", max_ctx)
        c = _CConfig(cfg.num_layers, cfg.hidden_size, cfg.intermediate_size,
                     cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                     cfg.vocab_size, cfg.rms_norm_eps, cfg.rope_theta, max_ctx)
        w, self._layers = weights.c_struct()
        call("grout_engine_create_q", C.byref(c), C.byref(w), device_ord, C.byref(self._h))
        self._logits = np.empty(cfg.vocab_size, np.float32)
        return self

    # -- src/api.rs:60-90
    @classmethod
    def load(cls, model_dir: str, max_ctx: int = 0, device_ord: int = 0) -> "Engine":
        """Loads a Qwen3 safetensors directory (config.json, shards) onto the
        GPU and builds the engine over it (grout_engine_load); max_ctx 0 =
        max_position_embeddings."""
        if max_ctx < 0:
            raise ValueError("max_ctx must be >= 0")
        self = cls.__new__(cls)
        self._h = C.c_void_p()
        call("grout_engine_load", str(model_dir).encode(), max_ctx, device_ord, C.byref(self._h))
        info = _CModelInfo()
        call("grout_engine_model_info", self._h, C.byref(info))
        self.cfg, ctx = _config_from_info(info)
        self.weights = None  # owned by the engine
        self._meta = ModelMeta(self.cfg.vocab_size, tuple(self.cfg.eos_token_ids), "qwen3", ctx)
        return self

    # -- src/api.rs:92-108
    def prefill(self, tokens: Sequence[int]) -> Logits:
        ids = np.ascontiguousarray(np.asarray(tokens, dtype=np.int64), dtype=np.uint32)
        if ids.ndim != 1 or ids.size == 0:
            raise ValueError("prefill requires at least one token")
        out = np.empty(self.cfg.vocab_size, np.float32)
        call("grout_engine_prefill", self._h, ids.ctypes.data_as(C.c_void_p), ids.size,
             out.ctypes.data_as(C.c_void_p), None)
        return Logits(out)

    def prefill_greedy(self, tokens: Sequence[int]) -> int:
        """Prefill and return the greedy next token (device argmax only)."""
        ids = np.ascontiguousarray(np.asarray(tokens, dtype=np.int64), dtype=np.uint32)
        if ids.ndim != 1 or ids.size == 0:
            raise ValueError("prefill requires at least one token")
        tok = C.c_uint32()
        call("grout_engine_prefill", self._h, ids.ctypes.data_as(C.c_void_p), ids.size, None,
             C.byref(tok))
        return int(tok.value)

    def extend(self, tokens: Sequence[int]) -> Logits:
        """Chunked prefill: runs `tokens` at the session's next positions
        (grout_engine_extend) and returns the last one's logits."""
        ids = np.ascontiguousarray(np.asarray(tokens, dtype=np.int64), dtype=np.uint32)
        if ids.ndim != 1 or ids.size == 0:
            raise ValueError("extend requires at least one token")
        out = np.empty(self.cfg.vocab_size, np.float32)
        call("grout_engine_extend", self._h, ids.ctypes.data_as(C.c_void_p), ids.size,
             out.ctypes.data_as(C.c_void_p), None)
        return Logits(out)

    # -- src/api.rs:110-121
    def decode(self, token: int) -> Logits:
        out = np.empty(self.cfg.vocab_size, np.float32)
        call("grout_engine_decode", self._h, int(token), out.ctypes.data_as(C.c_void_p))
        return Logits(out)

    # -- src/api.rs:123-137
    def decode_greedy(self, token: int) -> int:
        tok = C.c_uint32()
        call("grout_engine_decode_greedy", self._h, int(token), C.byref(tok))
        return int(tok.value)

    # -- src/api.rs:139-154
    def reset(self) -> None:
        call("grout_engine_reset", self._h)

    def meta(self) -> ModelMeta:
        return self._meta

    @property
    def position(self) -> int:
        return int(lib().grout_engine_position(self._h))

    @property
    def num_splits(self) -> int:
        """Decode attention split count (GROUT_FMHA_NUM_KV_SPLITS, else the
        library's default for max_ctx)."""
        return int(lib().grout_engine_num_splits(self._h))

    @property
    def uses_decode_graph(self) -> bool:
        """True when decode replays the captured decode-step graph."""
        return bool(lib().grout_engine_uses_decode_graph(self._h))

    @property
    def decode_graph_error(self) -> str:
        """Why decode runs the sequential fallback ("" with the graph);
        GenerationOutput::decode_graph_error (src/model.rs:1359)."""
        return (lib().grout_engine_decode_graph_error(self._h) or b"").decode()

    # -- src/api.rs:153-162
    def warmup(self) -> None:
        """One-token steps at positions 0 and 1 (prefill, then a decode-graph
        replay) with the model's first stop token, then an in-place reset."""
        call("grout_engine_warmup", self._h)

    def generate_greedy(self, prompt: Sequence[int], max_new_tokens: int) -> List[int]:
        """Prefill, then greedy decode: returns the max_new_tokens generated ids."""
        out = [self.prefill_greedy(prompt)]
        while len(out) < max_new_tokens:
            out.append(self.decode_greedy(out[-1]))
        return out[:max_new_tokens]

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            lib().grout_engine_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
