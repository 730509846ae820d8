"""Tensor-level operators of the attention hot path, over the C ABI.

Each function mirrors one reference operator (names, argument meaning and
error behaviour); torch tensors only carry device memory and the stream.
Shapes follow the reference: q [S, Hq, D], k/v [S, Hkv, D], caches
[Hkv, max_ctx, D] fp16, D = 128.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Tuple, Union

import torch

from ._lib import call, lib

HEAD_DIM = 128


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need(cond: bool, msg: str):
    if not cond:
        raise ValueError(msg)


def _f16(t: torch.Tensor, name: str, shape=None):
    _need(t.dtype == torch.float16, f"{name} must be float16, got {t.dtype}")
    _need(t.is_cuda, f"{name} must be a device tensor")
    _need(t.is_contiguous(), f"{name} must be contiguous")
    if shape is not None:
        _need(tuple(t.shape) == tuple(shape), f"{name} shape mismatch: {tuple(t.shape)} != {tuple(shape)}")


def inv_freq(head_dim: int = HEAD_DIM, theta: float = 1e6) -> torch.Tensor:
    """build_inv_freq (src/model.rs:7295-7306), on the host."""
    out = torch.empty(head_dim // 2, dtype=torch.float32)
    call("grout_rope_inv_freq", head_dim, theta, C.c_void_p(out.data_ptr()))
    return out


def rope_tables(max_ctx: int, head_dim: int = HEAD_DIM, theta: float = 1e6,
                device: Union[str, torch.device] = "cuda") -> Tuple[torch.Tensor, torch.Tensor]:
    """Host-built fp32 cos/sin tables [max_ctx, head_dim/2], uploaded to `device`."""
    c = torch.empty((max_ctx, head_dim // 2), dtype=torch.float32)
    s = torch.empty_like(c)
    call("grout_rope_table_host", max_ctx, head_dim, theta, C.c_void_p(c.data_ptr()),
         C.c_void_p(s.data_ptr()))
    return c.to(device), s.to(device)


def qk_norm_rope_kv_prefill(q, k, v, q_norm, k_norm, rope, k_cache, v_cache, position_start: int,
                            eps: float = 1e-6, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """GraphOp::QkNormRopeKvPrefill (src/model.rs:4753-4888): returns rotated q
    [S, Hq, D] and writes cache rows position_start .. position_start+S-1."""
    S, Hq, D = q.shape
    Hkv, max_ctx = k_cache.shape[0], k_cache.shape[1]
    _f16(q, "q")
    _f16(k, "k", (S, Hkv, D))
    _f16(v, "v", (S, Hkv, D))
    _f16(k_cache, "k_cache", (Hkv, max_ctx, D))
    _f16(v_cache, "v_cache", (Hkv, max_ctx, D))
    out = torch.empty_like(q) if out is None else out
    _f16(out, "out", (S, Hq, D))
    cos, sin = rope
    call("grout_qk_norm_rope_kv_prefill", _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm),
         _ptr(cos), _ptr(sin), _ptr(out), _ptr(k_cache), _ptr(v_cache), position_start, S, Hq,
         Hkv, D, max_ctx, max_ctx * D, eps, _stream(q.device))
    return out


def qk_norm_rope_kv_decode(qkv, q_norm, k_norm, rope, k_cache, v_cache, position: torch.Tensor,
                           num_q_heads: int, eps: float = 1e-6,
                           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """qk_norm_rope_kv_decode_raw_f16 (src/kernels.rs:5170-5452): qkv =
    [Q | K | V] flat, position = device u32 [1].  Returns rotated q [Hq, D]."""
    Hkv, max_ctx, D = k_cache.shape
    _f16(qkv, "qkv", ((num_q_heads + 2 * Hkv) * D,))
    _need(position.dtype in (torch.int32, torch.uint32) and position.numel() == 1 and position.is_cuda,
          "position must be a device [1] u32/i32 tensor")
    out = torch.empty((num_q_heads, D), dtype=torch.float16, device=qkv.device) if out is None else out
    cos, sin = rope
    call("grout_qk_norm_rope_kv_decode", _ptr(qkv), _ptr(q_norm), _ptr(k_norm), _ptr(cos),
         _ptr(sin), _ptr(out), _ptr(k_cache), _ptr(v_cache), _ptr(position), num_q_heads, Hkv, D,
         max_ctx, max_ctx * D, eps, _stream(qkv.device))
    return out


def fmha_prefill(q, k_cache, v_cache, position_start: int, out=None,
                 qk_scale: Optional[float] = None) -> torch.Tensor:
    """Causal GQA prefill (fmha_prefill_causal / _gqa_lpt, src/kernels.rs:2559-3298)."""
    S, Hq, D = q.shape
    Hkv = k_cache.shape[0]
    _f16(q, "q")
    _f16(k_cache, "k_cache")
    _f16(v_cache, "v_cache", tuple(k_cache.shape))
    out = torch.empty_like(q) if out is None else out
    _f16(out, "out", (S, Hq, D))
    qk_scale = 1.0 / math.sqrt(D) if qk_scale is None else qk_scale
    call("grout_fmha_prefill", _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), S,
         position_start, Hq, Hkv, D, k_cache.shape[1] * D, qk_scale, _stream(q.device))
    return out


PREFILL_FORMS = {0: "shared K/V stream, 256-row q blocks", 1: "per-team, 128-row q blocks",
                 2: "per-team, 64-row q blocks"}


def prefill_plan(seq_len: int, num_q_heads: int, num_kv_heads: int) -> dict:
    """The work split grout_fmha_prefill launches for these shapes (host only)."""
    import ctypes as C

    form, paired, wgs = C.c_int(), C.c_int(), C.c_long()
    call("grout_fmha_prefill_plan", seq_len, num_q_heads, num_kv_heads, C.byref(form),
         C.byref(paired), C.byref(wgs))
    return dict(form=form.value, name=PREFILL_FORMS[form.value], paired=bool(paired.value),
                workgroups=int(wgs.value))


def default_splits(ctx_len: int, num_q_heads: int, num_kv_heads: int) -> int:
    return int(lib().grout_attn_decode_default_splits(ctx_len, num_q_heads, num_kv_heads))


def decode_workspace(num_q_heads: int, num_kv_heads: int, num_splits: int, device) -> torch.Tensor:
    nbytes = int(lib().grout_attn_decode_workspace_bytes(num_q_heads, num_kv_heads, HEAD_DIM,
                                                         num_splits))
    _need(nbytes > 0, "invalid decode workspace request")
    return torch.empty(nbytes // 4, dtype=torch.float32, device=device)


def attn_decode(q, k_cache, v_cache, position: torch.Tensor, num_splits: Optional[int] = None,
                out=None, workspace=None, qk_scale: Optional[float] = None) -> torch.Tensor:
    """Split-K decode + LSE merge (fmha_decode_gqa_split + splitk_reduce_merge,
    src/kernels.rs:3996-4304).  q [Hq, D] (or [1, Hq, D]), position device [1]."""
    Hkv, max_ctx, D = k_cache.shape
    q2 = q.reshape(-1, D)
    Hq = q2.shape[0]
    _f16(q2, "q")
    _f16(k_cache, "k_cache")
    _f16(v_cache, "v_cache", tuple(k_cache.shape))
    ns = default_splits(max_ctx, Hq, Hkv) if not num_splits else num_splits
    ws = decode_workspace(Hq, Hkv, ns, q.device) if workspace is None else workspace
    out = torch.empty((Hq, D), dtype=torch.float16, device=q.device) if out is None else out
    qk_scale = 1.0 / math.sqrt(D) if qk_scale is None else qk_scale
    call("grout_attn_decode", _ptr(q2), _ptr(k_cache), _ptr(v_cache), _ptr(out), _ptr(ws),
         ws.numel() * ws.element_size(), _ptr(position), Hq, Hkv, D, max_ctx, max_ctx * D, ns,
         qk_scale, _stream(q.device))
    return out.view(q.shape)


def attn_decode_fused(qkv, q_norm, k_norm, rope, k_cache, v_cache, position: torch.Tensor,
                      num_q_heads: int, num_splits: Optional[int] = None, out=None,
                      workspace=None, eps: float = 1e-6,
                      qk_scale: Optional[float] = None) -> torch.Tensor:
    """One layer's decode attention from the raw QKV projection: QK-RMSNorm +
    RoPE + K/V cache write at `position`, then split-K attention (one launch
    for num_splits == 1).  qkv [(Hq+2Hkv)*D]; returns out [Hq, D]."""
    Hkv, max_ctx, D = k_cache.shape
    Hq = num_q_heads
    _f16(qkv, "qkv", ((Hq + 2 * Hkv) * D,))
    _f16(k_cache, "k_cache")
    _f16(v_cache, "v_cache", tuple(k_cache.shape))
    cos, sin = rope
    _need(cos.shape[0] >= max_ctx, "rope tables shorter than the cache")
    ns = default_splits(max_ctx, Hq, Hkv) if not num_splits else num_splits
    if workspace is None and ns > 1:
        workspace = decode_workspace(Hq, Hkv, ns, qkv.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    out = torch.empty((Hq, D), dtype=torch.float16, device=qkv.device) if out is None else out
    qk_scale = 1.0 / math.sqrt(D) if qk_scale is None else qk_scale
    call("grout_attn_decode_fused", _ptr(qkv), _ptr(q_norm), _ptr(k_norm), _ptr(cos), _ptr(sin),
         _ptr(k_cache), _ptr(v_cache), _ptr(out), _ptr(workspace), ws_bytes, _ptr(position), Hq,
         Hkv, D, max_ctx, max_ctx * D, ns, eps, qk_scale, _stream(qkv.device))
    return out


def fmha_decode_gqa_split(q, k_cache, v_cache, position, num_splits: int,
                          qk_scale: Optional[float] = None):
    """The split pass alone: returns (part_acc [Hkv, splits, G, D], part_ml [Hkv, splits, G, 2])."""
    Hkv, max_ctx, D = k_cache.shape
    q2 = q.reshape(-1, D)
    Hq = q2.shape[0]
    G = Hq // Hkv
    acc = torch.empty((Hkv, num_splits, G, D), dtype=torch.float32, device=q.device)
    ml = torch.empty((Hkv, num_splits, G, 2), dtype=torch.float32, device=q.device)
    qk_scale = 1.0 / math.sqrt(D) if qk_scale is None else qk_scale
    call("grout_fmha_decode_gqa_split", _ptr(q2), _ptr(k_cache), _ptr(v_cache), _ptr(acc),
         _ptr(ml), _ptr(position), Hq, Hkv, D, max_ctx, max_ctx * D, num_splits, qk_scale,
         _stream(q.device))
    return acc, ml


def splitk_reduce_merge(part_acc, part_ml, out=None) -> torch.Tensor:
    Hkv, ns, G, D = part_acc.shape
    out = torch.empty((Hkv * G, D), dtype=torch.float16, device=part_acc.device) if out is None else out
    call("grout_splitk_reduce_merge", _ptr(part_acc), _ptr(part_ml), _ptr(out), Hkv * G, Hkv, D,
         ns, _stream(part_acc.device))
    return out


def attention(q, k_cache, v_cache, position: Union[int, torch.Tensor], out=None,
              num_splits: Optional[int] = None) -> torch.Tensor:
    """GraphOp::Attention dispatch (attend_seq_arc_into_ctx_with_position,
    src/model.rs:6856-7182): a host position runs the causal prefill kernel
    (any q_len, kv_len = position + q_len); a device position is the decode
    graph path and requires q_len == 1."""
    _need(q.dim() == 3, f"q must be rank 3 [seqlen, heads, head_dim], got {tuple(q.shape)}")
    if isinstance(position, torch.Tensor):
        _need(q.shape[0] == 1, f"decode graph path expects q_len=1, got {q.shape[0]}")
        _need(position.numel() == 1, "attention position tensor must be shape [1]")
        return attn_decode(q, k_cache, v_cache, position, num_splits=num_splits, out=out)
    return fmha_prefill(q, k_cache, v_cache, int(position), out=out)


def diag_mfma_layout(device="cuda") -> torch.Tensor:
    out = torch.empty((64, 4), dtype=torch.float32, device=device)
    call("grout_diag_mfma_layout", _ptr(out), _stream(out.device))
    return out
