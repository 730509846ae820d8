"""ctypes/numpy wrapper over oracle/_build/libgrout_oracle.so (test infrastructure only)."""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import threading

import numpy as np

__all__ = [
    "lib", "build", "h2f", "f2h", "fill_normal_f16", "fill_uniform_f16", "fill_normal_f64",
    "splitmix64_at", "inv_freq", "rope_table", "rope_rows", "rsqrt_det", "sumsq_row128",
    "qk_norm_rope_row", "qk_norm_rope_kv_prefill", "qk_norm_rope_kv_decode",
    "attention_prefill_rows", "attention_decode", "decode_split", "splitk_merge",
    "Q8_0", "Q4_K", "Q5_K", "Q6_K", "qblock", "dequant", "gemv_q",
    "SEED_BASE", "seed_for",
]

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "libgrout_oracle.so")
_lock = threading.Lock()
_lib = None

# Per-tensor seeds: SEED_BASE ^ tag (tags are small ASCII words packed in a u64).
SEED_BASE = 0x4752_4F55_5441_5454  # "GROUTATT"


def seed_for(tag: str, base: int = SEED_BASE) -> int:
    t = int.from_bytes(tag.encode()[:8].ljust(8, b"\0"), "little")
    return (base ^ t) & 0xFFFF_FFFF_FFFF_FFFF


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, -O2, no fast-math, no contraction)."""
    srcs = ("grout_oracle.c", "ggml_quant.c", "Makefile")
    if force or not os.path.exists(_SO) or any(
        os.path.getmtime(_SO) < os.path.getmtime(os.path.join(_HERE, f)) for f in srcs
    ):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_sz, _i, _l, _f, _d, _u64 = C.c_size_t, C.c_int, C.c_long, C.c_float, C.c_double, C.c_uint64

_SIGS = {
    "go_h2f_array": (None, [_u16p, _f32p, _sz]),
    "go_f2h_array": (None, [_f32p, _u16p, _sz]),
    "go_splitmix64_at": (_u64, [_u64, _u64]),
    "go_fill_normal_f16": (None, [_u64, _sz, _u16p]),
    "go_fill_normal_f64": (None, [_u64, _sz, _f64p]),
    "go_fill_uniform_f16": (None, [_u64, _d, _d, _sz, _u16p]),
    "go_inv_freq": (None, [_i, _f, _f32p]),
    "go_rope_table": (None, [_i, _i, _f, _f32p, _f32p]),
    "go_rope_rows": (None, [_i, _i, _i, _f, _f32p, _f32p]),
    "go_rsqrt_det": (_f, [_f]),
    "go_sumsq_row128": (_f, [_u16p]),
    "go_qk_norm_rope_row": (None, [_u16p, _u16p, _f32p, _f32p, _f, _u16p]),
    "go_qk_norm_rope_kv_prefill": (None, [_u16p, _u16p, _u16p, _u16p, _u16p, _f32p, _f32p, _u16p,
                                          _u16p, _u16p, _i, _i, _i, _i, _i, _l, _f]),
    "go_qk_norm_rope_kv_decode": (None, [_u16p, _u16p, _u16p, _f32p, _f32p, _u16p, _u16p, _u16p,
                                         _i, _i, _i, _i, _l, _f]),
    "go_attention_prefill_rows": (None, [_u16p, _u16p, _u16p, _f32p, _i32p, _i, _i, _i, _i, _i,
                                         _i, _l, _f, _i]),
    "go_attention_decode": (None, [_u16p, _u16p, _u16p, _f32p, _i, _i, _i, _i, _l, _f, _i]),
    "go_decode_split": (None, [_u16p, _u16p, _u16p, _f32p, _f32p, _i, _i, _i, _i, _l, _f, _i,
                               _i]),
    "go_splitk_merge": (None, [_f32p, _f32p, _f32p, _i, _i, _i, _i]),
    "go_qblock_bytes": (_i, [_i]),
    "go_qblock_elems": (_i, [_i]),
    "go_dequant": (_i, [_i, _u8p, _sz, _f32p]),
    "go_dequant_decode": (_i, [_i, _u8p, _sz, _f32p]),
    "go_gemv_q": (_i, [_i, _u8p, _i, _i, _u16p, _f64p]),
}


def lib():
    global _lib
    with _lock:
        if _lib is None:
            build()
            L = C.CDLL(_SO)
            for name, (res, args) in _SIGS.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def h2f(h) -> np.ndarray:
    h = _u16(h)
    out = np.empty(h.shape, np.float32)
    lib().go_h2f_array(h.reshape(-1), out.reshape(-1), h.size)
    return out


def f2h(f) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().go_f2h_array(f.reshape(-1), out.reshape(-1), f.size)
    return out


def splitmix64_at(seed: int, k: int) -> int:
    return int(lib().go_splitmix64_at(seed, k))


def fill_normal_f16(seed: int, shape) -> np.ndarray:
    out = np.empty(shape, np.uint16)
    lib().go_fill_normal_f16(seed, out.size, out.reshape(-1))
    return out


def fill_normal_f64(seed: int, shape) -> np.ndarray:
    out = np.empty(shape, np.float64)
    lib().go_fill_normal_f64(seed, out.size, out.reshape(-1))
    return out


def fill_uniform_f16(seed: int, lo: float, hi: float, shape) -> np.ndarray:
    out = np.empty(shape, np.uint16)
    lib().go_fill_uniform_f16(seed, lo, hi, out.size, out.reshape(-1))
    return out


def inv_freq(D: int, theta: float) -> np.ndarray:
    out = np.empty(D // 2, np.float32)
    lib().go_inv_freq(D, theta, out)
    return out


def rope_table(max_ctx: int, D: int, theta: float):
    c = np.empty((max_ctx, D // 2), np.float32)
    s = np.empty((max_ctx, D // 2), np.float32)
    lib().go_rope_table(max_ctx, D, theta, c, s)
    return c, s


def rope_rows(p0: int, n: int, D: int, theta: float):
    """Rows p0 .. p0+n-1 of rope_table (for caches too long to tabulate whole)."""
    c = np.empty((n, D // 2), np.float32)
    s = np.empty((n, D // 2), np.float32)
    lib().go_rope_rows(p0, n, D, theta, c, s)
    return c, s


def rsqrt_det(v: float) -> float:
    return float(lib().go_rsqrt_det(v))


def sumsq_row128(x) -> float:
    return float(lib().go_sumsq_row128(_u16(x)))


def qk_norm_rope_row(x, gamma, cos_row, sin_row, eps: float) -> np.ndarray:
    out = np.empty(128, np.uint16)
    lib().go_qk_norm_rope_row(_u16(x), _u16(gamma), np.ascontiguousarray(cos_row, np.float32),
                              np.ascontiguousarray(sin_row, np.float32), eps, out)
    return out


def qk_norm_rope_kv_prefill(q, k, v, gamma_q, gamma_k, cos_t, sin_t, k_cache, v_cache, pos0: int,
                            eps: float):
    """q [S,Hq,D], k/v [S,Hkv,D] f16 bits; caches [Hkv,max_ctx,D] updated in place.
    Returns q_out [S,Hq,D]."""
    S, Hq, D = q.shape
    Hkv = k.shape[1]
    q_out = np.empty_like(_u16(q))
    lib().go_qk_norm_rope_kv_prefill(_u16(q), _u16(k), _u16(v), _u16(gamma_q), _u16(gamma_k),
                                     cos_t, sin_t, q_out, k_cache, v_cache, pos0, S, Hq, Hkv, D,
                                     k_cache.shape[1] * D, eps)
    return q_out


def qk_norm_rope_kv_decode(qkv, gamma_q, gamma_k, cos_t, sin_t, k_cache, v_cache, pos: int,
                           Hq: int, Hkv: int, eps: float):
    D = k_cache.shape[2]
    q_out = np.empty((Hq, D), np.uint16)
    lib().go_qk_norm_rope_kv_decode(_u16(qkv), _u16(gamma_q), _u16(gamma_k), cos_t, sin_t, q_out,
                                    k_cache, v_cache, pos, Hq, Hkv, D, k_cache.shape[1] * D, eps)
    return q_out


def attention_prefill_rows(q, k_cache, v_cache, pos0: int, rows=None, scale=None,
                           nthreads: int = 1) -> np.ndarray:
    """q [S,Hq,D] f16 bits, caches [Hkv,max_ctx,D]; returns fp32 [len(rows),Hq,D]."""
    S, Hq, D = q.shape
    Hkv = k_cache.shape[0]
    rows = np.arange(S, dtype=np.int32) if rows is None else np.ascontiguousarray(rows, np.int32)
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    out = np.empty((len(rows), Hq, D), np.float32)
    lib().go_attention_prefill_rows(_u16(q), _u16(k_cache), _u16(v_cache), out, rows, len(rows),
                                    S, pos0, Hq, Hkv, D, k_cache.shape[1] * D, scale, nthreads)
    return out


def attention_decode(q, k_cache, v_cache, pos: int, scale=None, nthreads: int = 1) -> np.ndarray:
    """q [Hq,D] f16 bits; attends to cache positions 0..pos; returns fp32 [Hq,D]."""
    Hq, D = q.shape
    Hkv = k_cache.shape[0]
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    out = np.empty((Hq, D), np.float32)
    lib().go_attention_decode(_u16(q), _u16(k_cache), _u16(v_cache), out, pos, Hq, Hkv, D,
                              k_cache.shape[1] * D, scale, nthreads)
    return out


def decode_split(q, k_cache, v_cache, pos: int, BN: int, NKS: int, scale=None):
    Hq, D = q.shape
    Hkv = k_cache.shape[0]
    G = Hq // Hkv
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    att = np.empty((Hkv, NKS * G, D), np.float32)
    lse = np.empty((Hkv, NKS * G), np.float32)
    lib().go_decode_split(_u16(q), _u16(k_cache), _u16(v_cache), att, lse, pos, Hq, Hkv, D,
                          k_cache.shape[1] * D, scale, BN, NKS)
    return att, lse


Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14  # ggml type ids


def qblock(fmt: int):
    """(weights per block, bytes per block) of a ggml quantized format."""
    return int(lib().go_qblock_elems(fmt)), int(lib().go_qblock_bytes(fmt))


def dequant(fmt: int, blocks, n: int, decode: bool = False) -> np.ndarray:
    """ggml blocks (uint8) -> n fp32 weights: the CPU rule
    (src/dequant.rs:211-323), or with decode=True the reference's GPU decode
    layout, whose Q4_K scale and min are folded and rounded to f16
    (src/loader.rs:437-486)."""
    out = np.empty(n, np.float32)
    fn = lib().go_dequant_decode if decode else lib().go_dequant
    rc = fn(fmt, np.ascontiguousarray(blocks, np.uint8).reshape(-1), n, out)
    if rc != 0:
        raise ValueError(f"dequant of format {fmt} with {n} weights failed")
    return out


def gemv_q(fmt: int, blocks, N: int, K: int, x) -> np.ndarray:
    """y = W x in fp64 for rows of ggml blocks, W the decode-layout weights
    (the reference's decode GEMVs, src/kernels.rs:565-803)."""
    y = np.empty(N, np.float64)
    rc = lib().go_gemv_q(fmt, np.ascontiguousarray(blocks, np.uint8).reshape(-1), N, K, _u16(x), y)
    if rc != 0:
        raise ValueError("gemv_q failed")
    return y


def splitk_merge(att, lse, Hq: int) -> np.ndarray:
    Hkv, nsg, D = att.shape
    NKS = nsg // (Hq // Hkv)
    out = np.empty((Hq, D), np.float32)
    lib().go_splitk_merge(np.ascontiguousarray(att, np.float32),
                          np.ascontiguousarray(lse, np.float32), out, Hq, Hkv, D, NKS)
    return out
