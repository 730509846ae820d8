"""ctypes binding of grout_amd/libgrout_attn.so (the C ABI in include/grout_attn.h).

The library is the only compute path: if it is missing this module raises, it
never falls back to PyTorch or CPU code.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgrout_attn.so")
_lock = threading.Lock()
_lib = None


class GroutError(RuntimeError):
    """A C ABI call returned a non-zero status (message from grout_last_error)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


_p, _i, _l, _f, _sz, _u32 = C.c_void_p, C.c_int, C.c_long, C.c_float, C.c_size_t, C.c_uint32


class DecodeLayer(C.Structure):
    _fields_ = [("qkv", _p), ("gamma_q", _p), ("gamma_k", _p), ("q_rope", _p),
                ("k_cache", _p), ("v_cache", _p), ("attn_out", _p)]


class Qwen3Config(C.Structure):
    _fields_ = [("num_layers", _i), ("hidden_size", _i), ("intermediate_size", _i),
                ("num_q_heads", _i), ("num_kv_heads", _i), ("head_dim", _i), ("vocab_size", _i),
                ("rms_norm_eps", _f), ("rope_theta", _f), ("max_ctx", _i)]


class Qwen3Layer(C.Structure):
    _fields_ = [("input_layernorm", _p), ("qkv_proj", _p), ("q_norm", _p), ("k_norm", _p),
                ("o_proj", _p), ("post_attention_layernorm", _p), ("gate_up_proj", _p),
                ("down_proj", _p)]


class Qwen3Weights(C.Structure):
    _fields_ = [("embed_tokens", _p), ("norm", _p), ("lm_head", _p),
                ("layers", C.POINTER(Qwen3Layer))]


class WPart(C.Structure):
    _fields_ = [("fmt", _i), ("rows", _i), ("data", _p)]


class Qwen3QLayer(C.Structure):
    _fields_ = [("input_layernorm", _p), ("num_qkv_parts", _i), ("qkv", WPart * 3),
                ("q_norm", _p), ("k_norm", _p), ("o_proj", WPart),
                ("post_attention_layernorm", _p), ("num_gate_up_parts", _i),
                ("gate_up", WPart * 2), ("down_proj", WPart)]


class Qwen3QWeights(C.Structure):
    _fields_ = [("embed_tokens", WPart), ("norm", _p), ("lm_head", WPart),
                ("layers", C.POINTER(Qwen3QLayer))]


class ModelInfo(C.Structure):
    _fields_ = [("config", Qwen3Config), ("tie_word_embeddings", _i), ("num_eos", _i),
                ("eos_token_ids", _u32 * 8), ("weight_bytes", _sz)]


# name -> (restype, argtypes).  Every symbol declared in include/*.h.
SIGNATURES = {
    "grout_last_error": (C.c_char_p, []),
    "grout_abi_version": (_i, []),
    "grout_rope_inv_freq": (_i, [_i, _f, _p]),
    "grout_rope_table_host": (_i, [_i, _i, _f, _p, _p]),
    "grout_qk_norm_rope_kv_prefill": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i,
                                           _i, _i, _l, _f, _p]),
    "grout_qk_norm_rope_kv_decode": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _l,
                                          _f, _p]),
    "grout_fmha_prefill": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _l, _f, _p]),
    "grout_attn_decode_default_splits": (_i, [_i, _i, _i]),
    "grout_fmha_prefill_plan": (_i, [_i, _i, _i, _p, _p, _p]),
    "grout_attn_decode_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "grout_attn_decode": (_i, [_p, _p, _p, _p, _p, _sz, _p, _i, _i, _i, _i, _l, _i, _f, _p]),
    "grout_attn_decode_noalloc": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _l, _i, _f, _p]),
    "grout_fmha_decode_gqa_split": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _l, _i, _f, _p]),
    "grout_splitk_reduce_merge": (_i, [_p, _p, _p, _i, _i, _i, _i, _p]),
    "grout_attn_decode_fused": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p, _i, _i, _i, _i,
                                     _l, _i, _f, _f, _p]),
    "grout_decode_graph_create": (_i, [C.POINTER(DecodeLayer), _i, _p, _p, _p, _sz, _i, _i, _i,
                                       _i, _i, _f, _f, _p, C.POINTER(_p)]),
    "grout_decode_graph_launch": (_i, [_p, _u32, _p]),
    "grout_decode_graph_position_ptr": (_p, [_p]),
    "grout_decode_graph_destroy": (_i, [_p]),
    "grout_diag_mfma_layout": (_i, [_p, _p]),
    # include/grout_engine.h
    "grout_embedding": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "grout_rms_norm": (_i, [_p, _p, _p, _i, _i, _f, _p]),
    "grout_add_rms_norm": (_i, [_p, _p, _p, _p, _p, _i, _i, _f, _p]),
    "grout_silu_mul": (_i, [_p, _p, _i, _i, _p]),
    "grout_gemv": (_i, [_p, _p, _p, _i, _i, _p]),
    "grout_gemv_rms_norm": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _f, _p]),
    "grout_gemv_rms_norm_silu_mul": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _f, _p]),
    "grout_qweight_bytes": (_sz, [_i, _i, _i]),
    "grout_qweight_repack": (_i, [_i, _p, _i, _i, _p, _p]),
    "grout_gemv_q": (_i, [_i, _p, _p, _p, _i, _i, _p]),
    "grout_gemv_q_silu_mul": (_i, [_i, _p, _p, _p, _i, _i, _p]),
    "grout_qweight_dequant": (_i, [_i, _p, _i, _i, _p, _p]),
    "grout_qweight_gather": (_i, [_i, _p, _i, _i, _p, _i, _p, _p]),
    "grout_gemv_q_rms_norm": (_i, [_i, _p, _p, _p, _p, _p, _p, _i, _i, _f, _p]),
    "grout_gemv_q_rms_norm_silu_mul": (_i, [_i, _p, _p, _p, _p, _p, _p, _i, _i, _f, _p]),
    "grout_argmax_workspace_bytes": (_sz, [_i]),
    "grout_argmax": (_i, [_p, _i, _p, _sz, _p, _p]),
    "grout_engine_create": (_i, [C.POINTER(Qwen3Config), C.POINTER(Qwen3Weights), _i,
                                 C.POINTER(_p)]),
    "grout_engine_create_q": (_i, [C.POINTER(Qwen3Config), C.POINTER(Qwen3QWeights), _i,
                                   C.POINTER(_p)]),
    "grout_model_inspect": (_i, [C.c_char_p, C.POINTER(ModelInfo)]),
    "grout_model_load": (_i, [C.c_char_p, _i, C.POINTER(_p)]),
    "grout_model_get_info": (_i, [_p, C.POINTER(ModelInfo)]),
    "grout_model_weights": (_i, [_p, C.POINTER(Qwen3Weights)]),
    "grout_model_qweights": (_i, [_p, C.POINTER(Qwen3QWeights)]),
    "grout_model_free": (_i, [_p]),
    "grout_engine_load": (_i, [C.c_char_p, _i, _i, C.POINTER(_p)]),
    "grout_engine_model_info": (_i, [_p, C.POINTER(ModelInfo)]),
    "grout_engine_prefill": (_i, [_p, _p, _i, _p, _p]),
    "grout_engine_extend": (_i, [_p, _p, _i, _p, _p]),
    "grout_engine_decode": (_i, [_p, _u32, _p]),
    "grout_engine_decode_greedy": (_i, [_p, _u32, _p]),
    "grout_engine_reset": (_i, [_p]),
    "grout_engine_warmup": (_i, [_p]),
    "grout_engine_position": (_i, [_p]),
    "grout_env_flag": (_i, [C.c_char_p, _i]),
    "grout_env_usize": (C.c_long, [C.c_char_p, C.c_long]),
    "grout_engine_num_splits": (_i, [_p]),
    "grout_engine_vram_preflight": (_i, [C.POINTER(Qwen3Config), _sz, _sz, _sz, _sz,
                                         C.POINTER(_sz)]),
    "grout_engine_uses_decode_graph": (_i, [_p]),
    "grout_engine_decode_graph_error": (C.c_char_p, [_p]),
    "grout_engine_destroy": (_i, [_p]),
}


def lib():
    """Load the HIP library (raises if it has not been built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the gfx950 HIP library with "
                    "`python -m grout_amd.build` (there is no fallback path)")
            L = C.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def last_error() -> str:
    return lib().grout_last_error().decode()


def call(name: str, *args) -> int:
    """Call a status-returning ABI function; raise GroutError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise GroutError(name, rc, last_error())
    return rc
