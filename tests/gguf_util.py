"""Writes GGUF files for the tests, from the container's published layout:
header (magic "GGUF", version, tensor count, metadata count), typed metadata
key/values, tensor infos (name, dimensions innermost first, ggml type, data
offset) and the tensor data, each tensor aligned to general.alignment."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
T_F32, T_F16, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K, T_BF16 = 0, 1, 8, 12, 13, 14, 30

_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}


def gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def gval(t: int, v) -> bytes:
    if t == STRING:
        return gstr(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(gval(et, x) for x in items)
    return struct.pack(_SCALAR[t], v)


def gguf_bytes(meta, tensors, version=3, alignment=32) -> bytes:
    """meta: [(key, type, value)]; tensors: [(name, ggml type, shape outermost
    first, raw bytes)]."""
    out = bytearray(struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(meta)))
    for k, t, v in meta:
        out += gstr(k) + struct.pack("<I", t) + gval(t, v)
    offs, off = [], 0
    for name, t, shape, raw in tensors:
        out += gstr(name) + struct.pack("<I", len(shape))
        out += b"".join(struct.pack("<Q", d) for d in reversed(shape))
        out += struct.pack("<IQ", t, off)
        offs.append(off)
        off += (len(raw) + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    for (_, _, _, raw), o in zip(tensors, offs):
        out += raw + b"\0" * ((-len(raw)) % alignment)
    return bytes(out)


def qwen3_meta(cfg, eos=7, ctx=4096, extra=()):
    return [("general.architecture", STRING, "qwen3"),
            ("qwen3.block_count", U32, cfg.num_layers),
            ("qwen3.embedding_length", U32, cfg.hidden_size),
            ("qwen3.feed_forward_length", U32, cfg.intermediate_size),
            ("qwen3.attention.head_count", U32, cfg.num_attention_heads),
            ("qwen3.attention.head_count_kv", U32, cfg.num_key_value_heads),
            ("qwen3.attention.key_length", U32, 128),
            ("qwen3.rope.freq_base", F32, cfg.rope_theta),
            ("qwen3.attention.layer_norm_rms_epsilon", F32, cfg.rms_norm_eps),
            ("qwen3.context_length", U32, ctx),
            ("tokenizer.ggml.eos_token_id", U32, eos),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, ["<a>", "<b>", "<c>"])),
            *extra]


_GGUF_NAMES = {"input_layernorm": "attn_norm", "post_attention_layernorm": "ffn_norm",
               "q_norm": "attn_q_norm", "k_norm": "attn_k_norm", "q_proj": "attn_q",
               "k_proj": "attn_k", "v_proj": "attn_v", "o_proj": "attn_output",
               "gate_proj": "ffn_gate", "up_proj": "ffn_up", "down_proj": "ffn_down"}


def _mat(name, m, rows, k):
    fmt, data = m
    raw = np.ascontiguousarray(data).tobytes()
    return (name, T_F16 if fmt == 0 else fmt, (rows, k), raw)


def _vec(name, bits):
    """fp16 bit patterns stored as F32 (exact), as GGUF files keep norms."""
    v = np.ascontiguousarray(bits).view(np.float16).astype(np.float32)
    return (name, T_F32, (v.size,), v.tobytes())


def qwen3_tensors(cfg, spec):
    """GGUF tensors from tests/qutil.py mixed_weights' QuantWeights arguments."""
    H, I, V, qd, kd = (cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.q_dim,
                       cfg.kv_dim)
    t = [_mat("token_embd.weight", spec["embed_tokens"], V, H),
         _vec("output_norm.weight", spec["norm"])]
    if spec["lm_head"] is not None:
        t.append(_mat("output.weight", spec["lm_head"], V, H))
    shapes = {"q_proj": (qd, H), "k_proj": (kd, H), "v_proj": (kd, H), "o_proj": (H, qd),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
    for l, L in enumerate(spec["layers"]):
        for key, g in _GGUF_NAMES.items():
            name = f"blk.{l}.{g}.weight"
            t.append(_mat(name, L[key], *shapes[key]) if key in shapes else _vec(name, L[key]))
    return t
