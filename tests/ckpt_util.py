"""Writes Qwen3-style checkpoint directories (HF tensor names, safetensors
files written byte by byte, so any dtype including bf16 can be stored) for
the loader tests."""
import json
import os
import struct

import numpy as np

from oracle import qwen3 as Q

DT_SIZE = {"F16": 2, "BF16": 2, "F32": 4, "F64": 8, "I8": 1}


def write_safetensors(path, tensors):
    """tensors: {name: (dtype, shape, raw_bytes)}."""
    header, blobs, off = {}, [], 0
    for name, (dtype, shape, raw) in tensors.items():
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    header["__metadata__"] = {"format": "pt"}
    hb = json.dumps(header).encode()
    hb += b" " * (-len(hb) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for b in blobs:
            f.write(b)


def encode(values_f64, dtype):
    """(raw bytes in dtype, the f16 bits the loader must produce)."""
    v = np.asarray(values_f64, np.float64)
    if dtype == "F16":
        h = v.astype(np.float16)
        return h.tobytes(), h.view(np.uint16)
    if dtype == "F32":
        f = v.astype(np.float32)
        return f.tobytes(), f.astype(np.float16).view(np.uint16)
    if dtype == "F64":
        return v.tobytes(), v.astype(np.float32).astype(np.float16).view(np.uint16)
    if dtype == "BF16":
        bits = v.astype(np.float32).view(np.uint32)
        # round to nearest even into the upper 16 bits
        bf = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
        f32 = (bf.astype(np.uint32) << 16).view(np.float32)
        return bf.tobytes(), f32.astype(np.float16).view(np.uint16)
    raise ValueError(dtype)


def config_json(cfg, max_pos=4096, **over):
    d = {"architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3",
         "vocab_size": cfg.vocab_size, "hidden_size": cfg.hidden_size,
         "intermediate_size": cfg.intermediate_size, "num_hidden_layers": cfg.num_layers,
         "num_attention_heads": cfg.num_attention_heads,
         "num_key_value_heads": cfg.num_key_value_heads, "head_dim": cfg.head_dim,
         "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta,
         "max_position_embeddings": max_pos, "tie_word_embeddings": cfg.tie_word_embeddings,
         "use_sliding_window": False, "sliding_window": None, "rope_scaling": None,
         "eos_token_id": 151645, "torch_dtype": "bfloat16"}
    d.update(over)
    return d


def write_checkpoint(dirpath, cfg, seed=0, dtypes=("BF16",), shards=2, std=0.05, max_pos=4096,
                     config_over=None, drop=(), reshape=None, generation_eos=None):
    """Random Qwen3 weights under HF names.  Tensor i is stored in
    dtypes[i % len(dtypes)].  Returns the host weights in the engine's fused
    layout (fp16 bits) exactly as the loader must produce them."""
    os.makedirs(dirpath, exist_ok=True)
    rng = np.random.default_rng(seed)
    H, I = cfg.hidden_size, cfg.intermediate_size
    qd, kd = cfg.q_dim, cfg.kv_dim
    names = {"model.embed_tokens.weight": (cfg.vocab_size, H), "model.norm.weight": (H,)}
    if not cfg.tie_word_embeddings:
        names["lm_head.weight"] = (cfg.vocab_size, H)
    per_layer = {"input_layernorm.weight": (H,), "post_attention_layernorm.weight": (H,),
                 "self_attn.q_norm.weight": (128,), "self_attn.k_norm.weight": (128,),
                 "self_attn.q_proj.weight": (qd, H), "self_attn.k_proj.weight": (kd, H),
                 "self_attn.v_proj.weight": (kd, H), "self_attn.o_proj.weight": (H, qd),
                 "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
                 "mlp.down_proj.weight": (H, I)}
    for l in range(cfg.num_layers):
        for k, shp in per_layer.items():
            names[f"model.layers.{l}.{k}"] = shp
    raw, f16 = {}, {}
    for i, (name, shp) in enumerate(names.items()):
        dt = dtypes[i % len(dtypes)]
        vals = (rng.uniform(0.8, 1.2, shp) if len(shp) == 1 else rng.standard_normal(shp) * std)
        if reshape and name in reshape:  # store a tensor of the wrong shape
            shp = reshape[name]
            vals = np.zeros(shp)
        b, bits = encode(vals, dt)
        if name not in drop:
            raw[name] = (dt, shp, b)
        f16[name] = bits.reshape(shp)
    items = list(raw.items())
    if shards == 1:
        write_safetensors(os.path.join(dirpath, "model.safetensors"), dict(items))
    else:
        wm = {}
        per = (len(items) + shards - 1) // shards
        for s in range(shards):
            fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            part = dict(items[s * per:(s + 1) * per])
            write_safetensors(os.path.join(dirpath, fn), part)
            wm.update({k: fn for k in part})
        with open(os.path.join(dirpath, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {"total_size": 0}, "weight_map": wm}, f)
    cj = config_json(cfg, max_pos, **(config_over or {}))
    with open(os.path.join(dirpath, "config.json"), "w") as f:
        json.dump(cj, f)
    if generation_eos is not None:
        with open(os.path.join(dirpath, "generation_config.json"), "w") as f:
            json.dump({"eos_token_id": generation_eos, "do_sample": True}, f)
    # fused host layout for the oracle
    layers = []
    for l in range(cfg.num_layers):
        g = lambda k: f16[f"model.layers.{l}.{k}"]
        layers.append({
            "input_layernorm": g("input_layernorm.weight"),
            "qkv_proj": np.concatenate([g("self_attn.q_proj.weight"), g("self_attn.k_proj.weight"),
                                        g("self_attn.v_proj.weight")]),
            "q_norm": g("self_attn.q_norm.weight"), "k_norm": g("self_attn.k_norm.weight"),
            "o_proj": g("self_attn.o_proj.weight"),
            "post_attention_layernorm": g("post_attention_layernorm.weight"),
            "gate_up_proj": np.concatenate([g("mlp.gate_proj.weight"), g("mlp.up_proj.weight")]),
            "down_proj": g("mlp.down_proj.weight")})
    return {"embed_tokens": f16["model.embed_tokens.weight"], "norm": f16["model.norm.weight"],
            "layers": layers,
            "lm_head": None if cfg.tie_word_embeddings else f16["lm_head.weight"]}
