"""CPU checks of the checkpoint loader (grout_model_inspect: config.json,
generation_config.json, the shard index and every safetensors header are
parsed and validated on the host; no GPU needed)."""
import json
import os
import struct

import pytest

from ckpt_util import write_checkpoint, write_safetensors
from grout_amd import model as M
from grout_amd._lib import GroutError

TINY = M.Qwen3Config(num_layers=2, hidden_size=64, intermediate_size=96,
                     num_attention_heads=2, num_key_value_heads=1, vocab_size=50)


def test_inspect_reads_config_and_sizes(tmp_path):
    write_checkpoint(tmp_path, TINY, dtypes=("BF16", "F32", "F16", "F64"), shards=3,
                     generation_eos=[151645, 151643])
    r = M.inspect(tmp_path)
    cfg = r["config"]
    assert (cfg.num_layers, cfg.hidden_size, cfg.intermediate_size) == (2, 64, 96)
    assert (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.vocab_size) == (2, 1, 50)
    assert cfg.tie_word_embeddings and r["max_position_embeddings"] == 4096
    assert cfg.eos_token_ids == (151645, 151643)
    assert abs(cfg.rms_norm_eps - 1e-6) < 1e-12 and cfg.rope_theta == 1e6
    # fp16 bytes of the fused layout, each piece rounded up to 256 bytes
    assert r["weight_bytes"] >= 2 * TINY.num_params()


def test_single_file_untied_checkpoint(tmp_path):
    cfg = M.Qwen3Config(**{**TINY.__dict__, "tie_word_embeddings": False})
    write_checkpoint(tmp_path, cfg, shards=1)
    r = M.inspect(tmp_path)
    assert not r["config"].tie_word_embeddings
    assert r["config"].eos_token_ids == (151645,)


@pytest.mark.parametrize("kind,match", [
    ("missing_tensor", "missing tensor model.layers.1.mlp.up_proj.weight"),
    ("wrong_shape", "has shape"),
    ("sliding_window", "use_sliding_window"),
    ("head_dim", "head_dim=64"),
    ("kv_heads", "not divisible"),
    ("missing_field", "rope_theta"),
    ("nan_eps", "rms_norm_eps"),
    ("range", "out of range"),
    ("bad_shard_name", "plain file name"),
    ("missing_lm_head", "missing tensor lm_head.weight"),
])
def test_inspect_rejects_bad_checkpoints(tmp_path, kind, match):
    over, drop, reshape, cfg = {}, (), None, TINY
    if kind == "missing_tensor":
        drop = ("model.layers.1.mlp.up_proj.weight",)
    elif kind == "wrong_shape":
        reshape = {"model.layers.0.self_attn.k_proj.weight": (64, 64)}
    elif kind == "sliding_window":
        over = {"use_sliding_window": True}
    elif kind == "head_dim":
        over = {"head_dim": 64}
    elif kind == "kv_heads":
        over = {"num_key_value_heads": 3}
    elif kind == "missing_field":
        over = {"rope_theta": None}
    elif kind == "nan_eps":
        over = {"rms_norm_eps": -1.0}
    elif kind == "range":
        over = {"num_hidden_layers": 0}
    elif kind == "missing_lm_head":
        over = {"tie_word_embeddings": False}
    write_checkpoint(tmp_path, cfg, config_over=over, drop=drop, reshape=reshape)
    if kind == "bad_shard_name":
        idx = os.path.join(tmp_path, "model.safetensors.index.json")
        d = json.load(open(idx))
        d["weight_map"]["model.norm.weight"] = "../model-00001-of-00002.safetensors"
        json.dump(d, open(idx, "w"))
    with pytest.raises(GroutError, match=match):
        M.inspect(tmp_path)


def test_inspect_rejects_corrupt_safetensors(tmp_path):
    write_checkpoint(tmp_path, TINY, shards=1)
    path = os.path.join(tmp_path, "model.safetensors")
    data = bytearray(open(path, "rb").read())
    # header length past the end of the file
    bad = bytearray(data)
    bad[:8] = struct.pack("<Q", len(data) * 2)
    open(path, "wb").write(bytes(bad))
    with pytest.raises(GroutError, match="header length"):
        M.inspect(tmp_path)
    # data range past the end of the file
    write_safetensors(path, {"model.norm.weight": ("F16", [64], b"\0" * 100)})
    d = bytearray(open(path, "rb").read())
    hlen = struct.unpack("<Q", d[:8])[0]
    hdr = json.loads(d[8:8 + hlen])
    hdr["model.norm.weight"]["data_offsets"] = [0, 10 ** 6]
    hb = json.dumps(hdr).encode()
    open(path, "wb").write(struct.pack("<Q", len(hb)) + hb + b"\0" * 100)
    with pytest.raises(GroutError, match="outside the file"):
        M.inspect(tmp_path)
    # byte count that does not match the shape
    write_safetensors(path, {"model.norm.weight": ("F16", [64], b"\0" * 100)})
    with pytest.raises(GroutError, match="holds 100 bytes"):
        M.inspect(tmp_path)
    # malformed JSON header
    hb = b'{"model.norm.weight": {"dtype": "F16", "shape": [64], "data_offsets": [0, 128]'
    open(path, "wb").write(struct.pack("<Q", len(hb)) + hb + b"\0" * 128)
    with pytest.raises(GroutError, match="bad header"):
        M.inspect(tmp_path)


def test_unsupported_dtype_on_a_needed_tensor(tmp_path):
    write_checkpoint(tmp_path, TINY, shards=1)
    path = os.path.join(tmp_path, "model.safetensors")
    d = bytearray(open(path, "rb").read())
    hlen = struct.unpack("<Q", d[:8])[0]
    hdr = json.loads(d[8:8 + hlen])
    e = hdr["model.norm.weight"]
    e["dtype"] = "I16"  # same byte size, a dtype the cast does not accept
    hb = json.dumps(hdr).encode()
    hb += b" " * (-len(hb) % 8)
    open(path, "wb").write(struct.pack("<Q", len(hb)) + hb + bytes(d[8 + hlen:]))
    with pytest.raises(GroutError, match="unsupported dtype"):
        M.inspect(tmp_path)


def test_config_json_with_escapes_and_nesting(tmp_path):
    write_checkpoint(tmp_path, TINY, shards=1,
                     config_over={"name_or_path": "Qwen\\/é😀 \"x\"\n",
                                  "rope_scaling": {"a": [1, 2.5e-3, {"b": None}], "c": True}})
    assert M.inspect(tmp_path)["config"].hidden_size == 64
