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


_FUZZ_CHILD = r'''
import ctypes as C, json, os, struct, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from grout_amd._lib import ModelInfo, lib
d, n = sys.argv[2], int(sys.argv[3])
names = sorted(os.listdir(d))
orig = {f: open(os.path.join(d, f), "rb").read() for f in names}
def span(f, b):  # where the parser reads: JSON files whole, safetensors 8 + header bytes
    if f.endswith(".safetensors"):
        return min(len(b), 8 + struct.unpack("<Q", orig[f][:8])[0])
    return len(b)
L, rng = lib(), np.random.default_rng(31415)
rcs = {}
for i in range(n):
    f = names[int(rng.integers(0, len(names)))]
    b = bytearray(orig[f])
    kind, hi = i % 6, span(f, b)
    pos = int(rng.integers(0, hi))
    if kind == 0:    # flipped bits
        for _ in range(int(rng.integers(1, 9))):
            b[int(rng.integers(0, hi))] ^= 1 << int(rng.integers(0, 8))
    elif kind == 1:  # truncated
        del b[pos:]
    elif kind == 2:  # inserted JSON punctuation, escapes, digits or random bytes
        pool = [b"{", b"}", b"[", b"]", b'"', b"\\", b"\\u", b",", b":", b"-", b"1e999",
                b"18446744073709551616", b"\x00", rng.bytes(int(rng.integers(1, 32)))]
        b[pos:pos] = pool[int(rng.integers(0, len(pool)))]
    elif kind == 3:  # dropped bytes
        del b[pos:pos + int(rng.integers(1, 32))]
    elif kind == 4:  # the safetensors header length (or any 8 bytes) set to an extreme
        v = [2**64 - 1, 2**63, 2**32, 0, 7, len(b), int(rng.integers(0, 2**63))]
        at = 0 if f.endswith(".safetensors") and rng.random() < 0.5 else pos
        b[at:at + 8] = struct.pack("<Q", v[int(rng.integers(0, len(v)))])
    else:            # a digit replaced: numbers out of range, negative, huge
        digits = [j for j in range(hi) if 48 <= b[j] <= 57]
        if digits:
            j = digits[int(rng.integers(0, len(digits)))]
            b[j:j + 1] = [b"9999999999999999999999", b"-1", b"0", b"1.5", b"nan"][int(rng.integers(0, 5))]
    with open(os.path.join(d, f), "wb") as fh:
        fh.write(b)
    info = ModelInfo()
    rc = L.grout_model_inspect(d.encode(), C.byref(info))
    if rc != 0 and not L.grout_last_error():
        print(json.dumps({"case": i, "file": f, "rc": rc, "error": "no message"}))
        sys.exit(3)
    rcs[str(rc)] = rcs.get(str(rc), 0) + 1
    with open(os.path.join(d, f), "wb") as fh:
        fh.write(orig[f])
print(json.dumps(rcs))
'''


def test_inspect_survives_corrupted_checkpoints(tmp_path):
    """3000 seeded corruptions of a two-shard checkpoint (one file per case:
    config.json, generation_config.json, the shard index or a safetensors
    header; flipped bits, truncation, inserted JSON punctuation and escapes,
    dropped bytes, header lengths and numbers set to extremes), inspected in
    one child process: every call returns OK or an error status with a
    message, and nothing crashes or hangs."""
    import subprocess
    import sys

    write_checkpoint(tmp_path, TINY, dtypes=("BF16", "F32", "F16"), shards=2,
                     generation_eos=[151645, 151643])
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FUZZ_CHILD, root, str(tmp_path), "3000"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    rcs = json.loads(r.stdout.strip().splitlines()[-1])
    assert sum(rcs.values()) == 3000
    assert set(rcs) <= {"0", "-1", "-3"}, rcs   # OK, EINVAL, ENOTSUP
    assert rcs.get("-1", 0) > 1000, rcs
