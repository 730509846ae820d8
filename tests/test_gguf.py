"""GGUF checkpoint reading (grout_model_inspect on a .gguf path: host only, no
GPU) over files written by tests/gguf_util.py: the config from the qwen3.*
metadata, the tied head, the device byte count, and the reader's error paths
with the reference's bounds (src/gguf.rs:212-445, its tests at 466-544)."""
import ctypes as C
import struct

import pytest

import oracle as O
import qutil
from gguf_util import (ARRAY, I32, STRING, U8, U32, U64, gguf_bytes, gstr, qwen3_meta,
                       qwen3_tensors)

Q4, Q5, Q6, Q8, F16 = O.Q4_K, O.Q5_K, O.Q6_K, O.Q8_0, 0
T_Q3_K = 11


def cfg_small():
    from grout_amd.model import Qwen3Config

    return Qwen3Config(num_layers=2, hidden_size=256, intermediate_size=512,
                       num_attention_heads=4, num_key_value_heads=2, vocab_size=300)


PLAN = {"embed": Q6, "lm_head": None,
        "layers": [{"q": Q4, "k": Q4, "v": Q6, "o": Q4, "gate": Q4, "up": Q4, "down": Q6},
                   {"q": Q8, "k": Q8, "v": Q5, "o": F16, "gate": Q5, "up": Q5, "down": Q5}]}


def inspect(path):
    from grout_amd._lib import ModelInfo, call

    info = ModelInfo()
    call("grout_model_inspect", str(path).encode(), C.byref(info))
    return info


def write(tmp_path, meta, tensors, name="m.gguf", **kw):
    p = tmp_path / name
    p.write_bytes(gguf_bytes(meta, tensors, **kw))
    return p


def model_file(tmp_path, plan=PLAN, meta_extra=(), **kw):
    cfg = cfg_small()
    spec, _, _ = qutil.mixed_weights(cfg, plan, 3, 0.05)
    return cfg, write(tmp_path, qwen3_meta(cfg, extra=meta_extra), qwen3_tensors(cfg, spec), **kw)


def expected_bytes(cfg, plan):
    """Device bytes: parts 256-aligned, one per same-format run."""
    from grout_amd._lib import lib

    def part(fmt, rows, k):
        b = rows * k * 2 if fmt == F16 else lib().grout_qweight_bytes(fmt, rows, k)
        return (b + 255) // 256 * 256

    def runs(fmts, rows, k):
        total, i = 0, 0
        while i < len(fmts):
            j, r = i, 0
            while j < len(fmts) and fmts[j] == fmts[i]:
                r += rows[j]
                j += 1
            total += part(fmts[i], r, k)
            i = j
        return total

    H, I, V, qd, kd = (cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.q_dim,
                       cfg.kv_dim)
    vec = lambda n: (n * 2 + 255) // 256 * 256
    total = part(plan["embed"], V, H) + vec(H)
    if plan["lm_head"] is not None:
        total += part(plan["lm_head"], V, H)
    for p in plan["layers"]:
        total += 2 * vec(H) + 2 * vec(128)
        total += runs([p["q"], p["k"], p["v"]], [qd, kd, kd], H)
        total += runs([p["gate"], p["up"]], [I, I], H)
        total += part(p["o"], H, qd) + part(p["down"], H, I)
    return total


def test_inspect_reads_config_and_sizes(tmp_path):
    cfg, path = model_file(tmp_path)
    info = inspect(path)
    c = info.config
    assert (c.num_layers, c.hidden_size, c.intermediate_size, c.num_q_heads, c.num_kv_heads,
            c.head_dim, c.vocab_size, c.max_ctx) == (2, 256, 512, 4, 2, 128, 300, 4096)
    assert c.rms_norm_eps == pytest.approx(cfg.rms_norm_eps) and c.rope_theta == cfg.rope_theta
    assert info.tie_word_embeddings == 1 and info.num_eos == 1 and info.eos_token_ids[0] == 7
    assert info.weight_bytes == expected_bytes(cfg, PLAN)


def test_untied_head_and_alignment(tmp_path):
    plan = dict(PLAN, lm_head=Q8)
    cfg, path = model_file(tmp_path, plan, meta_extra=[("general.alignment", U32, 64)],
                           alignment=64)
    info = inspect(path)
    assert info.tie_word_embeddings == 0
    assert info.weight_bytes == expected_bytes(cfg, plan)


def _err(path, match):
    from grout_amd._lib import GroutError

    with pytest.raises(GroutError, match=match):
        inspect(path)


def test_header_errors(tmp_path):
    cfg, path = model_file(tmp_path)
    data = path.read_bytes()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + data[4:])
    _err(bad, "magic")
    bad.write_bytes(data[:4] + struct.pack("<I", 1) + data[8:])
    _err(bad, "version 1")
    for cut in (30, 200, len(data) // 2, len(data) - 10):
        bad.write_bytes(data[:cut])
        _err(bad, "truncated|outside the file|exceeds|too short")
    bad.write_bytes(data[:4])
    _err(bad, "too short")


def test_metadata_bounds(tmp_path):
    # a string longer than the rest of the file
    head = struct.pack("<IIQQ", 0x46554747, 3, 0, 1)
    p = tmp_path / "s.gguf"
    p.write_bytes(head + struct.pack("<Q", 5) + b"k" * 5 + struct.pack("<I", STRING)
                  + struct.pack("<Q", 1 << 20) + b"abc")
    _err(p, "string length")
    # an array claiming more elements than the metadata budget (16M), before
    # anything is read or allocated
    p.write_bytes(head + gstr("arr") + struct.pack("<I", ARRAY) + struct.pack("<IQ", U8, 1 << 25)
                  + b"\0" * 64)
    _err(p, "budget")
    # sibling arrays cannot exceed the budget together
    two = struct.pack("<IIQQ", 0x46554747, 3, 0, 2)
    arr = struct.pack("<I", ARRAY) + struct.pack("<IQ", U8, 9 << 20)
    p.write_bytes(two + gstr("a") + arr + b"\0" * (9 << 20) + gstr("b") + arr + b"\0" * (9 << 20))
    _err(p, "budget")
    # an invalid bool
    p.write_bytes(head + gstr("b") + struct.pack("<I", 7) + b"\x02")
    _err(p, "bool")


def test_config_errors(tmp_path):
    cfg = cfg_small()
    spec, _, _ = qutil.mixed_weights(cfg, PLAN, 3, 0.05)
    tensors = qwen3_tensors(cfg, spec)
    meta = qwen3_meta(cfg)
    arch = [m for m in meta if m[0] != "general.architecture"]
    _err(write(tmp_path, arch + [("general.architecture", STRING, "llama")], tensors),
         "architecture `llama`")
    _err(write(tmp_path, [m for m in meta if m[0] != "qwen3.block_count"], tensors),
         "qwen3.block_count is missing")
    _err(write(tmp_path, [m for m in meta if m[0] != "qwen3.rope.freq_base"]
               + [("qwen3.rope.freq_base", I32, 5)], tensors), "not f32")
    kl = [m for m in meta if m[0] != "qwen3.attention.key_length"]
    _err(write(tmp_path, kl + [("qwen3.attention.key_length", U32, 64)], tensors),
         "only 128")
    # duplicate keys: the last one wins (as in the reference)
    info = inspect(write(tmp_path, meta + [("tokenizer.ggml.eos_token_id", U64, 11)], tensors))
    assert info.eos_token_ids[0] == 11


def test_tensor_errors(tmp_path):
    cfg = cfg_small()
    spec, _, _ = qutil.mixed_weights(cfg, PLAN, 3, 0.05)
    meta = qwen3_meta(cfg)
    tensors = qwen3_tensors(cfg, spec)

    def with_tensor(name, new):
        return [new if t[0] == name else t for t in tensors]

    _err(write(tmp_path, meta, [t for t in tensors if t[0] != "blk.1.ffn_up.weight"]),
         "missing tensor blk.1.ffn_up.weight")
    t = next(t for t in tensors if t[0] == "blk.0.attn_k.weight")
    _err(write(tmp_path, meta, with_tensor(t[0], (t[0], t[1], (t[2][0] * 2, t[2][1] // 2), t[3]))),
         "blk.0.attn_k.weight has shape")
    # a Q3_K matrix is a GGUF type but not a format this build runs
    q3 = (t[0], T_Q3_K, t[2], b"\0" * (t[2][0] * t[2][1] // 256 * 110))
    _err(write(tmp_path, meta, with_tensor(t[0], q3)), "unsupported ggml type Q3_K")
    # a low-bit norm vector is refused
    n = next(t for t in tensors if t[0] == "blk.0.attn_norm.weight")
    _err(write(tmp_path, meta, with_tensor(n[0], (n[0], 8, (256,), b"\0" * 272))),
         "unsupported ggml type Q8_0")
    # five dimensions
    _err(write(tmp_path, meta, tensors + [("extra", 0, (1, 1, 1, 1, 1), b"\0" * 4)]),
         "5 dimensions")
    # a tensor whose data runs past the end of the file
    data = bytearray(gguf_bytes(meta, tensors))
    p = tmp_path / "short.gguf"
    p.write_bytes(bytes(data[:-1000]))
    _err(p, "outside the file|truncated")


_FUZZ_CHILD = r'''
import ctypes as C, json, struct, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from grout_amd._lib import ModelInfo, lib
base, path, n = open(sys.argv[2], "rb").read(), sys.argv[3], int(sys.argv[4])
L, rng = lib(), np.random.default_rng(2718)
head = min(len(base), 8192)  # header, metadata and tensor infos live here
rcs = {}
for i in range(n):
    b = bytearray(base)
    kind = i % 6
    pos = int(rng.integers(0, head if rng.random() < 0.85 else len(b)))
    if kind == 0:    # flipped bits
        for _ in range(int(rng.integers(1, 9))):
            b[int(rng.integers(0, head))] ^= 1 << int(rng.integers(0, 8))
    elif kind == 1:  # truncated
        del b[pos:]
    elif kind == 2:  # a 64-bit field (length, count, dimension, offset) set to an extreme
        v = [2**64 - 1, 2**63, 2**62 + 1, 2**32, 2**31 - 1, int(rng.integers(0, 2**63))]
        b[pos:pos + 8] = struct.pack("<Q", v[int(rng.integers(0, len(v)))])
    elif kind == 3:  # inserted bytes
        b[pos:pos] = rng.bytes(int(rng.integers(1, 64)))
    elif kind == 4:  # dropped bytes
        del b[pos:pos + int(rng.integers(1, 64))]
    else:            # a 32-bit field (type, version, dimension count) set to an extreme
        v = [0, 1, 12, 13, 30, 31, 255, 2**31, 2**32 - 1]
        b[pos:pos + 4] = struct.pack("<I", v[int(rng.integers(0, len(v)))])
    with open(path, "wb") as f:
        f.write(b)
    info = ModelInfo()
    rc = L.grout_model_inspect(path.encode(), C.byref(info))
    if rc != 0 and not L.grout_last_error():
        print(json.dumps({"case": i, "rc": rc, "error": "no message"}))
        sys.exit(3)
    rcs[str(rc)] = rcs.get(str(rc), 0) + 1
print(json.dumps(rcs))
'''


def test_inspect_survives_corrupted_files(tmp_path):
    """3000 seeded corruptions of a valid GGUF (flipped bits, truncation,
    inserted and dropped bytes, 32- and 64-bit fields set to extremes, mostly
    in the header, metadata and tensor infos), inspected in one child
    process: every call returns OK or an error status with a message, and
    nothing crashes or hangs (a crash fails this test with its signal)."""
    import json
    import os
    import subprocess
    import sys

    _, path = model_file(tmp_path)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FUZZ_CHILD, root, str(path),
                        str(tmp_path / "fuzz.gguf"), "3000"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    rcs = json.loads(r.stdout.strip().splitlines()[-1])
    assert sum(rcs.values()) == 3000
    assert set(rcs) <= {"0", "-1", "-3"}, rcs   # OK, EINVAL, ENOTSUP
    assert rcs.get("-1", 0) > 1000, rcs           # most corruptions are caught
