"""CPU checks of the C ABI boundary: the library loads, exports every symbol
include/grout_attn.h declares, and rejects bad arguments before touching a GPU."""
import ctypes as C
import glob
import os
import re

import numpy as np
import pytest

import grout_amd
from grout_amd import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def header_functions():
    text = "\n".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(grout_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


EXAMPLE = os.path.join(ROOT, "grout_amd", "examples", "grout_generate")


def test_cpp_api_header_compiles_strictly(tmp_path):
    """include/grout.hpp (the C++ mirror of the reference's Engine API) as a
    C++17 caller sees it: -Wall -Wextra -Werror -pedantic."""
    import shutil
    import subprocess

    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not found")
    src = tmp_path / "use.cpp"
    src.write_text('#include "grout.hpp"\n'
                   "int main() {\n"
                   "  grout::LoadOpts o; grout::Logits l; grout::ModelMeta m;\n"
                   "  (void)o; (void)l.as_slice(); (void)m;\n"
                   "  return std::is_nothrow_move_constructible<grout::Engine>::value ? 0 : 1;\n"
                   "}\n")
    r = subprocess.run([cxx, "-std=c++17", "-Wall", "-Wextra", "-Werror", "-pedantic",
                        "-include", "type_traits", f"-I{os.path.join(ROOT, 'include')}",
                        "-fsyntax-only", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_cpp_example_reports_errors_before_any_gpu_call():
    """grout_amd/examples/grout_generate (built with the library) reports a
    missing model directory, bad arguments and usage without touching a GPU."""
    import subprocess

    assert os.path.exists(EXAMPLE), "run `python -m grout_amd.build` first"
    r = subprocess.run([EXAMPLE, "/nonexistent-model-dir", "16", "1", "3"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 1 and "grout error -1" in r.stderr and "config.json" in r.stderr
    r = subprocess.run([EXAMPLE, "/nonexistent-model-dir", "16", "x", "3"], capture_output=True,
                       text=True, timeout=60)
    assert r.returncode == 1 and "bad n_decode" in r.stderr
    r = subprocess.run([EXAMPLE], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr


def test_library_is_built_and_loads():
    assert os.path.exists(grout_amd.LIB_PATH), "run `python -m grout_amd.build` first"
    L = grout_amd.lib()
    assert L.grout_abi_version() >> 16 == 1


def test_every_declared_symbol_is_exported_and_bound():
    names = header_functions()
    assert len(HEADERS) >= 2 and len(names) >= 31
    L = grout_amd.lib()
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/ but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_headers_compile_as_c11_and_a_c_caller_links(tmp_path):
    """What an FFI crate binds: both headers compile as strict C11 (-pedantic
    -Werror), a C program takes the address of every declared function, links
    against the library and runs the host-only entry points and an argument
    error (no GPU call), with the same results as the ctypes binding."""
    import shutil
    import subprocess

    import oracle as O

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    names = header_functions()
    src = ["#include \"grout_attn.h\"", "#include \"grout_engine.h\"", "#include <stdio.h>",
           "typedef void (*fp)(void);", "static fp const table[] = {"]
    src += [f"    (fp){n}," for n in names]
    src += ["};",
            "int main(void) {",
            "  size_t i;",
            "  float inv[64];",
            "  int r;",
            "  for (i = 0; i < sizeof table / sizeof table[0]; ++i)",
            "    if (!table[i]) return 10;",
            "  if (grout_rope_inv_freq(128, 1e6f, inv) != GROUT_OK) return 11;",
            "  printf(\"%d %d %zu %.9g\\n\", grout_abi_version(),",
            "         grout_attn_decode_default_splits(32768, 64, 8),",
            "         grout_attn_decode_workspace_bytes(64, 8, 128, 32), (double)inv[1]);",
            "  r = grout_fmha_prefill(NULL, NULL, NULL, NULL, 16, 0, 0, 8, 128, 0, 0.1f, NULL);",
            "  printf(\"%d %s\\n\", r, grout_last_error());",
            "  return r == GROUT_EINVAL ? 0 : 12;",
            "}"]
    (tmp_path / "abi.c").write_text("\n".join(src) + "\n")
    libdir = os.path.dirname(grout_amd.LIB_PATH)
    exe = tmp_path / "abi"
    subprocess.run([gcc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic",
                    "-I", os.path.join(ROOT, "include"), str(tmp_path / "abi.c"), "-L", libdir,
                    "-lgrout_attn", f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, (run.returncode, run.stdout, run.stderr)
    first, second = run.stdout.strip().splitlines()
    ver, splits, ws, inv1 = first.split()
    L = grout_amd.lib()
    assert int(ver) == L.grout_abi_version()
    assert int(splits) == L.grout_attn_decode_default_splits(32768, 64, 8)
    assert int(ws) == L.grout_attn_decode_workspace_bytes(64, 8, 128, 32)
    assert np.float32(float(inv1)) == O.inv_freq(128, 1e6)[1]
    assert second.startswith("-1 ") and "num_q_heads" in second


def test_integration_rust_block_declares_every_header_function():
    """The Rust `extern "C"` block of the integration notes (what a maintainer
    would paste into the FFI crate) declares exactly the functions the headers
    do."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = text[text.index("## 1."):text.index("## 2.")]
    declared = set(re.findall(r"pub fn (grout_[a-z0-9_]+)", block))
    assert declared == set(header_functions())


def test_integration_rust_constants_match_the_headers():
    """Every value #define of both headers appears in the Rust block as a
    `pub const` of the same value (status codes, limits, weight formats)."""
    defines = {}
    for h in ("grout_attn.h", "grout_engine.h"):
        for name, val in re.findall(r"^#define (GROUT_[A-Z0-9_]+) +([^/\n]+)",
                                    open(os.path.join(ROOT, "include", h)).read(), re.M):
            defines[name] = eval(val.strip())  # integer literals, shifts, negation
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = text[text.index("## 1."):text.index("## 2.")]
    consts = {n: eval(v) for n, v in re.findall(r"pub const (GROUT_[A-Z0-9_]+): \w+ = ([^;]+);",
                                                block)}
    assert consts == defines


def test_rope_host_functions_match_oracle_bit_for_bit():
    import oracle as O

    inv = np.empty(64, np.float32)
    assert grout_amd.lib().grout_rope_inv_freq(128, 1e6, inv.ctypes.data_as(C.c_void_p)) == 0
    assert np.array_equal(inv, O.inv_freq(128, 1e6))
    c = np.empty((300, 64), np.float32)
    s = np.empty((300, 64), np.float32)
    assert grout_amd.lib().grout_rope_table_host(300, 128, 1e6, c.ctypes.data_as(C.c_void_p),
                                                 s.ctypes.data_as(C.c_void_p)) == 0
    oc, os_ = O.rope_table(300, 128, 1e6)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)


def _aligned(n=4096):
    buf = (C.c_char * (n + 64))()
    addr = (C.addressof(buf) + 63) & ~63
    return buf, C.c_void_p(addr)


def test_argument_validation_without_gpu():
    L = grout_amd.lib()
    keep, p = _aligned()
    # head_dim != 128 -> not supported
    rc = L.grout_fmha_prefill(p, p, p, p, 16, 0, 8, 2, 64, 16 * 64, 0.125, None)
    assert rc == -3 and "head_dim" in _lib.last_error()
    # Hq not a multiple of Hkv
    rc = L.grout_fmha_prefill(p, p, p, p, 16, 0, 6, 4, 128, 16 * 128, 0.088, None)
    assert rc == -1 and "multiple" in _lib.last_error()
    # empty prefill
    rc = L.grout_fmha_prefill(p, p, p, p, 0, 0, 8, 2, 128, 16 * 128, 0.088, None)
    assert rc == -1
    # misaligned pointer
    bad = C.c_void_p(p.value + 2)
    rc = L.grout_fmha_prefill(bad, p, p, p, 4, 0, 8, 2, 128, 16 * 128, 0.088, None)
    assert rc == -2 and "aligned" in _lib.last_error()
    # kv head stride too small for pos0 + seq_len rows
    rc = L.grout_fmha_prefill(p, p, p, p, 8, 10, 8, 2, 128, 16 * 128, 0.088, None)
    assert rc == -1 and "kv_head_stride" in _lib.last_error()
    # fused write out of cache range
    rc = L.grout_qk_norm_rope_kv_prefill(p, p, p, p, p, p, p, p, p, p, 30, 8, 8, 2, 128, 32,
                                         32 * 128, 1e-6, None)
    assert rc == -1 and "exceeds max_seq_len" in _lib.last_error()
    # decode group above 16
    rc = L.grout_attn_decode(p, p, p, p, p, 1 << 20, p, 34, 2, 128, 64, 64 * 128, 4, 0.088, None)
    assert rc == -3
    # workspace too small
    rc = L.grout_attn_decode(p, p, p, p, p, 16, p, 8, 2, 128, 64, 64 * 128, 4, 0.088, None)
    assert rc == -1 and "workspace" in _lib.last_error()
    # NULL position pointer
    rc = L.grout_fmha_decode_gqa_split(p, p, p, p, p, None, 8, 2, 128, 64, 64 * 128, 2, 0.088, None)
    assert rc == -1 and "d_pos" in _lib.last_error()
    # split counts past GROUT_MAX_SPLITS (4096)
    rc = L.grout_fmha_decode_gqa_split(p, p, p, p, p, p, 8, 2, 128, 64, 64 * 128, 4097, 0.088, None)
    assert rc == -1 and "4096" in _lib.last_error()
    rc = L.grout_attn_decode(p, p, p, p, p, 1 << 30, p, 8, 2, 128, 64, 64 * 128, 4097, 0.088, None)
    assert rc == -1 and "4096" in _lib.last_error()
    rc = L.grout_splitk_reduce_merge(p, p, p, 8, 2, 128, 4097, None)
    assert rc == -1 and "4096" in _lib.last_error()


# Qwen3-4B (32 / 8 heads) and Qwen3-32B (64 / 8): the pick at each length, the
# fastest of the six forms in a sweep on MI355X (form 0 shared stream, 1 per-team
# 128-row blocks, 2 per-team 64-row blocks; paired; workgroups).
PREFILL_PLANS = {
    (256, 32): (2, 0, 128), (512, 32): (2, 0, 256), (768, 32): (2, 1, 192),
    (1024, 32): (2, 1, 256), (1280, 32): (1, 0, 320), (1536, 32): (1, 1, 192),
    (2048, 32): (1, 1, 256), (2560, 32): (1, 0, 640), (3072, 32): (0, 0, 384),
    (4096, 32): (0, 1, 256), (5120, 32): (1, 0, 1280), (6144, 32): (1, 1, 768),
    (8192, 32): (0, 1, 512),
    (256, 64): (2, 0, 256), (512, 64): (2, 1, 256), (768, 64): (1, 1, 192),
    (1024, 64): (1, 1, 256), (1536, 64): (0, 0, 384), (2048, 64): (0, 1, 256),
    (3072, 64): (1, 1, 768), (4096, 64): (0, 1, 512),
}


@pytest.mark.parametrize("S,Hq", sorted(PREFILL_PLANS))
def test_prefill_work_split_plan(monkeypatch, S, Hq):
    for k in ("SHARED", "PAIRED", "WAVE_ROWS"):
        monkeypatch.delenv("GROUT_FMHA_PREFILL_" + k, raising=False)
    p = ops.prefill_plan(S, Hq, 8)
    assert (p["form"], int(p["paired"]), p["workgroups"]) == PREFILL_PLANS[(S, Hq)]


def test_prefill_plan_overrides_and_errors(monkeypatch):
    monkeypatch.setenv("GROUT_FMHA_PREFILL_SHARED", "1")
    assert ops.prefill_plan(512, 32, 8)["form"] == 0
    monkeypatch.setenv("GROUT_FMHA_PREFILL_SHARED", "0")
    monkeypatch.setenv("GROUT_FMHA_PREFILL_WAVE_ROWS", "32")
    monkeypatch.setenv("GROUT_FMHA_PREFILL_PAIRED", "0")
    p = ops.prefill_plan(2048, 32, 8)
    assert (p["form"], p["paired"], p["workgroups"]) == (1, False, 512)
    monkeypatch.setenv("GROUT_FMHA_PREFILL_WAVE_ROWS", "16")
    monkeypatch.setenv("GROUT_FMHA_PREFILL_PAIRED", "1")
    p = ops.prefill_plan(2048, 32, 8)
    assert (p["form"], p["paired"], p["workgroups"]) == (2, True, 512)
    L = grout_amd.lib()
    assert L.grout_fmha_prefill_plan(0, 32, 8, None, None, None) == -1
    assert L.grout_fmha_prefill_plan((1 << 22) + 1, 32, 8, None, None, None) == -1
    assert L.grout_fmha_prefill_plan(16, 30, 8, None, None, None) == -1


def test_decode_split_defaults_and_workspace():
    L = grout_amd.lib()
    assert L.grout_attn_decode_default_splits(1, 32, 8) == 1
    assert L.grout_attn_decode_default_splits(4096, 32, 8) == 32
    assert L.grout_attn_decode_default_splits(32768, 64, 8) == 32
    assert L.grout_attn_decode_default_splits(100, 32, 8) == 1
    assert L.grout_attn_decode_default_splits(128, 32, 8) == 1
    assert L.grout_attn_decode_default_splits(129, 32, 8) == 5
    assert L.grout_attn_decode_default_splits(512, 32, 8) == 16
    assert L.grout_attn_decode_default_splits(1024, 32, 8) == 32
    assert L.grout_attn_decode_default_splits(1024, 64, 4) == 32
    assert L.grout_attn_decode_default_splits(40960, 32, 1) == 256
    ws = L.grout_attn_decode_workspace_bytes(64, 8, 128, 64)
    assert ws == 8 * 64 * 8 * 130 * 4  # fp32 partial acc + (max, sum) per (kv head, split, head)
    assert L.grout_attn_decode_workspace_bytes(64, 8, 96, 64) == 0


def test_graph_create_rejects_bad_layers_without_gpu():
    L = grout_amd.lib()
    layers = (_lib.DecodeLayer * 1)()
    h = C.c_void_p()
    keep, p = _aligned()
    rc = L.grout_decode_graph_create(layers, 1, p, p, p, 1 << 20, 32, 8, 128, 4096, 0, 1e-6, 0.088,
                                     None, C.byref(h))
    assert rc == -1 and "layer 0" in _lib.last_error()
    assert L.grout_decode_graph_launch(None, 0, None) == -1
    assert L.grout_decode_graph_destroy(None) == 0


def test_ops_fail_loudly_without_library(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="missing"):
        _lib.lib()


def _cfg4b(max_ctx):
    return _lib.Qwen3Config(36, 2560, 9728, 32, 8, 128, 151936, 1e-6, 1e6, max_ctx)


def test_vram_preflight_sums_and_refuses_without_gpu():
    """The preflight's byte total and its refusal are host arithmetic: KV is
    layers x 2 x Hkv x max_ctx x 256 B, rope max_ctx x 512 B, plus weights,
    scratch and 700 MiB of slack (src/model.rs:181, 345-380)."""
    L = grout_amd.lib()
    cfg = _cfg4b(32768)
    req = _lib._sz(0)
    kv = 36 * 2 * 8 * 32768 * 128 * 2
    rope = 32768 * 128 * 4
    slack = 700 << 20
    w, scr = 8_044_936_192, 123_456
    assert L.grout_engine_vram_preflight(C.byref(cfg), w, scr, 1 << 40, 1 << 40, C.byref(req)) == 0
    assert req.value == w + kv + rope + scr + slack
    # one byte short of the requirement -> GROUT_ENOMEM with the itemized summary
    rc = L.grout_engine_vram_preflight(C.byref(cfg), w, scr, req.value - 1, 1 << 40, None)
    assert rc == -5
    msg = _lib.last_error()
    assert "VRAM preflight failed" in msg and "max_ctx=32768" in msg and "KV=32768 tokens" in msg
    assert L.grout_engine_vram_preflight(C.byref(cfg), w, scr, req.value, 1 << 40, None) == 0
    assert L.grout_engine_vram_preflight(None, 0, 0, 0, 0, None) == -1


def test_max_ctx_cap_and_engine_queries_without_gpu():
    L = grout_amd.lib()
    keep, p = _aligned()
    # cache lengths past GROUT_MAX_CTX (32-bit row offsets) are refused up front
    big = (1 << 22) + 1
    rc = L.grout_attn_decode(p, p, p, p, p, 1 << 20, p, 8, 2, 128, big, big * 128, 4, 0.088, None)
    assert rc == -3 and "GROUT_MAX_CTX" in _lib.last_error()
    rc = L.grout_fmha_prefill(p, p, p, p, 8, (1 << 22) - 4, 8, 2, 128, big * 128, 0.088, None)
    assert rc == -3 and "GROUT_MAX_CTX" in _lib.last_error()
    # engine status queries on NULL
    assert L.grout_engine_uses_decode_graph(None) == 0
    assert L.grout_engine_decode_graph_error(None) == b""
    # an engine config past the cap is refused before any device call
    cfg = _cfg4b(big)
    h = C.c_void_p()
    w = _lib.Qwen3Weights()
    assert L.grout_engine_create(C.byref(cfg), C.byref(w), 0, C.byref(h)) in (-1, -3)


def test_gemv_norm_rejects_residual_aliasing_without_gpu():
    """The norm-folded GEMVs' first workgroup writes residual_out while the
    others still read residual and x: any overlap of those k-element f16
    vectors is refused (same start, or an offset inside either range); a
    range that only touches them gets past the check."""
    L = grout_amd.lib()
    keep, p = _aligned(1 << 16)
    k = 64  # 128 bytes per vector
    a = C.c_void_p(p.value + 4096)   # residual
    b = C.c_void_p(p.value + 8192)   # x
    at = lambda base, off: C.c_void_p(base.value + off)
    overlapping = (a, b, at(a, 16), at(a, -112), at(b, 112), at(b, -16))
    touching = (at(a, 128), at(a, -128), at(b, 128), at(b, -128))
    f16_forms = [getattr(L, fn) for fn in ("grout_gemv_rms_norm", "grout_gemv_rms_norm_silu_mul")]
    q_forms = [getattr(L, fn) for fn in ("grout_gemv_q_rms_norm", "grout_gemv_q_rms_norm_silu_mul")]
    for ro in overlapping + touching:
        calls = [lambda f=f: f(p, a, b, p, ro, p, 16, k, 1e-6, None) for f in f16_forms]
        calls += [lambda f=f: f(8, p, a, b, p, ro, p, 16, k, 1e-6, None) for f in q_forms]
        for c in calls:
            rc = c()
            if any(ro.value == o.value for o in overlapping):
                assert rc == -1 and "overlap" in _lib.last_error(), (ro.value - p.value, rc)
            else:
                assert rc == 0 or "overlap" not in _lib.last_error(), ro.value - p.value


def test_env_flag_parses_like_env_bool_or():
    """GROUT_HIP_GRAPH_DECODE is read like the reference's env_bool_or
    (src/model.rs:212-224): trimmed, case-insensitive, explicit spellings
    only, anything else (or unset) the default."""
    L = grout_amd.lib()
    for raw in (b"1", b"true", b"TRUE", b" on ", b"Yes", b"\tyes\n"):
        assert L.grout_env_flag(raw, 0) == 1, raw
    for raw in (b"0", b"false", b"Off", b" no ", b"", b"   "):
        assert L.grout_env_flag(raw, 1) == 0, raw
    for raw in (b"2", b"enabled", b"nope", b"0x1", b"y"):
        assert L.grout_env_flag(raw, 0) == 0 and L.grout_env_flag(raw, 1) == 1, raw
    assert L.grout_env_flag(None, 1) == 1 and L.grout_env_flag(None, 0) == 0


def test_env_usize_parses_like_env_usize_or():
    """GROUT_FMHA_NUM_KV_SPLITS is read like the reference's env_usize_or
    (src/model.rs:204-210, Rust's usize parse): an optional '+' and decimal
    digits; zero, whitespace, signs other than '+', other text, overflow or
    unset give the default."""
    L = grout_amd.lib()
    for raw, want in ((b"16", 16), (b"+7", 7), (b"007", 7), (b"4096", 4096),
                      (b"18446744073709551615", 17), (b"18446744073709551616", 17),
                      (b"0", 17), (b"-3", 17), (b" 16", 17), (b"16 ", 17), (b"", 17),
                      (b"+", 17), (b"1e3", 17), (b"0x10", 17), (b"abc", 17), (None, 17)):
        assert L.grout_env_usize(raw, 17) == want, raw
    assert L.grout_env_usize(b"9223372036854775807", 5) == 9223372036854775807


def test_low_bit_k_limit_covers_qwen3_without_gpu():
    """The low-bit GEMVs stage x in LDS: every Qwen3 ffn_down width up to
    32B's 25600 is accepted, K past 32768 is refused (host-side sizing)."""
    L = grout_amd.lib()
    for fmt, blk in ((8, 32), (12, 256), (13, 256), (14, 256)):
        for k in (17408, 25600, 32768):
            assert L.grout_qweight_bytes(fmt, 5120, k) > 0, (fmt, k)
        assert L.grout_qweight_bytes(fmt, 5120, 32768 + blk) == 0, fmt
