"""GPU parity of the Qwen3 engine over mixed-format (GGUF block) weights
(grout_engine_create_q) against the CPU oracle, through the C ABI.

Weights: seeded N(0, std) matrices quantized by tests/qutil.py into the plan's
formats, Q4_K_M-style mixes (q/k Q4_K with v Q6_K, gate/up in one format or
two, f16 parts among low-bit ones, tied and untied heads).  The oracle
multiplies decode steps (and the head) by the fp32 dequantized weights the
GEMVs use, prefill and extend rows by those weights rounded to f16 (the
dequant + GEMM path), and gathers embeddings by the CPU dequantization rule.
Tolerances as the f16 engine's (tests/test_gpu_model.py)."""
import numpy as np
import pytest

import oracle as O
from oracle import qwen3 as Q
import qutil
from test_gpu_model import check_logits, check_token

pytestmark = pytest.mark.gpu

F16, Q8, Q4, Q5, Q6 = qutil.F16, O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K


def configs():
    from grout_amd.model import Qwen3Config

    return {
        "g2": Qwen3Config(num_layers=2, hidden_size=256, intermediate_size=512,
                          num_attention_heads=4, num_key_value_heads=2, vocab_size=300),
        "k1024": Qwen3Config(num_layers=2, hidden_size=1024, intermediate_size=2048,
                             num_attention_heads=8, num_key_value_heads=2, vocab_size=16500),
        "4b-dims-2l": Qwen3Config(num_layers=2, hidden_size=2560, intermediate_size=9728,
                                  num_attention_heads=32, num_key_value_heads=8,
                                  vocab_size=32000),
    }


Q4KM = {"q": Q4, "k": Q4, "v": Q6, "o": Q4, "gate": Q4, "up": Q4, "down": Q6}
MIXED = {"q": Q8, "k": Q8, "v": Q8, "o": Q6, "gate": Q4, "up": Q8, "down": F16}
SPLIT = {"q": Q6, "k": F16, "v": Q4, "o": F16, "gate": Q6, "up": Q6, "down": Q4}
Q5KM = {"q": Q5, "k": Q5, "v": Q6, "o": Q5, "gate": Q5, "up": Q5, "down": Q6}

PLANS = {
    "q4km-tied": {"embed": Q4, "lm_head": None, "layers": [Q4KM, MIXED]},
    "mixed-untied": {"embed": Q8, "lm_head": Q6, "layers": [SPLIT, Q4KM]},
    "f16-embed": {"embed": F16, "lm_head": Q8, "layers": [MIXED, SPLIT]},
    "q5km-tied": {"embed": Q5, "lm_head": None, "layers": [Q5KM, MIXED]},
}


def build(name, plan_name, seed, max_ctx):
    from grout_amd.model import Engine, QuantWeights

    cfg = configs()[name]
    std = 0.05 if cfg.hidden_size < 2048 else 0.02
    spec, host, w64 = qutil.mixed_weights(cfg, PLANS[plan_name], seed, std)
    qw = QuantWeights(cfg, **spec)
    eng = Engine.from_quantized(cfg, qw, max_ctx=max_ctx)
    orc = Q.Qwen3Oracle(cfg, host, max_ctx, decode_w64=w64)
    return cfg, eng, orc


@pytest.mark.parametrize("name,plan,n_prompt,n_decode,max_ctx", [
    ("g2", "q4km-tied", 37, 5, 64), ("g2", "mixed-untied", 1, 3, 16),
    ("g2", "f16-embed", 20, 3, 64), ("k1024", "q4km-tied", 70, 4, 256),
    ("k1024", "mixed-untied", 33, 3, 256), ("4b-dims-2l", "q4km-tied", 41, 3, 1024),
    ("g2", "q5km-tied", 29, 4, 64), ("k1024", "q5km-tied", 45, 3, 256)])
def test_qengine_prefill_and_decode_vs_oracle(gpu, name, plan, n_prompt, n_decode, max_ctx):
    print(f"qengine {name} {plan} prompt={n_prompt} decode={n_decode}", flush=True)
    cfg, eng, orc = build(name, plan, 5 + n_prompt, max_ctx)
    prompt = np.random.default_rng(n_prompt).integers(0, cfg.vocab_size, n_prompt)
    try:
        got = eng.prefill(prompt).values
        ref, _ = orc.prefill(prompt, nthreads=8)
        tol = check_logits(got, ref, f"q {name} {plan} prefill")
        tok = int(np.argmax(got))
        check_token(tok, ref, tol, "prefill token")
        for i in range(n_decode):
            got = eng.decode(tok).values
            ref, _ = orc.decode(tok, nthreads=8)
            tol = check_logits(got, ref, f"q {name} {plan} decode {i}")
            tok = int(np.argmax(got))
            check_token(tok, ref, tol, f"decode token {i}")
        assert eng.position == n_prompt + n_decode
    finally:
        eng.close()


def test_qengine_extend_and_greedy_vs_oracle(gpu):
    """Extend chunks (dequant + GEMM rows at pos0 > 0, one of them a single
    token) between decode steps; decode_greedy agrees with the oracle."""
    cfg, eng, orc = build("k1024", "mixed-untied", 9, 256)
    rng = np.random.default_rng(4)
    try:
        prompt = rng.integers(0, cfg.vocab_size, 25)
        got = eng.prefill(prompt).values
        ref, _ = orc.prefill(prompt, nthreads=8)
        check_logits(got, ref, "q prefill")
        tok = int(np.argmax(got))
        got = eng.decode(tok).values
        ref, _ = orc.decode(tok, nthreads=8)
        check_logits(got, ref, "q decode")
        for chunk in (rng.integers(0, cfg.vocab_size, 17), [int(np.argmax(got))]):
            got = eng.extend(chunk).values
            ref, _ = orc.forward(chunk, orc.next_pos, nthreads=8)
            tol = check_logits(got, ref, f"q extend {len(chunk)}")
        tok = int(np.argmax(got))
        nxt = eng.decode_greedy(tok)
        ref, _ = orc.decode(tok, nthreads=8)
        check_token(nxt, ref, tol, "decode_greedy token")
        assert eng.position == 25 + 1 + 17 + 1 + 1
    finally:
        eng.close()


def test_qengine_warmup_leaves_a_fresh_session(gpu):
    """grout_engine_warmup on a mixed-format engine: after a session, the
    warmup's one-token prefill (dequant + GEMM path) and decode-graph replay,
    then the reset, leave position 0, and the next prefill and greedy steps
    equal a fresh engine's bit for bit."""
    cfg, eng, _ = build("k1024", "q4km-tied", 21, 256)
    _, fresh, _ = build("k1024", "q4km-tied", 21, 256)
    rng = np.random.default_rng(8)
    try:
        eng.prefill(rng.integers(0, cfg.vocab_size, 9))
        eng.decode_greedy(5)
        eng.warmup()
        assert eng.position == 0
        prompt = rng.integers(0, cfg.vocab_size, 30)
        a, b = eng.prefill(prompt).values, fresh.prefill(prompt).values
        assert np.array_equal(a, b)
        tok = int(np.argmax(a))
        for i in range(3):
            ta, tb = eng.decode_greedy(tok), fresh.decode_greedy(tok)
            assert ta == tb, f"step {i}"
            tok = ta
        assert eng.position == fresh.position == 33
    finally:
        eng.close()
        fresh.close()


def test_qengine_argument_errors(gpu):
    """Shape, format and part-layout errors are reported by name."""
    import ctypes as C

    from grout_amd._lib import GroutError, Qwen3Config as CConfig, call
    from grout_amd.model import Qwen3Config, QuantWeights

    cfg = configs()["g2"]
    spec, _, _ = qutil.mixed_weights(cfg, PLANS["q4km-tied"], 1, 0.05)
    qw = QuantWeights(cfg, **spec)
    c = CConfig(cfg.num_layers, cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads,
                cfg.num_key_value_heads, cfg.head_dim, cfg.vocab_size, cfg.rms_norm_eps,
                cfg.rope_theta, 16)

    def create(mutate, match):
        w, layers = qw.c_struct()
        mutate(w, layers)
        h = C.c_void_p()
        with pytest.raises(GroutError, match=match):
            call("grout_engine_create_q", C.byref(c), C.byref(w), 0, C.byref(h))

    create(lambda w, L: setattr(L[0], "num_qkv_parts", 0), "num_qkv_parts")
    create(lambda w, L: setattr(L[1].down_proj, "fmt", 11), "format 11")
    create(lambda w, L: setattr(L[0].o_proj, "rows", 128), "o_proj")
    create(lambda w, L: setattr(L[0].qkv[0], "rows", L[0].qkv[0].rows - 1), "qkv parts cover")
    create(lambda w, L: setattr(w.lm_head, "rows", 299), "vocab_size")
    create(lambda w, L: setattr(L[1].gate_up[0], "data", None), "gate_up part")
    # a low-bit matrix whose k is not a multiple of its block size is refused
    odd = Qwen3Config(num_layers=1, hidden_size=384, intermediate_size=512, num_attention_heads=4,
                      num_key_value_heads=2, vocab_size=64)
    plan = {"embed": F16, "lm_head": None, "layers": [{k: F16 for k in Q4KM}]}
    spec2, _, _ = qutil.mixed_weights(odd, plan, 1, 0.05)
    spec2["layers"][0]["q_proj"] = (Q4, np.zeros((odd.q_dim, 384 // 256 * 144), np.uint8))
    with pytest.raises(ValueError, match="not a multiple of 256"):
        QuantWeights(odd, **spec2)


@pytest.mark.parametrize("plan", ["q4km-tied", "mixed-untied", "f16-embed", "q5km-tied"])
def test_gguf_load_vs_quantized_engine_and_oracle(gpu, tmp_path, plan):
    """A GGUF file of the same weights (norms as F32, matrices as their ggml
    blocks) loaded by grout_engine_load gives the engine built from the
    blocks directly, bit for bit, and the oracle's logits."""
    from gguf_util import gguf_bytes, qwen3_meta, qwen3_tensors
    from grout_amd.model import Engine, QuantWeights

    cfg = configs()["g2"]
    spec, host, w64 = qutil.mixed_weights(cfg, PLANS[plan], 13, 0.05)
    path = tmp_path / "qwen3.gguf"
    path.write_bytes(gguf_bytes(qwen3_meta(cfg, eos=3, ctx=64), qwen3_tensors(cfg, spec)))
    print(f"gguf {plan} {path.stat().st_size} bytes", flush=True)
    loaded = Engine.load(str(path))
    direct = Engine.from_quantized(cfg, QuantWeights(cfg, **spec), max_ctx=64)
    orc = Q.Qwen3Oracle(cfg, host, 64, decode_w64=w64)
    assert loaded.meta().max_ctx == 64 and loaded.meta().eos_token_ids == (3,)
    prompt = np.random.default_rng(8).integers(0, cfg.vocab_size, 19)
    try:
        a, b = loaded.prefill(prompt).values, direct.prefill(prompt).values
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        ref, _ = orc.prefill(prompt, nthreads=8)
        tol = check_logits(a, ref, f"gguf {plan} prefill")
        tok = int(np.argmax(a))
        for i in range(3):
            a, b = loaded.decode(tok).values, direct.decode(tok).values
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
            ref, _ = orc.decode(tok, nthreads=8)
            check_logits(a, ref, f"gguf {plan} decode {i}")
            tok = int(np.argmax(a))
    finally:
        loaded.close()
        direct.close()


def test_qengine_qwen3_4b_q4km_shapes_consistency(gpu):
    """Full Qwen3-4B shapes (36 layers, vocab 151936) over random GGUF-block
    weights in a Q4_K_M-style mix (attn_v / ffn_down Q6_K in the first and
    last eighth of the layers and every third between, Q6_K tied embedding):
    the decode step at position n (low-bit GEMVs on the decode-layout
    scales) equals a prefill of n + 1 tokens (dequantized f16 weights
    through the GEMMs) within the engine tolerance, and the device argmax
    equals the host argmax of the same logits."""
    import torch
    from grout_amd.model import Engine, QuantWeights, Qwen3Config

    cfg = Qwen3Config.qwen3_4b()
    L = cfg.num_layers

    def fmts(l):
        hi = Q6 if l < L // 8 or l >= 7 * L // 8 or (l - L // 8) % 3 == 2 else Q4
        return {"q": Q4, "k": Q4, "v": hi, "o": Q4, "gate": Q4, "up": Q4, "down": hi}

    qw = QuantWeights.random(cfg, fmts, embed_fmt=Q6, seed=0)
    eng = Engine.from_quantized(cfg, qw, max_ctx=1024)
    try:
        prompt = [int(t) for t in np.random.default_rng(4).integers(0, cfg.vocab_size, 96)]
        eng.prefill(prompt)
        t = 777
        step = eng.decode(t).values
        full = eng.prefill(prompt + [t]).values
        check_logits(step, full, "q4km 4b decode vs prefill")
        eng.prefill(prompt)
        assert eng.decode_greedy(t) == int(np.argmax(step))
    finally:
        eng.close()
        del qw
        torch.cuda.empty_cache()
