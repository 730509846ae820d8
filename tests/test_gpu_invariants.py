"""Closed forms and invariants of attention, checked on the GPU kernels
directly (no oracle in the loop): whatever the oracle says, these hold for
softmax attention by construction.

* V = c everywhere: every output is c;
* K constant: uniform weights, so output = mean of V over the visible
  positions (float64 numpy mean of the fp16 V rows);
* a context of one position: output = v_0;
* q = lambda * k_j with lambda = 8: the weight of position j dominates by
  e^60 or more, so output = v_j for every query that sees j;
* GQA == MHA with each kv head repeated G times (the kernels' head grouping
  changes, the math does not);
* the split count of decode changes nothing beyond one f16 ulp;
* the norm/RoPE kernel: position 0 is the identity, RoPE keeps pair norms and
  relative positions, RMSNorm ignores an exact 4x scale.

Decode runs with one, several and the default number of splits (and the
fused norm/RoPE/KV layer for the first two forms, with the cache row it writes
taken from the kernel itself); prefill runs in every work-split form."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import D, assert_close, dev, host, host_f32, normal

pytestmark = pytest.mark.gpu

PREFILL_FORMS = {
    "rows64": {"GROUT_FMHA_PREFILL_SHARED": "0", "GROUT_FMHA_PREFILL_WAVE_ROWS": "16"},
    "rows32": {"GROUT_FMHA_PREFILL_SHARED": "0", "GROUT_FMHA_PREFILL_WAVE_ROWS": "32"},
    "rows32_paired": {"GROUT_FMHA_PREFILL_SHARED": "0", "GROUT_FMHA_PREFILL_WAVE_ROWS": "32",
                      "GROUT_FMHA_PREFILL_PAIRED": "1"},
    "shared": {"GROUT_FMHA_PREFILL_SHARED": "1", "GROUT_FMHA_PREFILL_PAIRED": "0"},
    "shared_paired": {"GROUT_FMHA_PREFILL_SHARED": "1", "GROUT_FMHA_PREFILL_PAIRED": "1"},
}


def _say(*a):
    print("[case]", *a, flush=True)


def _h(x: float) -> np.uint16:
    return np.float16(x).view(np.uint16)


def _f64(a16: np.ndarray) -> np.ndarray:
    return a16.view(np.float16).astype(np.float64)


def _decode(gpu, q, kc, vc, pos, splits):
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    out = gpu.ops.attn_decode(dev(q), dev(kc), dev(vc), p, num_splits=splits)
    torch.cuda.synchronize()
    return host_f32(out)


def _prefill(gpu, q, kc, vc, pos0):
    out = gpu.ops.fmha_prefill(dev(q), dev(kc), dev(vc), pos0)
    torch.cuda.synchronize()
    return host_f32(out)


@pytest.mark.parametrize("splits", [1, 7, None])
def test_decode_closed_forms(gpu, splits):
    Hq, Hkv, max_ctx, pos = 32, 8, 1024, 700
    G = Hq // Hkv
    _say("decode closed forms", Hq, Hkv, pos, splits)
    q = normal("iq", (Hq, D))
    kc, vc = normal("ik", (Hkv, max_ctx, D)), normal("iv", (Hkv, max_ctx, D))
    # V = c
    out = _decode(gpu, q, kc, np.full_like(vc, _h(0.375)), pos, splits)
    assert np.max(np.abs(out - 0.375)) <= 2.0**-12, "V = c"
    # K constant: the mean of V over positions 0..pos
    out = _decode(gpu, q, np.full_like(kc, _h(0.5)), vc, pos, splits)
    mean_v = np.repeat(_f64(vc[:, :pos + 1]).mean(1), G, 0)
    assert_close(out, mean_v, f"decode K const, splits={splits}")
    # one position
    out = _decode(gpu, q, kc, vc, 0, splits)
    assert np.array_equal(out, np.repeat(_f64(vc[:, 0]), G, 0).astype(np.float32)), "ctx = 1"
    # q = 8 k_j: position j takes all the weight
    j = 123
    qj = (np.repeat(_f64(kc[:, j]), G, 0) * 8.0).astype(np.float16).view(np.uint16)
    out = _decode(gpu, qj, kc, vc, pos, splits)
    assert_close(out, np.repeat(_f64(vc[:, j]), G, 0), f"decode q = 8 k_j, splits={splits}")


@pytest.mark.parametrize("splits", [1, 7])
def test_fused_decode_closed_forms(gpu, splits):
    """The fused layer writes cache row pos from its own inputs first; the
    closed forms then hold over rows 0..pos as the kernel left them."""
    Hq, Hkv, max_ctx, pos = 32, 8, 1024, 700
    G = Hq // Hkv
    _say("fused decode closed forms", Hq, Hkv, pos, splits)
    qkv = normal("ifqkv", ((Hq + 2 * Hkv) * D,))
    gq = gk = O.fill_uniform_f16(O.seed_for("ifg"), 0.8, 1.2, D)
    rope = gpu.ops.rope_tables(max_ctx)
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    # V = c in the cache and in the new row
    qkv_c = qkv.copy()
    qkv_c[(Hq + Hkv) * D:] = _h(0.375)
    kc, vc = dev(normal("ifk", (Hkv, max_ctx, D))), dev(np.full((Hkv, max_ctx, D), _h(0.375)))
    out = gpu.ops.attn_decode_fused(dev(qkv_c), dev(gq), dev(gk), rope, kc, vc, p, Hq,
                                    num_splits=splits)
    torch.cuda.synchronize()
    assert np.max(np.abs(host_f32(out) - 0.375)) <= 2.0**-12, "fused V = c"
    # K constant in the cache: the new row's K differs, so compare with the
    # exact softmax over the cache as the kernel wrote it
    kc = dev(np.full((Hkv, max_ctx, D), _h(0.5)))
    vc = dev(normal("ifv", (Hkv, max_ctx, D)))
    out = gpu.ops.attn_decode_fused(dev(qkv), dev(gq), dev(gk), rope, kc, vc, p, Hq,
                                    num_splits=splits)
    q_rot = gpu.ops.qk_norm_rope_kv_decode(dev(qkv), dev(gq), dev(gk), rope, kc.clone(),
                                           vc.clone(), p, Hq)
    torch.cuda.synchronize()
    kf, vf = _f64(host(kc)[:, :pos + 1]), _f64(host(vc)[:, :pos + 1])
    qf = _f64(host(q_rot)).reshape(Hkv, G, D)
    s = np.einsum("hgd,hnd->hgn", qf, kf) / np.sqrt(D)
    w = np.exp(s - s.max(-1, keepdims=True))
    ref = (np.einsum("hgn,hnd->hgd", w, vf) / w.sum(-1)[..., None]).reshape(Hq, D)
    assert_close(host_f32(out), ref, f"fused decode K const, splits={splits}")


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (64, 8), (16, 2)])
def test_decode_gqa_equals_mha(gpu, Hq, Hkv):
    G = Hq // Hkv
    max_ctx, pos = 2048, 1500
    _say("decode gqa == mha", Hq, Hkv, pos)
    q = normal("gq", (Hq, D))
    kc, vc = normal("gk", (Hkv, max_ctx, D)), normal("gv", (Hkv, max_ctx, D))
    gqa = _decode(gpu, q, kc, vc, pos, None)
    mha = _decode(gpu, q, np.repeat(kc, G, 0), np.repeat(vc, G, 0), pos, None)
    assert np.max(np.abs(gqa - mha)) <= 2e-3 and np.mean(np.abs(gqa - mha)) <= 2e-4


@pytest.mark.parametrize("form", sorted(PREFILL_FORMS))
def test_prefill_closed_forms(gpu, monkeypatch, form):
    for k, v in PREFILL_FORMS[form].items():
        monkeypatch.setenv(k, v)
    S, Hq, Hkv, pos0 = 600, 32, 8, 37
    G = Hq // Hkv
    max_ctx = pos0 + S
    _say("prefill closed forms", form, S, Hq, Hkv, pos0)
    q = normal("pq", (S, Hq, D))
    kc, vc = normal("pk", (Hkv, max_ctx, D)), normal("pv", (Hkv, max_ctx, D))
    # V = c
    out = _prefill(gpu, q, kc, np.full_like(vc, _h(0.375)), pos0)
    assert np.max(np.abs(out - 0.375)) <= 2.0**-12, "V = c"
    # K constant: row r sees positions 0..pos0+r, the mean of their V
    out = _prefill(gpu, q, np.full_like(kc, _h(0.5)), vc, pos0)
    csum = np.cumsum(_f64(vc), axis=1)[:, pos0:pos0 + S]             # [Hkv, S, D]
    mean_v = csum / (pos0 + 1 + np.arange(S))[None, :, None]
    assert_close(out, np.repeat(mean_v.transpose(1, 0, 2), G, 1), f"prefill K const {form}")
    # q = 8 k_j for every row: rows that see j (pos0 + r >= j) return v_j
    j = 200
    qj = np.broadcast_to(np.repeat(_f64(kc[:, j]), G, 0) * 8.0, (S, Hq, D))
    out = _prefill(gpu, qj.astype(np.float16).view(np.uint16), kc, vc, pos0)
    r0 = j - pos0
    want = np.broadcast_to(np.repeat(_f64(vc[:, j]), G, 0), (S - r0, Hq, D))
    assert_close(out[r0:], want, f"prefill q = 8 k_j {form}")
    # one position: pos0 = 0, row 0 sees only v_0
    out = _prefill(gpu, q[:1], kc, vc, 0)
    assert np.array_equal(out[0], np.repeat(_f64(vc[:, 0]), G, 0).astype(np.float32)), "ctx = 1"


@pytest.mark.parametrize("form", ["rows64", "rows32", "shared"])
def test_prefill_gqa_equals_mha(gpu, monkeypatch, form):
    for k, v in PREFILL_FORMS[form].items():
        monkeypatch.setenv(k, v)
    S, Hq, Hkv, pos0 = 300, 32, 8, 11
    G = Hq // Hkv
    _say("prefill gqa == mha", form, S, Hq, Hkv, pos0)
    q = normal("mq", (S, Hq, D))
    kc, vc = normal("mk", (Hkv, pos0 + S, D)), normal("mv", (Hkv, pos0 + S, D))
    gqa = _prefill(gpu, q, kc, vc, pos0)
    mha = _prefill(gpu, q, np.repeat(kc, G, 0), np.repeat(vc, G, 0), pos0)
    assert np.max(np.abs(gqa - mha)) <= 2e-3 and np.mean(np.abs(gqa - mha)) <= 2e-4


def test_decode_split_count_invariance(gpu):
    """The same decode with 1, 2, 7, 16, 64 and 200 splits (200 > the 47 tiles
    of 16 positions: empty splits): outputs within one f16 ulp."""
    Hq, Hkv, max_ctx, pos = 32, 8, 1024, 750
    q = normal("sq", (Hq, D))
    kc, vc = normal("sk", (Hkv, max_ctx, D)), normal("sv", (Hkv, max_ctx, D))
    outs = {n: _decode(gpu, q, kc, vc, pos, n) for n in (1, 2, 7, 16, 64, 200)}
    for n, o in outs.items():
        d = np.abs(o - outs[1])
        # one f16 ulp: the f16 P is rounded against each split's own
        # reference point, so about half the outputs round the other way
        assert np.all(d <= 2.0**-10 * np.maximum(np.abs(outs[1]), 2.0**-3)), n


def test_norm_rope_invariants_on_the_kernel(gpu):
    """The fused QK-norm/RoPE prefill kernel on one q row x and one k row y
    repeated at positions 0..S-1 (gamma = 1): position 0 is the identity
    (unit RMS after the norm), every (i, i+64) pair keeps its norm at every
    position, <q(m), k(n)> depends only on m - n, and 4x (exact in f16)
    changes nothing, bit for bit (with eps = 1e-30: a finite eps next to
    the mean square would break the exact scale invariance)."""
    Hq, Hkv, S = 2, 1, 1400
    x, y = normal("rx", (D,)), normal("ry", (D,))
    ones = np.full(D, _h(1.0))
    rope = gpu.ops.rope_tables(S)

    def run(xs, ys):
        q = np.ascontiguousarray(np.broadcast_to(xs, (S, Hq, D)))
        k = np.ascontiguousarray(np.broadcast_to(ys, (S, Hkv, D)))
        kc = torch.zeros((Hkv, S, D), dtype=torch.float16, device="cuda")
        vc = torch.zeros_like(kc)
        qo = gpu.ops.qk_norm_rope_kv_prefill(dev(q), dev(k), dev(np.zeros_like(k)), dev(ones),
                                             dev(ones), rope, kc, vc, 0, eps=1e-30)
        torch.cuda.synchronize()
        return host(qo), host(kc)

    qo16, kc16 = run(x, y)
    qo, ko = _f64(qo16)[:, 0], _f64(kc16)[0]
    assert abs(np.sqrt(np.mean(qo[0] ** 2)) - 1.0) < 2e-3, "unit RMS at position 0"
    pair0 = qo[0, :64] ** 2 + qo[0, 64:] ** 2
    for p in (1, 100, 777, S - 1):
        pair = qo[p, :64] ** 2 + qo[p, 64:] ** 2
        assert np.allclose(pair, pair0, rtol=4e-3, atol=2e-4), p
    d1, d2 = qo[700] @ ko[650], qo[1350] @ ko[1300]
    assert abs(d1 - d2) < 2e-2 * max(1.0, abs(d1)), (d1, d2)
    x4 = (_f64(x) * 4.0).astype(np.float16).view(np.uint16)
    y4 = (_f64(y) * 4.0).astype(np.float16).view(np.uint16)
    qo4, kc4 = run(x4, y4)
    assert np.array_equal(qo4, qo16) and np.array_equal(kc4, kc16), "RMSNorm(4x) == RMSNorm(x)"


def test_repeated_calls_are_bit_identical(gpu, monkeypatch):
    """No kernel here accumulates with atomics or depends on scheduling:
    the same inputs give bit-identical outputs on every call, in every
    prefill work split and decode form (calls interleaved with others)."""
    S, Hq, Hkv, pos0, max_ctx = 700, 32, 8, 20, 1024
    q = dev(normal("dq", (S, Hq, D)))
    kc, vc = dev(normal("dk", (Hkv, max_ctx, D))), dev(normal("dv", (Hkv, max_ctx, D)))
    outs = {}
    for rep in range(2):
        for form in sorted(PREFILL_FORMS):
            for k in ("GROUT_FMHA_PREFILL_SHARED", "GROUT_FMHA_PREFILL_WAVE_ROWS",
                      "GROUT_FMHA_PREFILL_PAIRED"):
                monkeypatch.delenv(k, raising=False)
            for k, v in PREFILL_FORMS[form].items():
                monkeypatch.setenv(k, v)
            outs.setdefault(form, []).append(gpu.ops.fmha_prefill(q, kc, vc, pos0).clone())
        p = torch.tensor([900], dtype=torch.int32, device="cuda")
        for n in (1, 7, None):
            outs.setdefault(f"decode{n}", []).append(
                gpu.ops.attn_decode(q[0], kc, vc, p, num_splits=n).clone())
    torch.cuda.synchronize()
    for name, (a, b) in outs.items():
        assert torch.equal(a, b), name
