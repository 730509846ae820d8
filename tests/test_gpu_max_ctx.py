"""GPU parity at the largest cache the ABI accepts: GROUT_MAX_CTX positions
per kv head (the limit of the kernels' 32-bit row offsets).

Up to eight kv heads of 1 GiB K and 1 GiB V each, so cache addresses run past
2^32 bytes from the cache base and a head's rows reach 2^30 bytes from its
own base.  On top of that cache, in the order an engine would run them:

* the fused QK-norm/RoPE/KV write of a 40-token prefill ending at the last
  row (q rows and cache rows bit-exact, the row below untouched);
* causal prefill FMHA over those rows in each work-split form (sampled rows
  against the oracle);
* the fused decode step at the last position (cache row bit-exact, output
  against the oracle over all 2^22 positions), and the unfused split + merge
  decode on the oracle's rotated q.

The background of the cache is N(0,1).  Some rows are "spikes" (K x 6,
V x 2): the first and last rows of every decode split (32 or 128 splits), a
few seeded ones, and the rows the test writes (gamma_k ~ U(5,7)).  The
spikes' scores are ~6 times the background's, so both matter to every
output, and outputs stay within about +-5 (where one f16 rounding is at most
2e-3 of the 1e-2 bar).  Measured on the CPU at this size: with 32 splits,
dropping one split's background moves an output by 0.012-0.033, and dropping
the largest spike by 1.5-5.4; with 128 splits a split's background alone
moves it by 0.001-0.008, so there a dropped split shows through the spikes
at its edges."""
import os
import re

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import D, assert_close, dev, host, host_f32, normal

pytestmark = pytest.mark.gpu

_HDR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                    "grout_attn.h")
MAX_CTX = 1 << int(re.search(r"#define GROUT_MAX_CTX \(1 << (\d+)\)", open(_HDR).read()).group(1))


def _say(*a):
    print("[case]", *a, flush=True)


def _host_cache(t: torch.Tensor) -> np.ndarray:
    """Device [Hkv, ctx, D] fp16 -> host uint16, one kv head per copy."""
    out = np.empty(tuple(t.shape), np.uint16)
    for h in range(t.shape[0]):
        out[h] = host(t[h])
    return out


@pytest.mark.parametrize("Hq,Hkv", [(16, 8), (16, 2)])
def test_largest_cache_prefill_and_decode(gpu, monkeypatch, Hq, Hkv):
    """Hkv = 8, G = 2 (16 GiB of K/V, 32 decode splits); Hkv = 2, G = 8 (the
    Qwen3-32B grouping: 8-head prefill blocks, 128 decode splits)."""
    S = 40
    pos0, last = MAX_CTX - S, MAX_CTX - 1
    _say("largest cache", Hq, Hkv, MAX_CTX, "positions, prefill", pos0, "..", last)
    g = torch.Generator(device="cuda").manual_seed(2222)
    n_split = gpu.ops.default_splits(MAX_CTX, Hq, Hkv)
    assert n_split == 256 // Hkv and MAX_CTX % n_split == 0
    per = MAX_CTX // n_split
    rng = np.random.default_rng(2222)
    spikes = np.unique(np.r_[0, 1, np.arange(1, n_split) * per - 1, np.arange(1, n_split) * per,
                             rng.integers(2, pos0 - 1, 24), pos0 - 1])
    idx = torch.from_numpy(spikes).cuda()
    kc_d = torch.empty((Hkv, MAX_CTX, D), dtype=torch.float16, device="cuda")
    vc_d = torch.empty_like(kc_d)
    for h in range(Hkv):  # one 2^29-element head at a time
        kc_d[h].normal_(0.0, 1.0, generator=g)
        vc_d[h].normal_(0.0, 1.0, generator=g)
        kc_d[h, idx] = (6.0 * torch.randn((len(spikes), D), generator=g, device="cuda")).half()
        vc_d[h, idx] = (2.0 * torch.randn((len(spikes), D), generator=g, device="cuda")).half()
    torch.cuda.synchronize()
    kc, vc = _host_cache(kc_d), _host_cache(vc_d)
    _say("caches on the host")

    # RoPE rows pos0..last only (the kernels read the rows of the positions
    # they write); the rest of both tables stays zero.
    cr, sr = O.rope_rows(pos0, S, D, 1e6)
    cos, sin = np.zeros((MAX_CTX, D // 2), np.float32), np.zeros((MAX_CTX, D // 2), np.float32)
    cos[pos0:], sin[pos0:] = cr, sr
    cos_d = torch.zeros((MAX_CTX, D // 2), dtype=torch.float32, device="cuda")
    sin_d = torch.zeros_like(cos_d)
    cos_d[pos0:], sin_d[pos0:] = torch.from_numpy(cr).cuda(), torch.from_numpy(sr).cuda()
    rope = (cos_d, sin_d)

    q_in, k_in, v_in = normal("mq", (S, Hq, D)), normal("mk", (S, Hkv, D)), normal("mv", (S, Hkv, D))
    gq = O.fill_uniform_f16(O.seed_for("mgq"), 0.8, 1.2, D)
    gk = O.fill_uniform_f16(O.seed_for("mgk"), 5.0, 7.0, D)

    # fused norm/RoPE/KV write of the prefill rows
    q_ref = O.qk_norm_rope_kv_prefill(q_in, k_in, v_in, gq, gk, cos, sin, kc, vc, pos0, 1e-6)
    q_out = gpu.ops.qk_norm_rope_kv_prefill(dev(q_in), dev(k_in), dev(v_in), dev(gq), dev(gk),
                                            rope, kc_d, vc_d, pos0)
    torch.cuda.synchronize()
    assert np.array_equal(host(q_out), q_ref), "rotated q differs"
    assert np.array_equal(host(kc_d[:, pos0 - 1:]), kc[:, pos0 - 1:]), "k rows differ"
    assert np.array_equal(host(vc_d[:, pos0 - 1:]), vc[:, pos0 - 1:]), "v rows differ"
    _say("prefill write bit-exact")

    # prefill FMHA: the first and last rows of the block (pos0 + 1 and 2^22 keys)
    rows = np.array([0, S - 1])
    ref = O.attention_prefill_rows(q_ref, kc, vc, pos0, rows=rows, nthreads=16)
    for form, env in (("default", {}),
                      ("128-row", {"GROUT_FMHA_PREFILL_WAVE_ROWS": "32"}),
                      ("shared", {"GROUT_FMHA_PREFILL_SHARED": "1"})):
        for k in ("GROUT_FMHA_PREFILL_WAVE_ROWS", "GROUT_FMHA_PREFILL_SHARED"):
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        _say("prefill FMHA", form, gpu.ops.prefill_plan(S, Hq, Hkv))
        out = gpu.ops.fmha_prefill(q_out, kc_d, vc_d, pos0)
        torch.cuda.synchronize()
        assert_close(host_f32(out)[rows], ref, f"prefill {form} at the largest cache")
    print(f"[largest cache] max |prefill ref| = {np.abs(ref).max():.3f}", flush=True)

    # decode at the last position: the fused step, then split + merge on the oracle's q
    qkv = normal("mqkv", ((Hq + 2 * Hkv) * D,))
    q_dec = O.qk_norm_rope_kv_decode(qkv, gq, gk, cos, sin, kc, vc, last, Hq, Hkv, 1e-6)
    ref = O.attention_decode(q_dec, kc, vc, last, nthreads=16)
    p = torch.tensor([last], dtype=torch.int32, device="cuda")
    out = gpu.ops.attn_decode_fused(dev(qkv), dev(gq), dev(gk), rope, kc_d, vc_d, p, Hq)
    torch.cuda.synchronize()
    assert np.array_equal(host(kc_d[:, last - 1:]), kc[:, last - 1:]), "decode k row differs"
    assert np.array_equal(host(vc_d[:, last - 1:]), vc[:, last - 1:]), "decode v row differs"
    assert_close(host_f32(out), ref, "fused decode at the last position")
    out = gpu.ops.attn_decode(dev(q_dec), kc_d, vc_d, p)
    torch.cuda.synchronize()
    assert_close(host_f32(out), ref, "split + merge decode at the last position")
    print(f"[largest cache] max |decode ref| = {np.abs(ref).max():.3f}", flush=True)
    del kc_d, vc_d, cos_d, sin_d
    torch.cuda.empty_cache()
