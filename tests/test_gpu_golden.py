"""The HIP kernels against the committed golden fixtures (torch float64 from
the same seeded inputs; see tests/test_golden.py for the oracle side): the
benchmark configurations at their full shapes.  Rotated q and written K rows
within one f16 ulp plus the f32-angle slack, the V row bit-exact, attention
within max-abs 1e-2 / mean-abs 1e-3."""
import numpy as np
import pytest
import torch

from gpu_util import assert_close, dev, host, host_f32
from test_golden import GOLD, c1_inputs, c3_inputs, decode_inputs, within_rope

D = 128
pytestmark = pytest.mark.gpu


def test_config1_kernels_vs_golden(gpu):
    Hq, Hkv, pos, kc, vc, qkv, gq, gk = c1_inputs(1024)
    rope = gpu.ops.rope_tables(1024)
    kd, vd = dev(kc), dev(vc)
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    q_rot = gpu.ops.qk_norm_rope_kv_decode(dev(qkv), dev(gq), dev(gk), rope, kd.clone(),
                                           vd.clone(), p, Hq)
    out = gpu.ops.attn_decode_fused(dev(qkv), dev(gq), dev(gk), rope, kd, vd, p, Hq)
    torch.cuda.synchronize()
    within_rope(host(q_rot), GOLD["c1_q_rot"], [pos], "q")
    within_rope(host(kd)[:, pos], GOLD["c1_k_rot"], [pos], "k row")
    assert np.array_equal(host(vd)[:, pos], qkv[(Hq + Hkv) * D:].reshape(Hkv, D))
    assert_close(host_f32(out), GOLD["c1_out"], "config 1 fused decode vs golden")


@pytest.mark.parametrize("tag,Hq,Hkv,ctx,key", [("g2", 32, 8, 4096, "c2_out")] + [
    (f"g4{c}", 64, 8, c, f"c4_out_{c}") for c in (8192, 16384, 32768)])
def test_decode_configs_kernels_vs_golden(gpu, tag, Hq, Hkv, ctx, key):
    q, kc, vc = decode_inputs(tag, Hq, Hkv, ctx)
    p = torch.tensor([ctx - 1], dtype=torch.int32, device="cuda")
    out = gpu.ops.attn_decode(dev(q), dev(kc), dev(vc), p)
    torch.cuda.synchronize()
    assert_close(host_f32(out), GOLD[key], f"{key} vs golden")


def test_config3_kernels_vs_golden(gpu):
    S, Hq, Hkv, q, k, v, gq, gk = c3_inputs()
    rope = gpu.ops.rope_tables(S)
    kd = torch.zeros((Hkv, S, D), dtype=torch.float16, device="cuda")
    vd = torch.zeros_like(kd)
    q_rot = gpu.ops.qk_norm_rope_kv_prefill(dev(q), dev(k), dev(v), dev(gq), dev(gk), rope, kd,
                                            vd, 0)
    out = gpu.ops.fmha_prefill(q_rot, kd, vd, 0)
    torch.cuda.synchronize()
    rows = GOLD["c3_rows"]
    within_rope(host(q_rot)[rows].transpose(1, 0, 2), GOLD["c3_q_rot"].transpose(1, 0, 2), rows,
                "q rows")
    within_rope(host(kd)[:, rows], GOLD["c3_k_rot"].transpose(1, 0, 2), rows, "k rows")
    assert_close(host_f32(out)[rows], GOLD["c3_out"], "config 3 prefill rows vs golden")
