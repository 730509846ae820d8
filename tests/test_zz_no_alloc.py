"""grout_attn_decode_noalloc: the split partials live in the library's static
device scratch instead of a caller workspace.  Its output must equal
grout_attn_decode's with the same split count bit for bit (same kernels),
call after call on the shared scratch, and stay within the attention
tolerance of the CPU oracle."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import D, assert_close, dev, host_f32, normal


def _noalloc(L, q, kc, vc, out, pos, Hq, Hkv, max_ctx, ns):
    P = lambda t: C.c_void_p(t.data_ptr())
    s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    return L.grout_attn_decode_noalloc(P(q), P(kc), P(vc), P(out), P(pos), Hq, Hkv, D, max_ctx,
                                       max_ctx * D, ns, 1.0 / np.sqrt(D), s)


def test_noalloc_rejects_oversized_scratch_without_gpu():
    """The size check runs before any device call: 64 q heads over 8 kv heads
    at 200 splits need 6.6 MB > the 4 MiB static scratch."""
    import grout_amd
    from grout_amd import _lib

    L = grout_amd.lib()
    buf = (C.c_char * 8192)()
    p = C.c_void_p((C.addressof(buf) + 255) & ~255)
    assert L.grout_attn_decode_workspace_bytes(64, 8, 128, 200) > (4 << 20)
    rc = L.grout_attn_decode_noalloc(p, p, p, p, p, 64, 8, 128, 32768, 32768 * 128, 200, 0.088,
                                     None)
    assert rc == -1 and "static scratch" in _lib.last_error()
    rc = L.grout_attn_decode_noalloc(p, p, p, p, None, 64, 8, 128, 32768, 32768 * 128, 32, 0.088,
                                     None)
    assert rc == -1 and "d_pos" in _lib.last_error()


@pytest.mark.gpu
def test_noalloc_decode_equals_workspace_decode(gpu):
    L = gpu.lib()
    # a Qwen3-32B layer at 32k context, then a smaller call (fewer heads,
    # shorter context, fewer splits) on the same scratch
    cases = [(64, 8, 32768, 32768, 32), (32, 8, 1000, 4096, 7), (16, 1, 300, 512, 0)]
    for Hq, Hkv, ctx, max_ctx, ns in cases:
        print("[case] noalloc", Hq, Hkv, ctx, max_ctx, ns, flush=True)
        q = normal(f"na{Hq}q", (Hq, D))
        kc, vc = normal(f"na{Hq}k", (Hkv, max_ctx, D)), normal(f"na{Hq}v", (Hkv, max_ctx, D))
        qd, kd, vd = dev(q), dev(kc), dev(vc)
        p = torch.tensor([ctx - 1], dtype=torch.int32, device="cuda")
        ref = gpu.ops.attn_decode(qd, kd, vd, p, num_splits=ns or None)
        out = torch.full_like(qd, float("nan"))
        assert _noalloc(L, qd, kd, vd, out, p, Hq, Hkv, max_ctx, ns) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"noalloc differs from grout_attn_decode: {Hq} {ctx} {ns}"
        assert_close(host_f32(out), O.attention_decode(q, kc, vc, ctx - 1, nthreads=16),
                     f"noalloc Hq={Hq} ctx={ctx}")
