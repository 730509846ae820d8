"""GPU parity of the low-bit GEMVs (Q8_0, Q4_K, Q5_K, Q6_K) against the ggml
dequantization oracle, through the C ABI.

Inputs: random ggml blocks (random payload bytes, scales/mins, d and dmin
drawn as f16 in [1e-3, 2e-2]).  The oracle runs in its decode-layout mode
(Q4_K effective scale and min rounded to f16, as the reference's decode
repack holds them).  Bars: the repacked weights dequantize bit-exactly (the
kernel's fp32 dequantization rounded once to f16 equals the oracle's); GEMV
outputs within one f16 ulp plus 1e-5 x sum(|w x| + m |x|) of the fp64 oracle
(fp32 accumulation in another order; for Q4_K and Q5_K the scale and min are
factored out of each 16-weight run, so the min term enters the bound); the SiLU-pair
epilogue within the bound propagated through silu(g) * u plus one ulp."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


def ptr(t):
    return C.c_void_p(t.data_ptr())


def ulp(x):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -14)))
    return 2.0 ** (e - 10)


def call(L, name, *args):
    rc = getattr(L, name)(*args)
    assert rc == 0, f"{name} -> {rc}: {L.grout_last_error().decode()}"


def random_blocks(fmt, n, k, seed, dmax=2e-2):
    be, bb = O.qblock(fmt)
    rng = np.random.default_rng(seed)
    nb = n * (k // be)
    b = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    d = rng.uniform(dmax / 20, dmax, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    if fmt == O.Q8_0:
        b[:, 0:2] = d
    elif fmt in (O.Q4_K, O.Q5_K):
        b[:, 0:2] = d
        b[:, 2:4] = rng.uniform(dmax / 20, dmax, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    else:
        b[:, 208:210] = d
    return b.reshape(n, -1)


def min_term(fmt, blocks, n, k):
    """Per weight |dmin * m| (Q4_K, Q5_K: dequant with every q = 0), else zeros."""
    if fmt not in (O.Q4_K, O.Q5_K):
        return np.zeros((n, k))
    z = blocks.reshape(-1, O.qblock(fmt)[1]).copy()
    z[:, 16:] = 0
    return np.abs(O.dequant(fmt, z, n * k).reshape(n, k).astype(np.float64))


def upload(fmt, blocks, n, k, L):
    raw = torch.from_numpy(np.ascontiguousarray(blocks).reshape(-1)).cuda()
    nbytes = L.grout_qweight_bytes(fmt, n, k)
    assert nbytes > 0
    wq = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    call(L, "grout_qweight_repack", fmt, ptr(raw), n, k, ptr(wq), None)
    return wq


FMTS = [(O.Q8_0, "Q8_0"), (O.Q4_K, "Q4_K"), (O.Q5_K, "Q5_K"), (O.Q6_K, "Q6_K")]


@pytest.mark.parametrize("fmt,name", FMTS)
# 4-row workgroups with 5 / 19 / 8 pieces per lane and the any-K path; 16-row
# workgroups (>= 16384 rows) with a ragged last workgroup, exact and any-K;
# the ffn_down widths of Qwen3-14B (17408, any-K path) and Qwen3-32B (25600,
# 13 pieces per lane in 4 slices) and the largest K (32768, x in 64 KiB of LDS)
@pytest.mark.parametrize("n,k", [(6144, 2560), (2560, 9728), (2560, 4096), (37, 256), (1, 512),
                                 (16400, 2560), (16391, 768), (300, 17408), (300, 25600),
                                 (7, 32768)])
def test_gemv_q_vs_oracle(gpu, fmt, name, n, k):
    L = gpu.lib()
    print(f"gemv_q {name} n={n} k={k}", flush=True)
    blocks = random_blocks(fmt, n, k, seed=n + k + fmt)
    x = np.random.default_rng(k).standard_normal(k).astype(np.float16).view(np.uint16)
    wq = upload(fmt, blocks, n, k, L)
    xd = torch.from_numpy(x.view(np.float16)).cuda()
    y = torch.empty(n, dtype=torch.float16, device="cuda")
    call(L, "grout_gemv_q", fmt, ptr(wq), ptr(xd), ptr(y), n, k, None)
    torch.cuda.synchronize()
    ref = O.gemv_q(fmt, blocks, n, k, x)
    w = O.dequant(fmt, blocks, n * k).reshape(n, k).astype(np.float64)
    xf = O.h2f(x).astype(np.float64)
    mag = (np.abs(w) + min_term(fmt, blocks, n, k)) @ np.abs(xf)
    got = y.cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    print(f"[gemv_q {name}] max_err={err.max():.3e} max_rel_to_mag={np.max(err / mag):.2e}",
          flush=True)
    assert np.all(err <= ulp(ref) + 1e-5 * mag)


@pytest.mark.parametrize("fmt,name", FMTS)
@pytest.mark.parametrize("inter,k", [(1000, 2560), (8203, 2560), (9, 1280)])
def test_gemv_q_silu_pairs_vs_oracle(gpu, fmt, name, inter, k):
    L = gpu.lib()
    print(f"gemv_q_silu {name} inter={inter} k={k}", flush=True)
    # scales small enough that gate / up stay well inside the f16 range
    blocks = random_blocks(fmt, 2 * inter, k, seed=77 + fmt, dmax=4e-4)
    x = (np.random.default_rng(5).standard_normal(k) * 0.5).astype(np.float16).view(np.uint16)
    wq = upload(fmt, blocks, 2 * inter, k, L)
    xd = torch.from_numpy(x.view(np.float16)).cuda()
    y = torch.empty(inter, dtype=torch.float16, device="cuda")
    call(L, "grout_gemv_q_silu_mul", fmt, ptr(wq), ptr(xd), ptr(y), inter, k, None)
    torch.cuda.synchronize()
    gu = O.gemv_q(fmt, blocks, 2 * inter, k, x)
    g16, u16 = gu[:inter].astype(np.float16).astype(np.float64), gu[inter:].astype(np.float16).astype(np.float64)
    ref = (g16 / (1 + np.exp(-g16)) * u16).astype(np.float16).astype(np.float64)
    w = O.dequant(fmt, blocks, 2 * inter * k).reshape(2 * inter, k).astype(np.float64)
    mag = (np.abs(w) + min_term(fmt, blocks, 2 * inter, k)) @ np.abs(O.h2f(x).astype(np.float64))
    tol_p = ulp(gu) + 1e-5 * mag  # bound on each gate / up product
    sig = 1 / (1 + np.exp(-g16))
    dg = np.abs(u16 * sig * (1 + g16 * (1 - sig)))
    tol = dg * tol_p[:inter] + np.abs(g16 * sig) * tol_p[inter:] + 1.5 * ulp(ref) + 1e-7
    err = np.abs(y.cpu().numpy().astype(np.float64) - ref)
    print(f"[gemv_q_silu {name}] max_err={err.max():.3e} |g|max={np.abs(g16).max():.2f}",
          flush=True)
    assert np.all(np.isfinite(ref))
    assert np.all(err <= tol)


@pytest.mark.parametrize("fmt,name", FMTS)
def test_qweight_dequant_bit_exact(gpu, fmt, name):
    """The GPU's dequantization (decode-layout scales, fp32 arithmetic, one
    rounding to f16) equals the oracle's bit for bit."""
    L = gpu.lib()
    n, k = 48, 1024
    blocks = random_blocks(fmt, n, k, seed=3 + fmt)
    wq = upload(fmt, blocks, n, k, L)
    out = torch.empty((n, k), dtype=torch.float16, device="cuda")
    call(L, "grout_qweight_dequant", fmt, ptr(wq), n, k, ptr(out), None)
    torch.cuda.synchronize()
    want = O.dequant(fmt, blocks, n * k, decode=True).reshape(n, k).astype(np.float16)
    got = out.cpu().numpy()
    bad = np.argwhere(got.view(np.uint16) != want.view(np.uint16))
    if len(bad):
        r, c = bad[0]
        print(f"[dequant {name}] {len(bad)} mismatches, first at {r},{c}: got {got[r, c]} "
              f"want {want[r, c]}; cols {np.unique(bad[:, 1] % 256)[:20]}", flush=True)
    assert len(bad) == 0


@pytest.mark.parametrize("fmt,name", FMTS)
def test_qweight_gather_bit_exact(gpu, fmt, name):
    """Embedding rows gathered from the repacked table equal the oracle's CPU
    rule (fp32 scales, one rounding to f16) bit for bit; ids past the end
    read the last row."""
    L = gpu.lib()
    n, k = 40, 768
    blocks = random_blocks(fmt, n, k, seed=11 + fmt)
    wq = upload(fmt, blocks, n, k, L)
    ids = np.array([3, 0, 39, 17, 3, 1000], np.uint32)
    idd = torch.from_numpy(ids.view(np.int32)).cuda()
    out = torch.empty((len(ids), k), dtype=torch.float16, device="cuda")
    call(L, "grout_qweight_gather", fmt, ptr(wq), n, k, ptr(idd), len(ids), ptr(out), None)
    torch.cuda.synchronize()
    table = O.dequant(fmt, blocks, n * k).reshape(n, k).astype(np.float16)
    want = table[np.minimum(ids, n - 1)]
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want.view(np.uint16))


def test_quant_argument_errors(gpu):
    from grout_amd._lib import GroutError, call as lcall

    L = gpu.lib()
    assert L.grout_qweight_bytes(O.Q4_K, 10, 300) == 0   # k not a multiple of 256
    assert L.grout_qweight_bytes(O.Q4_K, 10, 32768) > 0
    assert L.grout_qweight_bytes(O.Q4_K, 10, 32768 + 256) == 0  # x no longer fits in LDS
    assert L.grout_qweight_bytes(3, 10, 256) == 0         # not a supported format
    buf = torch.empty(1 << 16, dtype=torch.uint8, device="cuda")
    with pytest.raises(GroutError, match="multiple of the block size"):
        lcall("grout_gemv_q", O.Q6_K, ptr(buf), ptr(buf), ptr(buf), 4, 100, None)
    with pytest.raises(GroutError, match="Q8_0"):
        lcall("grout_gemv_q", 2, ptr(buf), ptr(buf), ptr(buf), 4, 256, None)


@pytest.mark.parametrize("fmt,name", FMTS)
@pytest.mark.parametrize("n,k,silu,add", [(6144, 2560, False, True), (2560, 2560, False, False),
                                          (9728, 2560, True, True), (16400, 2560, False, True),
                                          (37, 256, False, True), (40, 256, True, False)])
def test_gemv_q_rms_norm_vs_oracle(gpu, fmt, name, n, k, silu, add):
    """Norm folded into the low-bit GEMV: x' as the oracle's (add_)rms_norm
    within one f16 ulp per element (another fp32 summation order), so the
    bound adds 2^-10 * sum |w x'|; residual_out bit-exact."""
    from oracle import qwen3 as Q

    L = gpu.lib()
    rows = 2 * n if silu else n
    print(f"gemv_q_rms_norm {name} n={n} k={k} silu={silu} add={add}", flush=True)
    blocks = random_blocks(fmt, rows, k, seed=rows + k + fmt, dmax=4e-4 if silu else 2e-2)
    rng = np.random.default_rng(k + n)
    x = rng.standard_normal(k).astype(np.float16).view(np.uint16)
    r = rng.standard_normal(k).astype(np.float16).view(np.uint16)
    g = rng.uniform(0.5, 1.5, k).astype(np.float16).view(np.uint16)
    wq = upload(fmt, blocks, rows, k, L)
    xd, rd, gd = (torch.from_numpy(a.view(np.float16)).cuda() for a in (x, r, g))
    ro = torch.zeros(k, dtype=torch.float16, device="cuda")
    y = torch.empty(n, dtype=torch.float16, device="cuda")
    fn = "grout_gemv_q_rms_norm_silu_mul" if silu else "grout_gemv_q_rms_norm"
    call(L, fn, fmt, ptr(wq), ptr(rd) if add else None, ptr(xd), ptr(gd), ptr(ro) if add else None,
         ptr(y), n, k, C.c_float(1e-6), None)
    torch.cuda.synchronize()
    if add:
        xn, c = Q.add_rms_norm(r[None], x[None], g, 1e-6)
        assert np.array_equal(ro.cpu().numpy().view(np.uint16), c[0])
    else:
        xn = Q.rms_norm(x[None], g, 1e-6)
    xn = xn[0]
    gu = O.gemv_q(fmt, blocks, rows, k, xn)
    w = O.dequant(fmt, blocks, rows * k, decode=True).reshape(rows, k).astype(np.float64)
    mag = (np.abs(w) + min_term(fmt, blocks, rows, k)) @ np.abs(O.h2f(xn).astype(np.float64))
    tol_p = ulp(gu) + 1e-5 * mag + 2.0 ** -10 * mag
    got = y.cpu().numpy().astype(np.float64)
    if silu:
        g16 = gu[:n].astype(np.float16).astype(np.float64)
        u16 = gu[n:].astype(np.float16).astype(np.float64)
        ref = (g16 / (1 + np.exp(-g16)) * u16).astype(np.float16).astype(np.float64)
        sig = 1 / (1 + np.exp(-g16))
        tol = np.abs(u16 * sig * (1 + g16 * (1 - sig))) * tol_p[:n] + np.abs(g16 * sig) * tol_p[n:] \
            + 1.5 * ulp(ref) + 1e-7
    else:
        ref, tol = gu, tol_p
    err = np.abs(got - ref)
    print(f"[gemv_q_rms_norm {name}] max_err={err.max():.3e}", flush=True)
    assert np.all(err <= tol)
