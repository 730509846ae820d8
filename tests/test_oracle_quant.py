"""CPU pins of the ggml dequantization oracle (oracle/ggml_quant.c), in both
its CPU-rule and decode-layout modes.

Each format is checked against blocks built by an independent *encoder*
written here from the published block layout (the inverse of the decode: a
wrong bit position, nibble order, scale index or sign in the oracle makes the
decoded weights differ from the values that were encoded), with the expected
weights computed in numpy float32 in the reference's operation order."""
import numpy as np
import pytest

import oracle as O

F16 = np.float16


def f16b(v):
    return np.array([v], F16).view(np.uint16)[0]


def enc_q8_0(d, q):
    """One Q8_0 block: f16 d then 32 int8."""
    b = np.zeros(34, np.uint8)
    b[0:2] = np.array([f16b(d)], np.uint16).view(np.uint8)
    b[2:] = np.asarray(q, np.int8).view(np.uint8)
    return b


def pack_scale_min_k4(sc, m):
    """12 bytes holding eight 6-bit (scale, min) pairs: pairs 0-3 in the low 6
    bits of bytes 0-3 / 4-7, pairs 4-7 split into a low nibble (bytes 8-11)
    and two high bits (bits 6-7 of bytes 0-3 / 4-7)."""
    out = np.zeros(12, np.uint8)
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    return out


def enc_q4_k(d, dmin, sc, m, q):
    """q: 256 values in [0, 15] in weight order."""
    b = np.zeros(144, np.uint8)
    b[0:4] = np.array([f16b(d), f16b(dmin)], np.uint16).view(np.uint8)
    b[4:16] = pack_scale_min_k4(sc, m)
    q = np.asarray(q)
    for g in range(4):
        lo, hi = q[64 * g:64 * g + 32], q[64 * g + 32:64 * g + 64]
        b[16 + 32 * g:16 + 32 * g + 32] = (lo | (hi << 4)).astype(np.uint8)
    return b


def enc_q5_k(d, dmin, sc, m, q):
    """q: 256 values in [0, 31] in weight order; bit 4 of weight 64g + l
    (+32) goes to bit 2g (2g+1) of qh[l]."""
    b = np.zeros(176, np.uint8)
    b[0:4] = np.array([f16b(d), f16b(dmin)], np.uint16).view(np.uint8)
    b[4:16] = pack_scale_min_k4(sc, m)
    q = np.asarray(q)
    qh = np.zeros(32, np.uint8)
    for g in range(4):
        lo, hi = q[64 * g:64 * g + 32], q[64 * g + 32:64 * g + 64]
        b[48 + 32 * g:48 + 32 * g + 32] = ((lo & 15) | ((hi & 15) << 4)).astype(np.uint8)
        qh |= ((lo >> 4) << (2 * g)).astype(np.uint8) | ((hi >> 4) << (2 * g + 1)).astype(np.uint8)
    b[16:48] = qh
    return b


def enc_q6_k(d, sc, q):
    """q: 256 6-bit values in [0, 63] in weight order (weight = d*sc*(q-32))."""
    b = np.zeros(210, np.uint8)
    q = np.asarray(q)
    ql, qh = b[0:128], b[128:192]
    for n in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q[128 * n + l + 32 * i] for i in range(4))
            ql[64 * n + l] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            ql[64 * n + l + 32] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            qh[32 * n + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = np.array([f16b(d)], np.uint16).view(np.uint8)
    return b


def test_block_geometry():
    assert O.qblock(O.Q8_0) == (32, 34)
    assert O.qblock(O.Q4_K) == (256, 144)
    assert O.qblock(O.Q5_K) == (256, 176)
    assert O.qblock(O.Q6_K) == (256, 210)


def test_q8_0_closed_form():
    q = np.arange(-16, 16, dtype=np.int8) * 7 // 2
    got = O.dequant(O.Q8_0, enc_q8_0(0.5, q), 32)
    assert np.array_equal(got, q.astype(np.float32) * np.float32(0.5))
    q = np.array([-128, 127] + [0] * 30, np.int8)
    got = O.dequant(O.Q8_0, enc_q8_0(-0.0078125, q), 32)
    assert got[0] == 1.0 and got[1] == np.float32(-0.9921875)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q4_k_against_encoder(seed):
    rng = np.random.default_rng(seed)
    d, dmin = F16(rng.uniform(1e-3, 0.1)), F16(rng.uniform(1e-3, 0.1))
    sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    sc[7], m[4] = 63, 63  # top bits of both halves of the packing
    q = rng.integers(0, 16, 256)
    got = O.dequant(O.Q4_K, enc_q4_k(d, dmin, sc, m, q), 256)
    f32 = np.float32
    s = np.repeat(sc, 32).astype(f32)
    mm = np.repeat(m, 32).astype(f32)
    want = (f32(d) * s) * q.astype(f32) - f32(dmin) * mm
    assert np.array_equal(got, want.astype(f32))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q4_k_decode_layout_against_encoder(seed):
    """Decode layout: effective scale f16(d * sc) and min f16(dmin * m)."""
    rng = np.random.default_rng(20 + seed)
    d, dmin = F16(rng.uniform(1e-3, 0.1)), F16(rng.uniform(1e-3, 0.1))
    sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    sc[5], m[6] = 63, 63
    q = rng.integers(0, 16, 256)
    blk = enc_q4_k(d, dmin, sc, m, q)
    got = O.dequant(O.Q4_K, blk, 256, decode=True)
    f32 = np.float32
    s_eff = (f32(d) * sc.astype(f32)).astype(F16).astype(f32)
    m_eff = (f32(dmin) * m.astype(f32)).astype(F16).astype(f32)
    want = np.repeat(s_eff, 32) * q.astype(f32) - np.repeat(m_eff, 32)
    assert np.array_equal(got, want.astype(f32))
    # the rounding is visible: the CPU rule differs somewhere in the block
    assert not np.array_equal(got, O.dequant(O.Q4_K, blk, 256))
    # Q8_0 and Q6_K: both modes agree
    b8 = enc_q8_0(0.37, rng.integers(-128, 128, 32))
    assert np.array_equal(O.dequant(O.Q8_0, b8, 32, decode=True), O.dequant(O.Q8_0, b8, 32))
    b6 = enc_q6_k(F16(0.0123), rng.integers(-128, 128, 16), rng.integers(0, 64, 256))
    assert np.array_equal(O.dequant(O.Q6_K, b6, 256, decode=True), O.dequant(O.Q6_K, b6, 256))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q5_k_against_encoder(seed):
    rng = np.random.default_rng(30 + seed)
    d, dmin = F16(rng.uniform(1e-3, 0.1)), F16(rng.uniform(1e-3, 0.1))
    sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    sc[6], m[5] = 63, 63
    q = rng.integers(0, 32, 256)
    q[:4] = [0, 31, 16, 15]
    blk = enc_q5_k(d, dmin, sc, m, q)
    f32 = np.float32
    want = (f32(d) * np.repeat(sc, 32).astype(f32)) * q.astype(f32) - \
        f32(dmin) * np.repeat(m, 32).astype(f32)
    for decode in (False, True):  # both modes: the reference keeps Q5_K scales as stored
        assert np.array_equal(O.dequant(O.Q5_K, blk, 256, decode=decode), want.astype(f32))


@pytest.mark.parametrize("seed", [0, 1])
def test_q6_k_against_encoder(seed):
    rng = np.random.default_rng(10 + seed)
    d = F16(rng.uniform(1e-3, 0.05))
    sc = rng.integers(-128, 128, 16)
    q = rng.integers(0, 64, 256)
    q[:4] = [0, 63, 32, 31]
    got = O.dequant(O.Q6_K, enc_q6_k(d, sc, q), 256)
    f32 = np.float32
    s = np.repeat(sc, 16).astype(f32)  # 16 weights share a scale, in weight order
    want = (f32(d) * s) * (q - 32).astype(f32)
    assert np.array_equal(got, want.astype(f32))


def test_gemv_q_is_dequant_times_x():
    rng = np.random.default_rng(3)
    N, K = 5, 512
    rows = [np.concatenate([enc_q4_k(F16(0.01), F16(0.02), rng.integers(0, 64, 8),
                                     rng.integers(0, 64, 8), rng.integers(0, 16, 256))
                            for _ in range(K // 256)]) for _ in range(N)]
    blocks = np.stack(rows)
    x = rng.standard_normal(K).astype(F16).view(np.uint16)
    w = O.dequant(O.Q4_K, blocks, N * K, decode=True).reshape(N, K).astype(np.float64)
    want = w @ O.h2f(x).astype(np.float64)
    assert np.allclose(O.gemv_q(O.Q4_K, blocks, N, K, x), want, rtol=0, atol=1e-12)


def test_bad_sizes_are_rejected():
    with pytest.raises(ValueError):
        O.dequant(O.Q4_K, np.zeros(144, np.uint8), 100)
    with pytest.raises(ValueError):
        O.dequant(3, np.zeros(144, np.uint8), 256)


@pytest.mark.parametrize("fmt,bound", [(O.Q8_0, 0.01), (O.Q4_K, 0.1), (O.Q5_K, 0.05),
                                       (O.Q6_K, 0.03)])
def test_test_quantizer_round_trip(fmt, bound):
    """tests/qutil.py's quantizer (used to build engine test weights) decodes,
    through the oracle, to within its quantization noise of the input."""
    import qutil

    w = (np.random.default_rng(fmt).standard_normal((6, 1024)) * 0.05).astype(np.float32)
    b = qutil.quantize(fmt, w)
    be, bb = O.qblock(fmt)
    assert b.shape == (6, 1024 // be * bb)
    d = O.dequant(fmt, b, w.size).reshape(w.shape)
    assert np.sqrt(((d - w) ** 2).mean() / (w ** 2).mean()) < bound
