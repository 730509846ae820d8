/*
 * ggml_quant.c -- CPU restatement of the quantized weight formats the
 * reference's low-bit decode reads (TEST INFRASTRUCTURE ONLY: the checker for
 * the HIP quantized GEMVs, never linked by the product).
 *
 * Formats (ggml block layouts, little endian), as dequantized by the
 * reference's dequantize_q8_0 / dequantize_q4k / dequantize_q6k
 * (src/dequant.rs:211-323) and get_scale_min_k4 (src/dequant.rs:325-335):
 *
 *   Q8_0  34 B per 32 weights:  f16 d; int8 q[32];            w = d*q
 *   Q4_K 144 B per 256 weights: f16 d, dmin; u8 scales[12]; u8 qs[128]
 *         sub-block s (32 weights) has 6-bit (sc, m) from scales;
 *         group g (64 weights) = bytes qs[32g .. 32g+31]: low nibble of byte l
 *         is weight 64g+l (sub-block 2g), high nibble weight 64g+32+l
 *         (sub-block 2g+1);                                    w = d*sc*q - dmin*m
 *   Q5_K 176 B per 256 weights: f16 d, dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]
 *         as Q4_K with a fifth bit: weight 64g + l (+32) takes bit 2g (2g+1)
 *         of qh[l] as 16;                                   w = d*sc*q - dmin*m
 *         (src/dequant.rs:255-294)
 *   Q6_K 210 B per 256 weights: u8 ql[128]; u8 qh[64]; int8 sc[16]; f16 d
 *         half n (128 weights), l < 32: 6-bit q = ql nibble | 2 bits of qh,
 *         weights 128n + l + 32i (i = 0..3) use
 *         i=0: ql[64n+l] low,    qh[32n+l] bits 0-1, sc[8n + l/16]
 *         i=1: ql[64n+l+32] low, qh bits 2-3,        sc[8n + l/16 + 2]
 *         i=2: ql[64n+l] high,   qh bits 4-5,        sc[8n + l/16 + 4]
 *         i=3: ql[64n+l+32] high,qh bits 6-7,        sc[8n + l/16 + 6]
 *                                                          w = d*sc*(q - 32)
 * Every product is fp32 in the order the reference writes it.
 *
 * Decode layout (decode != 0): the reference's GPU decode path repacks Q4_K
 * with the per-32 effective scale and min folded and rounded to f16,
 * sc = f16(d * sc6), mn = f16(dmin * m6) (repack_q4k_soa_host,
 * src/loader.rs:437-486), and both its decode GEMV (gemv_q4k_soa_f16,
 * src/kernels.rs:709-803) and its prefill dequant (dequant_q4k_soa_to_f16,
 * src/kernels.rs:1113-1160) compute w = sc * q - mn from those.  Its Q8_0
 * and Q6_K decode layouts keep d and sc as stored, so the two modes agree
 * for them.
 *
 * The GEMV reference is y[n] = sum_k w[n][k] * x[k] over the decode-layout
 * weights, accumulated in fp64 here (the reference accumulates in fp32), so
 * the GPU result differs from this only by fp32 rounding.
 */
#include <stdlib.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

float go_h2f(uint16_t h);
uint16_t go_f2h(float f);

enum { GQ_Q8_0 = 8, GQ_Q4_K = 12, GQ_Q5_K = 13, GQ_Q6_K = 14 };

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* src/dequant.rs:325-335 */
static void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

int go_qblock_bytes(int fmt) {
  return fmt == GQ_Q8_0 ? 34 : fmt == GQ_Q4_K ? 144 : fmt == GQ_Q5_K ? 176 : fmt == GQ_Q6_K ? 210 : -1;
}
int go_qblock_elems(int fmt) { return fmt == GQ_Q8_0 ? 32 : 256; }

static float round_f16(float f) { return go_h2f(go_f2h(f)); }

/* Dequantizes n weights (a multiple of the block size) into fp32; decode
 * selects the decode-layout Q4_K scales. */
static int dequant_mode(int fmt, const uint8_t* blocks, size_t n, float* out, int decode) {
  const int be = go_qblock_elems(fmt), bb = go_qblock_bytes(fmt);
  if (bb < 0 || n % (size_t)be) return -1;
  for (size_t b = 0; b < n / (size_t)be; ++b) {
    const uint8_t* x = blocks + b * (size_t)bb;
    float* y = out + b * (size_t)be;
    if (fmt == GQ_Q8_0) { /* src/dequant.rs:211-221 */
      const float d = go_h2f(rd16(x));
      for (int j = 0; j < 32; ++j) y[j] = (float)(int8_t)x[2 + j] * d;
    } else if (fmt == GQ_Q4_K) { /* src/dequant.rs:223-254 */
      const float d = go_h2f(rd16(x)), dmin = go_h2f(rd16(x + 2));
      const uint8_t* scales = x + 4;
      const uint8_t* qs = x + 16;
      for (int g = 0; g < 4; ++g) {
        int sc, m;
        scale_min_k4(2 * g, scales, &sc, &m);
        float d1 = d * (float)sc, m1 = dmin * (float)m;
        scale_min_k4(2 * g + 1, scales, &sc, &m);
        float d2 = d * (float)sc, m2 = dmin * (float)m;
        if (decode) { /* src/loader.rs:458-461 */
          d1 = round_f16(d1);
          m1 = round_f16(m1);
          d2 = round_f16(d2);
          m2 = round_f16(m2);
        }
        for (int l = 0; l < 32; ++l) {
          y[64 * g + l] = d1 * (float)(qs[32 * g + l] & 0xF) - m1;
          y[64 * g + 32 + l] = d2 * (float)(qs[32 * g + l] >> 4) - m2;
        }
      }
    } else if (fmt == GQ_Q5_K) { /* src/dequant.rs:255-294 (both modes: scales as stored) */
      const float d = go_h2f(rd16(x)), dmin = go_h2f(rd16(x + 2));
      const uint8_t* scales = x + 4;
      const uint8_t* qh = x + 16;
      const uint8_t* qs = x + 48;
      for (int g = 0; g < 4; ++g) {
        int sc, m;
        scale_min_k4(2 * g, scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = dmin * (float)m;
        scale_min_k4(2 * g + 1, scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; ++l) {
          const int q1 = (qs[32 * g + l] & 0xF) + ((qh[l] >> (2 * g)) & 1) * 16;
          const int q2 = (qs[32 * g + l] >> 4) + ((qh[l] >> (2 * g + 1)) & 1) * 16;
          y[64 * g + l] = d1 * (float)q1 - m1;
          y[64 * g + 32 + l] = d2 * (float)q2 - m2;
        }
      }
    } else { /* Q6_K, src/dequant.rs:296-323 */
      const uint8_t* ql = x;
      const uint8_t* qh = x + 128;
      const int8_t* sc = (const int8_t*)(x + 192);
      const float d = go_h2f(rd16(x + 208));
      for (int nh = 0; nh < 2; ++nh) {
        for (int l = 0; l < 32; ++l) {
          const int is = l / 16;
          const uint8_t a = ql[64 * nh + l], bq = ql[64 * nh + l + 32], h = qh[32 * nh + l];
          const int q1 = (int)((a & 0xF) | ((h & 3) << 4)) - 32;
          const int q2 = (int)((bq & 0xF) | (((h >> 2) & 3) << 4)) - 32;
          const int q3 = (int)((a >> 4) | (((h >> 4) & 3) << 4)) - 32;
          const int q4 = (int)((bq >> 4) | (((h >> 6) & 3) << 4)) - 32;
          float* ys = y + 128 * nh;
          ys[l] = d * (float)sc[8 * nh + is] * (float)q1;
          ys[l + 32] = d * (float)sc[8 * nh + is + 2] * (float)q2;
          ys[l + 64] = d * (float)sc[8 * nh + is + 4] * (float)q3;
          ys[l + 96] = d * (float)sc[8 * nh + is + 6] * (float)q4;
        }
      }
    }
  }
  return 0;
}

/* CPU dequantization rule (src/dequant.rs:211-323). */
int go_dequant(int fmt, const uint8_t* blocks, size_t n, float* out) {
  return dequant_mode(fmt, blocks, n, out, 0);
}

/* Decode-layout dequantization (Q4_K with f16 effective scales). */
int go_dequant_decode(int fmt, const uint8_t* blocks, size_t n, float* out) {
  return dequant_mode(fmt, blocks, n, out, 1);
}

/* y[r] = sum_k w[r][k] * x[k] (fp64) over the decode-layout weights of rows
 * of K weights stored as ggml blocks, rows contiguous. */
int go_gemv_q(int fmt, const uint8_t* blocks, int N, int K, const uint16_t* x, double* y) {
  const int be = go_qblock_elems(fmt), bb = go_qblock_bytes(fmt);
  if (bb < 0 || K <= 0 || K % be) return -1;
  float* row = (float*)malloc((size_t)K * sizeof(float));
  if (!row) return -2;
  const size_t row_bytes = (size_t)(K / be) * (size_t)bb;
  for (int r = 0; r < N; ++r) {
    dequant_mode(fmt, blocks + (size_t)r * row_bytes, (size_t)K, row, 1);
    double s = 0.0;
    for (int k = 0; k < K; ++k) s += (double)row[k] * (double)go_h2f(x[k]);
    y[r] = s;
  }
  free(row);
  return 0;
}
