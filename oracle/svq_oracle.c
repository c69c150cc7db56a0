/*
 * svq_oracle.c - C restatement of the GGUF SoA decode and GEMV (CPU).
 *
 * TEST INFRASTRUCTURE ONLY: the checker, loaded by tests/ and bench.py's
 * CPU-baseline leg through ctypes; the product never links it.
 *
 * Follows the reference's quantization.py:
 *   svqo_codes      _block_values, quantization.py:34-47
 *   svqo_dequant    dequantize_soa, quantization.py:93-105 (exact fp32 product)
 *   svqo_gemv_f64   _soa_gemv semantics, quantization.py:171-229, evaluated in
 *                   double: y[m,n] = sum_k x[m,k] W[n,k] + bias[n]
 * fp16 is converted by bit manipulation (no compiler half type), so this file
 * is an implementation independent of numpy's and of the GPU's conversions.
 */
#include <stdint.h>
#include <string.h>

static int payload_bytes(int qtype) {
  return qtype == 4 ? 16 : qtype == 5 ? 20 : qtype == 8 ? 32 : -1;
}

/* IEEE binary16 bits -> float (exact: every half is a float). */
float svqo_half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t exp = (h >> 10) & 31u;
  uint32_t man = h & 1023u;
  uint32_t bits;
  if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else if (exp != 0) {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  } else if (man == 0) {
    bits = sign;
  } else { /* subnormal: normalize */
    int e = -1;
    do {
      man <<= 1;
      ++e;
    } while ((man & 1024u) == 0);
    bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 1023u) << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* Signed integer weights of block b: out[32]. */
int svqo_codes(const uint8_t *q, int64_t b, int qtype, int32_t *out) {
  const int w = payload_bytes(qtype);
  if (w < 0) return -1;
  const uint8_t *p = q + b * w;
  if (qtype == 8) {
    for (int j = 0; j < 32; ++j) out[j] = (int8_t)p[j];
    return 0;
  }
  uint32_t mask = 0;
  const uint8_t *nib = p;
  if (qtype == 5) {
    mask = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
    nib = p + 4;
  }
  for (int j = 0; j < 16; ++j) {
    int lo = nib[j] & 15, hi = nib[j] >> 4;
    if (qtype == 4) {
      out[j] = lo - 8;
      out[j + 16] = hi - 8;
    } else {
      out[j] = (lo | (int)(((mask >> j) & 1u) << 4)) - 16;
      out[j + 16] = (hi | (int)(((mask >> (j + 16)) & 1u) << 4)) - 16;
    }
  }
  return 0;
}

/* out[b*32 + j] = (float)code * (float)d for every block. */
int svqo_dequant(const uint8_t *q, const uint16_t *s, float *out,
                 int64_t nblocks, int qtype) {
  int32_t c[32];
  if (payload_bytes(qtype) < 0) return -1;
  for (int64_t b = 0; b < nblocks; ++b) {
    svqo_codes(q, b, qtype, c);
    const float d = svqo_half_to_float(s[b]);
    for (int j = 0; j < 32; ++j) out[b * 32 + j] = (float)c[j] * d;
  }
  return 0;
}

/* y[m*n + row] in double; x and bias are fp16 bits; bias may be NULL. */
int svqo_gemv_f64(const uint16_t *x, const uint8_t *q, const uint16_t *s,
                  const uint16_t *bias, int m, int n, int k, int qtype,
                  double *y) {
  if (payload_bytes(qtype) < 0 || k % 32 || m < 1 || n < 1) return -1;
  const int kb = k / 32;
  int32_t c[32];
  for (int i = 0; i < m * n; ++i) y[i] = 0.0;
  for (int row = 0; row < n; ++row) {
    for (int blk = 0; blk < kb; ++blk) {
      const int64_t b = (int64_t)row * kb + blk;
      svqo_codes(q, b, qtype, c);
      const double d = (double)svqo_half_to_float(s[b]);
      for (int mi = 0; mi < m; ++mi) {
        const uint16_t *xr = x + (int64_t)mi * k + blk * 32;
        double acc = 0.0;
        for (int j = 0; j < 32; ++j)
          acc += (double)c[j] * (double)svqo_half_to_float(xr[j]);
        y[(int64_t)mi * n + row] += acc * d;
      }
    }
    if (bias) {
      const double bv = (double)svqo_half_to_float(bias[row]);
      for (int mi = 0; mi < m; ++mi) y[(int64_t)mi * n + row] += bv;
    }
  }
  return 0;
}
