/*
 * CPU ORACLE -- test infrastructure only (see oracle.h).
 *
 * Restates, in plain C, the reference's block formats and row dot products:
 *   value_at        src/quant.rs:349-456
 *   dot_row_scalar  src/quant.rs:458-648
 *   dot_row_avx2    src/simd.rs:11-311   (the CPU baseline; AVX2+FMA intrinsics)
 *   matvec          src/backend.rs:143-162 (row-parallel threading policy)
 *
 * Pinned by: tests/test_oracle.py -- an independent float64 numpy decoder
 * written from the GGML block layouts (bit-exact for every type), the
 * reference's own unit-test vectors (src/quant.rs:973-1063: dot == sum of
 * dequantized*x within 1e-4, AVX2 vs scalar within 2e-4*max(|s|,1) incl. the
 * deterministic Q5_K block of src/quant.rs:1016-1023), brute-force float64
 * dots on random rows, and special cases (d = 0, Q8_0 code -128, every
 * 12-byte K-quant scale pattern).
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <string.h>
#include <unistd.h>

#define QK_K 256

int oq_block_size(uint32_t t) {
  switch (t) {
    case OQ_F32: case OQ_F16: case OQ_BF16: return 1;
    case OQ_Q4_0: case OQ_Q4_1: case OQ_Q5_0: case OQ_Q5_1: case OQ_Q8_0: return 32;
    case OQ_Q4_K: case OQ_Q5_K: case OQ_Q6_K: return QK_K;
    default: return 0;
  }
}

int oq_type_size(uint32_t t) {
  switch (t) {
    case OQ_F32: return 4;
    case OQ_F16: case OQ_BF16: return 2;
    case OQ_Q4_0: return 18;
    case OQ_Q4_1: return 20;
    case OQ_Q5_0: return 22;
    case OQ_Q5_1: return 24;
    case OQ_Q8_0: return 34;
    case OQ_Q4_K: return 144;
    case OQ_Q5_K: return 176;
    case OQ_Q6_K: return 210;
    default: return 0;
  }
}

size_t oq_row_bytes(uint32_t t, size_t cols) {
  int bs = oq_block_size(t);
  if (bs == 0 || cols % (size_t)bs) return 0;
  return cols / (size_t)bs * (size_t)oq_type_size(t);
}

/* IEEE binary16 -> binary32, exact (subnormals normalised, NaN quietened). */
float oq_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -1;
      do { man <<= 1; e++; } while ((man & 0x400u) == 0);
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13) | (man ? 0x00400000u : 0);
  } else {
    bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* bfloat16 -> binary32: the upper half of the f32 bit pattern (NaN quietened,
 * as the `half` crate does). */
float oq_bf16_to_f32(uint16_t h) {
  uint32_t bits = (uint32_t)h << 16;
  if ((h & 0x7fffu) > 0x7f80u) bits |= 0x00400000u;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static inline float rd_f16(const uint8_t *p, size_t off) {
  return oq_f16_to_f32((uint16_t)(p[off] | (p[off + 1] << 8)));
}
static inline float rd_bf16(const uint8_t *p, size_t off) {
  return oq_bf16_to_f32((uint16_t)(p[off] | (p[off + 1] << 8)));
}
static inline float rd_f32(const uint8_t *p, size_t off) {
  float f;
  memcpy(&f, p + off, 4);
  return f;
}

/* scale_min_k4 (src/quant.rs:338-347): 6-bit (scale, min) of sub-block `i`. */
static inline void scale_min_k4(int i, const uint8_t *s, uint8_t *sc, uint8_t *mn) {
  if (i < 4) {
    *sc = s[i] & 63;
    *mn = s[i + 4] & 63;
  } else {
    *sc = (uint8_t)((s[i + 4] & 0x0f) | ((s[i - 4] >> 6) << 4));
    *mn = (uint8_t)((s[i + 4] >> 4) | ((s[i] >> 6) << 4));
  }
}

float oq_value_at(const uint8_t *row, uint32_t ty, size_t col) {
  switch (ty) {
    case OQ_F32: return rd_f32(row, col * 4);
    case OQ_F16: return rd_f16(row, col * 2);
    case OQ_BF16: return rd_bf16(row, col * 2);
    case OQ_Q4_0: {
      const uint8_t *b = row + col / 32 * 18;
      size_t j = col % 32;
      uint8_t q = j < 16 ? (b[2 + j] & 0x0f) : (b[2 + j - 16] >> 4);
      return rd_f16(b, 0) * ((float)q - 8.0f);
    }
    case OQ_Q4_1: {
      const uint8_t *b = row + col / 32 * 20;
      size_t j = col % 32;
      uint8_t q = j < 16 ? (b[4 + j] & 0x0f) : (b[4 + j - 16] >> 4);
      return rd_f16(b, 0) * (float)q + rd_f16(b, 2);
    }
    case OQ_Q5_0:
    case OQ_Q5_1: {
      size_t bsz = (size_t)oq_type_size(ty);
      const uint8_t *b = row + col / 32 * bsz;
      size_t j = col % 32;
      size_t qh_off = ty == OQ_Q5_0 ? 2 : 4, qs_off = ty == OQ_Q5_0 ? 6 : 8;
      uint8_t lo = j < 16 ? (b[qs_off + j] & 0x0f) : (b[qs_off + j - 16] >> 4);
      uint8_t hi = (b[qh_off + j / 8] >> (j % 8)) & 1;
      uint8_t q = (uint8_t)(lo | (hi << 4));
      if (ty == OQ_Q5_0) return rd_f16(b, 0) * ((float)q - 16.0f);
      return rd_f16(b, 0) * (float)q + rd_f16(b, 2);
    }
    case OQ_Q8_0: {
      const uint8_t *b = row + col / 32 * 34;
      return rd_f16(b, 0) * (float)(int8_t)b[2 + col % 32];
    }
    case OQ_Q4_K: {
      const uint8_t *b = row + col / QK_K * 144;
      size_t j = col % QK_K;
      int group = (int)(j / 32);
      uint8_t sc, mn;
      scale_min_k4(group, b + 4, &sc, &mn);
      uint8_t packed = b[16 + (group / 2) * 32 + j % 32];
      uint8_t q = (group % 2 == 0) ? (packed & 0x0f) : (packed >> 4);
      return rd_f16(b, 0) * (float)sc * (float)q - rd_f16(b, 2) * (float)mn;
    }
    case OQ_Q5_K: {
      const uint8_t *b = row + col / QK_K * 176;
      size_t j = col % QK_K;
      int group = (int)(j / 32);
      uint8_t sc, mn;
      scale_min_k4(group, b + 4, &sc, &mn);
      uint8_t packed = b[48 + (group / 2) * 32 + j % 32];
      uint8_t lo = (group % 2 == 0) ? (packed & 0x0f) : (packed >> 4);
      uint8_t hi = (b[16 + j % 32] & (uint8_t)(1u << group)) ? 16 : 0;
      return rd_f16(b, 0) * (float)sc * (float)(lo + hi) - rd_f16(b, 2) * (float)mn;
    }
    case OQ_Q6_K: {
      const uint8_t *b = row + col / QK_K * 210;
      size_t j = col % QK_K;
      size_t half = j / 128, within = j % 128, lane = within % 32, quarter = within / 32;
      uint8_t ql;
      switch (quarter) {
        case 0: ql = b[half * 64 + lane] & 0x0f; break;
        case 1: ql = b[half * 64 + 32 + lane] & 0x0f; break;
        case 2: ql = b[half * 64 + lane] >> 4; break;
        default: ql = b[half * 64 + 32 + lane] >> 4; break;
      }
      uint8_t qh = (b[128 + half * 32 + lane] >> (quarter * 2)) & 3;
      float q = (float)((int16_t)(ql | (qh << 4)) - 32);
      float scale = (float)(int8_t)b[192 + half * 8 + quarter * 2 + lane / 16];
      return rd_f16(b, 208) * scale * q;
    }
    default: return 0.0f;
  }
}

void oq_dequant_row(const uint8_t *row, uint32_t ty, size_t cols, float *out) {
  for (size_t c = 0; c < cols; c++) out[c] = oq_value_at(row, ty, c);
}

/* ------------------------------ scalar dots ------------------------------ */

static float dot_q4k(const uint8_t *row, const float *input, size_t nblocks) {
  float sum = 0.0f;
  for (size_t bi = 0; bi < nblocks; bi++) {
    const uint8_t *b = row + bi * 144;
    float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    const float *x = input + bi * QK_K;
    for (int g = 0; g < 8; g++) {
      uint8_t sc, mn;
      scale_min_k4(g, scales, &sc, &mn);
      float ds = d * (float)sc, dm = dmin * (float)mn;
      for (int j = 0; j < 32; j++) {
        uint8_t p = qs[g / 2 * 32 + j];
        uint8_t q = (g % 2 == 0) ? (p & 0x0f) : (p >> 4);
        sum += (ds * (float)q - dm) * x[g * 32 + j];
      }
    }
  }
  return sum;
}

static float dot_q5k(const uint8_t *row, const float *input, size_t nblocks) {
  float sum = 0.0f;
  for (size_t bi = 0; bi < nblocks; bi++) {
    const uint8_t *b = row + bi * 176;
    float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
    const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
    const float *x = input + bi * QK_K;
    for (int g = 0; g < 8; g++) {
      uint8_t sc, mn;
      scale_min_k4(g, scales, &sc, &mn);
      float ds = d * (float)sc, dm = dmin * (float)mn;
      uint8_t mask = (uint8_t)(1u << g);
      for (int j = 0; j < 32; j++) {
        uint8_t p = qs[g / 2 * 32 + j];
        uint8_t lo = (g % 2 == 0) ? (p & 0x0f) : (p >> 4);
        uint8_t q = (uint8_t)(lo + ((qh[j] & mask) ? 16 : 0));
        sum += (ds * (float)q - dm) * x[g * 32 + j];
      }
    }
  }
  return sum;
}

static float dot_q6k(const uint8_t *row, const float *input, size_t nblocks) {
  float sum = 0.0f;
  for (size_t bi = 0; bi < nblocks; bi++) {
    const uint8_t *b = row + bi * 210;
    float d = rd_f16(b, 208);
    const float *x = input + bi * QK_K;
    for (int half = 0; half < 2; half++) {
      const uint8_t *ql = b + half * 64, *qh = b + 128 + half * 32, *sc = b + 192 + half * 8;
      int base = half * 128;
      for (int lane = 0; lane < 32; lane++) {
        int si = lane / 16;
        int q1 = (int16_t)((ql[lane] & 0x0f) | ((qh[lane] & 3) << 4)) - 32;
        int q2 = (int16_t)((ql[32 + lane] & 0x0f) | (((qh[lane] >> 2) & 3) << 4)) - 32;
        int q3 = (int16_t)((ql[lane] >> 4) | (((qh[lane] >> 4) & 3) << 4)) - 32;
        int q4 = (int16_t)((ql[32 + lane] >> 4) | (((qh[lane] >> 6) & 3) << 4)) - 32;
        sum += d * (float)(int8_t)sc[si] * (float)q1 * x[base + lane];
        sum += d * (float)(int8_t)sc[si + 2] * (float)q2 * x[base + 32 + lane];
        sum += d * (float)(int8_t)sc[si + 4] * (float)q3 * x[base + 64 + lane];
        sum += d * (float)(int8_t)sc[si + 6] * (float)q4 * x[base + 96 + lane];
      }
    }
  }
  return sum;
}

float oq_dot_row_scalar(const uint8_t *row, uint32_t ty, const float *input, size_t cols) {
  switch (ty) {
    case OQ_F32: {
      float sum = -0.0f; /* Iterator::sum for f32 */
      for (size_t i = 0; i < cols; i++) sum += rd_f32(row, i * 4) * input[i];
      return sum;
    }
    case OQ_F16: {
      float sum = -0.0f;
      for (size_t i = 0; i < cols; i++) sum += rd_f16(row, i * 2) * input[i];
      return sum;
    }
    case OQ_BF16: {
      float sum = -0.0f;
      for (size_t i = 0; i < cols; i++) sum += rd_bf16(row, i * 2) * input[i];
      return sum;
    }
    case OQ_Q4_0: {
      float sum = 0.0f;
      for (size_t bi = 0; bi < cols / 32; bi++) {
        const uint8_t *b = row + bi * 18;
        float d = rd_f16(b, 0);
        const float *x = input + bi * 32;
        for (int j = 0; j < 16; j++) {
          uint8_t q = b[2 + j];
          sum += d * ((float)(q & 0x0f) - 8.0f) * x[j];
          sum += d * ((float)(q >> 4) - 8.0f) * x[j + 16];
        }
      }
      return sum;
    }
    case OQ_Q4_1: {
      float sum = 0.0f;
      for (size_t bi = 0; bi < cols / 32; bi++) {
        const uint8_t *b = row + bi * 20;
        float d = rd_f16(b, 0), m = rd_f16(b, 2);
        const float *x = input + bi * 32;
        for (int j = 0; j < 16; j++) {
          uint8_t q = b[4 + j];
          sum += (d * (float)(q & 0x0f) + m) * x[j];
          sum += (d * (float)(q >> 4) + m) * x[j + 16];
        }
      }
      return sum;
    }
    case OQ_Q5_0:
    case OQ_Q5_1: {
      float sum = 0.0f;
      size_t size = (size_t)oq_type_size(ty);
      for (size_t bi = 0; bi < cols / 32; bi++) {
        const uint8_t *b = row + bi * size;
        float d = rd_f16(b, 0);
        float m = ty == OQ_Q5_1 ? rd_f16(b, 2) : 0.0f;
        size_t qh_off = ty == OQ_Q5_0 ? 2 : 4, qs_off = ty == OQ_Q5_0 ? 6 : 8;
        uint32_t qh = (uint32_t)b[qh_off] | ((uint32_t)b[qh_off + 1] << 8) |
                      ((uint32_t)b[qh_off + 2] << 16) | ((uint32_t)b[qh_off + 3] << 24);
        const float *x = input + bi * 32;
        for (int j = 0; j < 16; j++) {
          uint8_t p = b[qs_off + j];
          uint32_t q0 = (uint32_t)(p & 0x0f) | (((qh >> j) & 1) << 4);
          uint32_t q1 = (uint32_t)(p >> 4) | (((qh >> (j + 16)) & 1) << 4);
          if (ty == OQ_Q5_0) {
            sum += d * ((float)q0 - 16.0f) * x[j];
            sum += d * ((float)q1 - 16.0f) * x[j + 16];
          } else {
            sum += (d * (float)q0 + m) * x[j];
            sum += (d * (float)q1 + m) * x[j + 16];
          }
        }
      }
      return sum;
    }
    case OQ_Q8_0: {
      float sum = 0.0f;
      for (size_t bi = 0; bi < cols / 32; bi++) {
        const uint8_t *b = row + bi * 34;
        float d = rd_f16(b, 0);
        const float *x = input + bi * 32;
        for (int j = 0; j < 32; j++) sum += d * (float)(int8_t)b[2 + j] * x[j];
      }
      return sum;
    }
    case OQ_Q4_K: return dot_q4k(row, input, cols / QK_K);
    case OQ_Q5_K: return dot_q5k(row, input, cols / QK_K);
    case OQ_Q6_K: return dot_q6k(row, input, cols / QK_K);
    default: return 0.0f;
  }
}

/* --------------------- AVX2 restatement (CPU baseline) --------------------- */

#define AVX2 __attribute__((target("avx2,fma")))

AVX2 static inline float hsum(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 s = _mm_add_ps(lo, hi);
  s = _mm_hadd_ps(s, s);
  s = _mm_hadd_ps(s, s);
  return _mm_cvtss_f32(s);
}

AVX2 static inline __m256i u8x8_i32(const uint8_t *p) {
  return _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i *)p));
}
AVX2 static inline __m256i i8x8_i32(const uint8_t *p) {
  return _mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)p));
}

AVX2 static float avx_f32(const uint8_t *row, const float *x, size_t n) {
  __m256 acc = _mm256_setzero_ps();
  size_t i = 0;
  for (; i + 8 <= n; i += 8)
    acc = _mm256_fmadd_ps(_mm256_loadu_ps((const float *)(row + i * 4)), _mm256_loadu_ps(x + i), acc);
  float sum = hsum(acc);
  for (; i < n; i++) sum += rd_f32(row, i * 4) * x[i];
  return sum;
}

/* Q4_0 (affine = 0) and Q4_1 (affine = 1), src/simd.rs:74-101. */
AVX2 static float avx_q4(const uint8_t *row, const float *input, size_t nb, int affine) {
  size_t bsz = affine ? 20 : 18, qoff = affine ? 4 : 2;
  float sum = 0.0f;
  for (size_t bi = 0; bi < nb; bi++) {
    const uint8_t *b = row + bi * bsz;
    float d = rd_f16(b, 0);
    float mn = affine ? rd_f16(b, 2) : -8.0f * d;
    const float *x = input + bi * 32;
    __m256 qdot = _mm256_setzero_ps(), xsum = _mm256_setzero_ps();
    for (int half = 0; half < 2; half++)
      for (int chunk = 0; chunk < 2; chunk++) {
        __m256i packed = u8x8_i32(b + qoff + chunk * 8);
        __m256i codes = half == 0 ? _mm256_and_si256(packed, _mm256_set1_epi32(15))
                                  : _mm256_srli_epi32(packed, 4);
        __m256 v = _mm256_loadu_ps(x + half * 16 + chunk * 8);
        qdot = _mm256_fmadd_ps(_mm256_cvtepi32_ps(codes), v, qdot);
        xsum = _mm256_add_ps(xsum, v);
      }
    sum += d * hsum(qdot) + mn * hsum(xsum);
  }
  return sum;
}

/* Q5_0 / Q5_1, src/simd.rs:103-151. */
AVX2 static float avx_q5(const uint8_t *row, const float *input, size_t nb, int affine) {
  size_t bsz = affine ? 24 : 22, qh_off = affine ? 4 : 2, qs_off = affine ? 8 : 6;
  float sum = 0.0f;
  for (size_t bi = 0; bi < nb; bi++) {
    const uint8_t *b = row + bi * bsz;
    float d = rd_f16(b, 0);
    float mn = affine ? rd_f16(b, 2) : -16.0f * d;
    uint32_t qh = (uint32_t)b[qh_off] | ((uint32_t)b[qh_off + 1] << 8) |
                  ((uint32_t)b[qh_off + 2] << 16) | ((uint32_t)b[qh_off + 3] << 24);
    const float *x = input + bi * 32;
    __m256 qdot = _mm256_setzero_ps(), xsum = _mm256_setzero_ps();
    for (int half = 0; half < 2; half++)
      for (int chunk = 0; chunk < 2; chunk++) {
        int base = chunk * 8;
        __m256i packed = u8x8_i32(b + qs_off + base);
        __m256i low = half == 0 ? _mm256_and_si256(packed, _mm256_set1_epi32(15))
                                : _mm256_srli_epi32(packed, 4);
        int bit = half * 16 + base;
        int32_t hv[8];
        for (int k = 0; k < 8; k++) hv[k] = (int32_t)(((qh >> (bit + k)) & 1) << 4);
        __m256i high = _mm256_loadu_si256((const __m256i *)hv);
        __m256i codes = _mm256_add_epi32(low, high);
        __m256 v = _mm256_loadu_ps(x + half * 16 + base);
        qdot = _mm256_fmadd_ps(_mm256_cvtepi32_ps(codes), v, qdot);
        xsum = _mm256_add_ps(xsum, v);
      }
    sum += d * hsum(qdot) + mn * hsum(xsum);
  }
  return sum;
}

/* Q8_0, src/simd.rs:153-167. */
AVX2 static float avx_q8(const uint8_t *row, const float *input, size_t nb) {
  float sum = 0.0f;
  for (size_t bi = 0; bi < nb; bi++) {
    const uint8_t *b = row + bi * 34;
    float d = rd_f16(b, 0);
    __m256 acc = _mm256_setzero_ps();
    for (int chunk = 0; chunk < 4; chunk++) {
      __m256i codes = i8x8_i32(b + 2 + chunk * 8);
      __m256 v = _mm256_loadu_ps(input + bi * 32 + chunk * 8);
      acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(codes), v, acc);
    }
    sum += d * hsum(acc);
  }
  return sum;
}

/* Q4_K, src/simd.rs:169-197. */
AVX2 static float avx_q4k(const uint8_t *row, const float *input, size_t nb) {
  float sum = 0.0f;
  for (size_t bi = 0; bi < nb; bi++) {
    const uint8_t *b = row + bi * 144;
    float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    const float *x = input + bi * 256;
    for (int g = 0; g < 8; g++) {
      uint8_t sc, mn;
      scale_min_k4(g, scales, &sc, &mn);
      __m256 qdot = _mm256_setzero_ps(), xsum = _mm256_setzero_ps();
      for (int chunk = 0; chunk < 4; chunk++) {
        __m256i packed = u8x8_i32(qs + g / 2 * 32 + chunk * 8);
        __m256i codes = g % 2 == 0 ? _mm256_and_si256(packed, _mm256_set1_epi32(15))
                                   : _mm256_srli_epi32(packed, 4);
        __m256 v = _mm256_loadu_ps(x + g * 32 + chunk * 8);
        qdot = _mm256_fmadd_ps(_mm256_cvtepi32_ps(codes), v, qdot);
        xsum = _mm256_add_ps(xsum, v);
      }
      sum += d * (float)sc * hsum(qdot) - dmin * (float)mn * hsum(xsum);
    }
  }
  return sum;
}

/* Q5_K, src/simd.rs:199-236. */
AVX2 static float avx_q5k(const uint8_t *row, const float *input, size_t nb) {
  float sum = 0.0f;
  for (size_t bi = 0; bi < nb; bi++) {
    const uint8_t *b = row + bi * 176;
    float d = rd_f16(b, 0), dmin = rd_f16(b, 2);
    const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
    const float *x = input + bi * 256;
    for (int g = 0; g < 8; g++) {
      uint8_t sc, mn;
      scale_min_k4(g, scales, &sc, &mn);
      __m256i mask = _mm256_set1_epi32(1 << g);
      __m256 qdot = _mm256_setzero_ps(), xsum = _mm256_setzero_ps();
      for (int chunk = 0; chunk < 4; chunk++) {
        __m256i packed = u8x8_i32(qs + g / 2 * 32 + chunk * 8);
        __m256i low = g % 2 == 0 ? _mm256_and_si256(packed, _mm256_set1_epi32(15))
                                 : _mm256_srli_epi32(packed, 4);
        __m256i hb = u8x8_i32(qh + chunk * 8);
        __m256i present = _mm256_cmpgt_epi32(_mm256_and_si256(hb, mask), _mm256_setzero_si256());
        __m256i high = _mm256_and_si256(present, _mm256_set1_epi32(16));
        __m256i codes = _mm256_add_epi32(low, high);
        __m256 v = _mm256_loadu_ps(x + g * 32 + chunk * 8);
        qdot = _mm256_fmadd_ps(_mm256_cvtepi32_ps(codes), v, qdot);
        xsum = _mm256_add_ps(xsum, v);
      }
      sum += d * (float)sc * hsum(qdot) - dmin * (float)mn * hsum(xsum);
    }
  }
  return sum;
}

/* Q6_K, src/simd.rs:238-281. */
AVX2 static float avx_q6k(const uint8_t *row, const float *input, size_t nb) {
  float sum = 0.0f;
  for (size_t bi = 0; bi < nb; bi++) {
    const uint8_t *b = row + bi * 210;
    float d = rd_f16(b, 208);
    const float *x = input + bi * 256;
    __m256 acc = _mm256_setzero_ps();
    for (int half = 0; half < 2; half++) {
      const uint8_t *ql = b + half * 64, *qh = b + 128 + half * 32, *scales = b + 192 + half * 8;
      for (int quarter = 0; quarter < 4; quarter++) {
        int ql_base = quarter % 2 == 0 ? 0 : 32;
        for (int chunk = 0; chunk < 4; chunk++) {
          __m256i pl = u8x8_i32(ql + ql_base + chunk * 8);
          __m256i low = quarter < 2 ? _mm256_and_si256(pl, _mm256_set1_epi32(15)) : _mm256_srli_epi32(pl, 4);
          __m256i ph = u8x8_i32(qh + chunk * 8);
          __m256i sh;
          switch (quarter) {
            case 0: sh = ph; break;
            case 1: sh = _mm256_srli_epi32(ph, 2); break;
            case 2: sh = _mm256_srli_epi32(ph, 4); break;
            default: sh = _mm256_srli_epi32(ph, 6); break;
          }
          __m256i high = _mm256_and_si256(sh, _mm256_set1_epi32(3));
          __m256i codes = _mm256_sub_epi32(_mm256_or_si256(low, _mm256_slli_epi32(high, 4)), _mm256_set1_epi32(32));
          float scale = (float)(int8_t)scales[quarter * 2 + (chunk * 8) / 16] * d;
          __m256 v = _mm256_loadu_ps(x + half * 128 + quarter * 32 + chunk * 8);
          __m256 w = _mm256_mul_ps(_mm256_cvtepi32_ps(codes), _mm256_set1_ps(scale));
          acc = _mm256_fmadd_ps(w, v, acc);
        }
      }
    }
    sum += hsum(acc);
  }
  return sum;
}

int oq_cpu_has_avx2_fma(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

float oq_dot_row_avx2(const uint8_t *row, uint32_t ty, const float *x, size_t cols) {
  static int has = -1;
  if (has < 0) has = oq_cpu_has_avx2_fma();
  if (!has) return oq_dot_row_scalar(row, ty, x, cols);
  switch (ty) {
    case OQ_F32: return avx_f32(row, x, cols);
    case OQ_Q4_0: return avx_q4(row, x, cols / 32, 0);
    case OQ_Q4_1: return avx_q4(row, x, cols / 32, 1);
    case OQ_Q5_0: return avx_q5(row, x, cols / 32, 0);
    case OQ_Q5_1: return avx_q5(row, x, cols / 32, 1);
    case OQ_Q8_0: return avx_q8(row, x, cols / 32);
    case OQ_Q4_K: return avx_q4k(row, x, cols / 256);
    case OQ_Q5_K: return avx_q5k(row, x, cols / 256);
    case OQ_Q6_K: return avx_q6k(row, x, cols / 256);
    default: return oq_dot_row_scalar(row, ty, x, cols); /* F16/BF16: src/simd.rs:296 */
  }
}

/* ------------------------------ matvec policy ----------------------------- */

/* A persistent worker pool, like the rayon ThreadPool the reference builds once
 * (src/backend.rs:109-112); rows are claimed in small chunks from an atomic
 * counter.  Each row is an independent sequential dot, so the split cannot
 * change any result: every thread count gives identical bits. */
typedef struct {
  const uint8_t *w;
  uint32_t ty;
  size_t rows, cols, row_bytes;
  const float *x;
  float *y;
  int kernel;
} mv_job;

static pthread_mutex_t pool_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t pool_cv = PTHREAD_COND_INITIALIZER, pool_done_cv = PTHREAD_COND_INITIALIZER;
static int pool_size = 0;
static unsigned long pool_gen = 0;
static int pool_active = 0;
static mv_job pool_job;
static size_t pool_next;
static pthread_mutex_t call_mu = PTHREAD_MUTEX_INITIALIZER;

static void run_rows(const mv_job *j, size_t r0, size_t r1) {
  for (size_t r = r0; r < r1; r++) {
    const uint8_t *row = j->w + r * j->row_bytes;
    j->y[r] = j->kernel == OQ_KERNEL_AVX2 ? oq_dot_row_avx2(row, j->ty, j->x, j->cols)
                                          : oq_dot_row_scalar(row, j->ty, j->x, j->cols);
  }
}

static void drain(const mv_job *j) {
  const size_t chunk = 8;
  for (;;) {
    size_t r0 = __atomic_fetch_add(&pool_next, chunk, __ATOMIC_RELAXED);
    if (r0 >= j->rows) break;
    run_rows(j, r0, r0 + chunk < j->rows ? r0 + chunk : j->rows);
  }
}

static void *pool_worker(void *arg) {
  (void)arg;
  unsigned long seen = 0;
  pthread_mutex_lock(&pool_mu);
  for (;;) {
    while (pool_gen == seen) pthread_cond_wait(&pool_cv, &pool_mu);
    seen = pool_gen;
    mv_job j = pool_job;
    pthread_mutex_unlock(&pool_mu);
    drain(&j);
    pthread_mutex_lock(&pool_mu);
    if (--pool_active == 0) pthread_cond_signal(&pool_done_cv);
  }
  return NULL;
}

static void pool_ensure(int n) {
  while (pool_size < n) {
    pthread_t t;
    pthread_create(&t, NULL, pool_worker, NULL);
    pthread_detach(t);
    pool_size++;
  }
}

int oq_matvec(const uint8_t *w, uint32_t ty, size_t rows, size_t cols, const float *x, float *y,
              int kernel, int threads, size_t parallel_threshold) {
  size_t rb = oq_row_bytes(ty, cols);
  if (rb == 0) return -1;
  if (threads <= 0) threads = (int)sysconf(_SC_NPROCESSORS_ONLN);
  if (threads < 1) threads = 1;
  mv_job job = {w, ty, rows, cols, rb, x, y, kernel};
  if (threads > 1 && rows >= (size_t)threads * 2 && rows * cols >= parallel_threshold) {
    pthread_mutex_lock(&call_mu);
    pthread_mutex_lock(&pool_mu);
    pool_ensure(threads - 1);
    pool_job = job;
    pool_next = 0;
    pool_active = threads - 1;
    pool_gen++;
    pthread_cond_broadcast(&pool_cv);
    pthread_mutex_unlock(&pool_mu);
    drain(&job); /* the caller thread works too */
    pthread_mutex_lock(&pool_mu);
    while (pool_active > 0) pthread_cond_wait(&pool_done_cv, &pool_mu);
    pthread_mutex_unlock(&pool_mu);
    pthread_mutex_unlock(&call_mu);
  } else {
    run_rows(&job, 0, rows);
  }
  return 0;
}
