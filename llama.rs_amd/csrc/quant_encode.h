// GGML block encoders and the synthetic-weight RNG, shared by host and device.
//
// The encoders restate the reference's quantizers (src/quant.rs:650-967).
// Rust semantics are kept: f32::round = roundf (half away from zero),
// f32::max/min = fmaxf/fminf, saturating float->int `as` casts with NaN -> 0,
// sequential f32 sums, f16 encoding round-to-nearest-even.  Every file that
// includes this header is compiled with -ffp-contract=off, and every
// operation used is an IEEE-754 correctly rounded one (+ - * / sqrt, round,
// floor, min, max), so the host build and the gfx950 build produce the same
// bytes for the same input.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__) || defined(__HIP__)
#include <hip/hip_runtime.h>
#define LLRS_HD __host__ __device__ inline
#else
#include <math.h>
#define LLRS_HD inline
#endif

namespace llrs {
namespace enc {

LLRS_HD uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
LLRS_HD float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// f32 -> IEEE binary16 bits, round to nearest even (half::f16::from_f32).
LLRS_HD uint16_t f32_to_f16(float f) {
  uint32_t x = f2u(f), sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    return (uint16_t)(sign | 0x7c00u);
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // >= 65520 rounds to inf
  if (ax < 0x38800000u) {                                     // f16 subnormal range
    if (ax < 0x33000000u) return (uint16_t)sign;
    uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, s = 126 - e;
    uint32_t r = m >> s, rem = m & ((1u << s) - 1), half = 1u << (s - 1);
    if (rem > half || (rem == half && (r & 1))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t r = (ax >> 13) - (112u << 10), rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
  return (uint16_t)(sign | r);
}

LLRS_HD float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1f, man = h & 0x3ffu, bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while ((man & 0x400u) == 0);
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13) | (man ? 0x00400000u : 0);
  } else {
    bits = sign | ((exp + 112) << 23) | (man << 13);
  }
  return u2f(bits);
}

LLRS_HD float f16_round(float v) { return f16_to_f32(f32_to_f16(v)); }

LLRS_HD void put_f16(uint8_t *o, float v) {
  uint16_t h = f32_to_f16(v);
  o[0] = (uint8_t)(h & 0xff);
  o[1] = (uint8_t)(h >> 8);
}

LLRS_HD bool is_nan(float f) { return (f2u(f) & 0x7fffffffu) > 0x7f800000u; }
// Rust `as` from f32: saturating, NaN -> 0, truncation toward zero.
LLRS_HD uint8_t as_u8(float f) {
  if (is_nan(f) || f <= 0.f) return 0;
  if (f >= 255.f) return 255;
  return (uint8_t)f;
}
LLRS_HD int8_t as_i8(float f) {
  if (is_nan(f)) return 0;
  if (f <= -128.f) return -128;
  if (f >= 127.f) return 127;
  return (int8_t)f;
}
LLRS_HD int32_t as_i32(float f) {
  if (is_nan(f)) return 0;
  if (f <= -2147483648.f) return INT32_MIN;
  if (f >= 2147483648.f) return INT32_MAX;
  return (int32_t)f;
}
// f32::clamp: NaN passes through.
LLRS_HD float clampf(float v, float lo, float hi) {
  if (v < lo) v = lo;
  if (v > hi) v = hi;
  return v;
}

// quantize_block_q8_0 (src/quant.rs:650-662): 32 values -> 34 bytes.
LLRS_HD void block_q8_0(const float *v, uint8_t *out) {
  float abs_max = 0.f;
  for (int i = 0; i < 32; i++) abs_max = fmaxf(abs_max, fabsf(v[i]));
  float d = abs_max / 127.0f;
  float inv = d == 0.f ? 0.f : 1.0f / d;
  put_f16(out, d);
  for (int i = 0; i < 32; i++) out[2 + i] = (uint8_t)as_i8(clampf(roundf(v[i] * inv), -127.f, 127.f));
}

// make_qx_quants_16 (src/quant.rs:726-777).
LLRS_HD float make_qx_quants_16(const float *v, uint8_t *codes) {
  float mx = 0.f, abs_max = 0.f;
  for (int i = 0; i < 16; i++)
    if (fabsf(v[i]) > abs_max) {
      abs_max = fabsf(v[i]);
      mx = v[i];
    }
  if (abs_max < 1e-15f) {
    for (int i = 0; i < 16; i++) codes[i] = 0;
    return 0.f;
  }
  float inv_scale = -32.0f / mx;
  float sum_lx = 0.f, sum_l2 = 0.f;
  for (int i = 0; i < 16; i++) {
    int32_t level = as_i32(clampf(roundf(inv_scale * v[i]), -32.f, 31.f));
    codes[i] = (uint8_t)(level + 32);
    float w = v[i] * v[i];
    sum_lx += w * v[i] * (float)level;
    sum_l2 += w * (float)(level * level);
  }
  float scale = sum_l2 > 0.f ? sum_lx / sum_l2 : 0.f;
  float best = scale * sum_lx;
  for (int step = -9; step <= 9; step++) {
    if (step == 0) continue;
    inv_scale = -(32.0f + 0.1f * (float)step) / mx;
    sum_lx = 0.f;
    sum_l2 = 0.f;
    for (int i = 0; i < 16; i++) {
      int32_t level = as_i32(clampf(roundf(inv_scale * v[i]), -32.f, 31.f));
      float w = v[i] * v[i];
      sum_lx += w * v[i] * (float)level;
      sum_l2 += w * (float)(level * level);
    }
    if (sum_l2 > 0.f && sum_lx * sum_lx > best * sum_l2) {
      for (int i = 0; i < 16; i++) {
        int32_t level = as_i32(clampf(roundf(inv_scale * v[i]), -32.f, 31.f));
        codes[i] = (uint8_t)(level + 32);
      }
      scale = sum_lx / sum_l2;
      best = scale * sum_lx;
    }
  }
  return scale;
}

// quantize_block_q6k (src/quant.rs:664-724): 256 values -> 210 bytes.
LLRS_HD void block_q6k(const float *v, uint8_t *out) {
  uint8_t codes[256];
  float scales[16];
  float max_scale = 0.f, max_abs_scale = 0.f;
  for (int g = 0; g < 16; g++) {
    float s = make_qx_quants_16(v + g * 16, codes + g * 16);
    scales[g] = s;
    if (fabsf(s) > max_abs_scale) {
      max_abs_scale = fabsf(s);
      max_scale = s;
    }
  }
  if (max_abs_scale < 1e-15f) {
    for (int i = 0; i < 210; i++) out[i] = 0;
    return;
  }
  float inv_scale = -128.0f / max_scale;
  float d = 1.0f / inv_scale;
  float d_f16 = f16_round(d);
  int8_t scale_codes[16];
  for (int g = 0; g < 16; g++) {
    scale_codes[g] = as_i8(fminf(roundf(inv_scale * scales[g]), 127.f));
    float group_d = d_f16 * (float)scale_codes[g];
    if (group_d == 0.f) continue;
    for (int i = 0; i < 16; i++) {
      int32_t level = as_i32(clampf(roundf(v[g * 16 + i] / group_d), -32.f, 31.f));
      codes[g * 16 + i] = (uint8_t)(level + 32);
    }
  }
  for (int half = 0; half < 2; half++) {
    int base = half * 128;
    for (int lane = 0; lane < 32; lane++) {
      uint8_t q1 = codes[base + lane], q2 = codes[base + 32 + lane], q3 = codes[base + 64 + lane],
              q4 = codes[base + 96 + lane];
      out[half * 64 + lane] = (uint8_t)((q1 & 0x0f) | ((q3 & 0x0f) << 4));
      out[half * 64 + 32 + lane] = (uint8_t)((q2 & 0x0f) | ((q4 & 0x0f) << 4));
      out[128 + half * 32 + lane] =
          (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
    }
  }
  for (int g = 0; g < 16; g++) out[192 + g] = (uint8_t)scale_codes[g];
  put_f16(out + 208, d);
}

// quantize_block_q5_0 (src/quant.rs:779-807): 32 values -> 22 bytes.
LLRS_HD void block_q5_0(const float *v, uint8_t *out) {
  float max_value = 0.f, abs_max = 0.f;
  for (int i = 0; i < 32; i++)
    if (fabsf(v[i]) > abs_max) {
      abs_max = fabsf(v[i]);
      max_value = v[i];
    }
  float d = abs_max == 0.f ? 0.f : max_value / -16.0f;
  float inv = d == 0.f ? 0.f : 1.0f / d;
  put_f16(out, d);
  uint32_t high = 0;
  for (int j = 0; j < 16; j++) {
    uint8_t q0 = as_u8(clampf(floorf(v[j] * inv + 16.5f), 0.f, 31.f));
    uint8_t q1 = as_u8(clampf(floorf(v[j + 16] * inv + 16.5f), 0.f, 31.f));
    out[6 + j] = (uint8_t)((q0 & 0x0f) | ((q1 & 0x0f) << 4));
    high |= (((uint32_t)q0 >> 4) & 1) << j;
    high |= (((uint32_t)q1 >> 4) & 1) << (j + 16);
  }
  for (int k = 0; k < 4; k++) out[2 + k] = (uint8_t)(high >> (8 * k));
}

// make_qkx2_quants (src/quant.rs:892-967).
LLRS_HD float make_qkx2_quants(const float *v, const float *w, uint8_t *codes, float *out_min,
                               uint8_t *aux) {
  float mn = v[0], mx = v[0];
  float sum_w = w[0], sum_x = w[0] * v[0];
  for (int i = 1; i < 32; i++) {
    mn = fminf(mn, v[i]);
    mx = fmaxf(mx, v[i]);
    sum_w += w[i];
    sum_x += w[i] * v[i];
  }
  mn = fminf(mn, 0.f);
  if (mx == mn) {
    for (int i = 0; i < 32; i++) codes[i] = 0;
    *out_min = -mn;
    return 0.f;
  }
  float range = mx - mn;
  float inv_scale = 15.0f / range;
  float scale = 1.0f / inv_scale;
  float best_error = 0.f;
  for (int i = 0; i < 32; i++) {
    uint8_t code = as_u8(clampf(roundf(inv_scale * (v[i] - mn)), 0.f, 15.f));
    codes[i] = code;
    float diff = scale * (float)code + mn - v[i];
    best_error += w[i] * diff * diff;
  }
  for (int step = 0; step <= 20; step++) {
    inv_scale = (-1.0f + 0.1f * (float)step + 15.0f) / range;
    float sum_l = 0.f, sum_l2 = 0.f, sum_xl = 0.f;
    for (int i = 0; i < 32; i++) {
      uint8_t code = as_u8(clampf(roundf(inv_scale * (v[i] - mn)), 0.f, 15.f));
      aux[i] = code;
      float wc = w[i] * (float)code;
      sum_l += wc;
      sum_l2 += wc * (float)code;
      sum_xl += wc * v[i];
    }
    float det = sum_w * sum_l2 - sum_l * sum_l;
    if (det > 0.f) {
      float cs = (sum_w * sum_xl - sum_x * sum_l) / det;
      float cm = (sum_l2 * sum_x - sum_l * sum_xl) / det;
      if (cm > 0.f) {
        cm = 0.f;
        cs = sum_xl / sum_l2;
      }
      float err = 0.f;
      for (int i = 0; i < 32; i++) {
        float diff = cs * (float)aux[i] + cm - v[i];
        err += w[i] * diff * diff;
      }
      if (err < best_error) {
        for (int i = 0; i < 32; i++) codes[i] = aux[i];
        best_error = err;
        scale = cs;
        mn = cm;
      }
    }
  }
  *out_min = -mn;
  return scale;
}

// quantize_block_q4k (src/quant.rs:809-890): 256 values -> 144 bytes.
LLRS_HD void block_q4k(const float *v, uint8_t *out) {
  float local_scales[8], local_mins[8], max_scale = 0.f, max_min = 0.f;
  uint8_t codes[256], aux[32];
  for (int g = 0; g < 8; g++) {
    const float *gv = v + g * 32;
    float sum_sq = -0.0f;
    for (int i = 0; i < 32; i++) sum_sq += gv[i] * gv[i];
    float average = sqrtf(sum_sq / 32.0f);
    float weights[32];
    for (int i = 0; i < 32; i++) weights[i] = average + fabsf(gv[i]);
    float mn = 0.f;
    float s = make_qkx2_quants(gv, weights, codes + g * 32, &mn, aux);
    local_scales[g] = s;
    local_mins[g] = mn;
    max_scale = fmaxf(max_scale, s);
    max_min = fmaxf(max_min, mn);
  }
  float inv_scale = max_scale > 0.f ? 63.0f / max_scale : 0.f;
  float inv_min = max_min > 0.f ? 63.0f / max_min : 0.f;
  uint8_t scales[12] = {0}, sc_codes[8], min_codes[8];
  for (int g = 0; g < 8; g++) {
    sc_codes[g] = as_u8(clampf(roundf(inv_scale * local_scales[g]), 0.f, 63.f));
    min_codes[g] = as_u8(clampf(roundf(inv_min * local_mins[g]), 0.f, 63.f));
    if (g < 4) {
      scales[g] = sc_codes[g];
      scales[g + 4] = min_codes[g];
    } else {
      scales[g + 4] = (uint8_t)((sc_codes[g] & 0x0f) | ((min_codes[g] & 0x0f) << 4));
      scales[g - 4] |= (uint8_t)((sc_codes[g] >> 4) << 6);
      scales[g] |= (uint8_t)((min_codes[g] >> 4) << 6);
    }
  }
  float d = max_scale / 63.0f, dmin = max_min / 63.0f;
  put_f16(out, d);
  put_f16(out + 2, dmin);
  for (int i = 0; i < 12; i++) out[4 + i] = scales[i];
  d = f16_round(d);
  dmin = f16_round(dmin);
  for (int g = 0; g < 8; g++) {
    float scale = d * (float)sc_codes[g];
    if (scale == 0.f) continue;
    float mn = dmin * (float)min_codes[g];
    for (int i = 0; i < 32; i++)
      codes[g * 32 + i] = as_u8(clampf(roundf((v[g * 32 + i] + mn) / scale), 0.f, 15.f));
  }
  for (int pair = 0; pair < 4; pair++)
    for (int i = 0; i < 32; i++)
      out[16 + pair * 32 + i] = (uint8_t)(codes[pair * 64 + i] | (codes[pair * 64 + 32 + i] << 4));
}

// ------------------------------------------------------------ synthetic RNG

LLRS_HD uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Natural log for x in (0, 1]: x = m * 2^e with m in [sqrt(1/2), sqrt(2)),
// ln m = 2 atanh(s), s = (m-1)/(m+1), atanh by its odd series to s^13.
LLRS_HD float ln_unit(float x) {
  uint32_t b = f2u(x);
  int e = (int)(b >> 23) - 127;
  float m = u2f((b & 0x7fffffu) | 0x3f800000u);
  if (m > 1.41421356f) {
    m = m * 0.5f;
    e += 1;
  }
  float s = (m - 1.0f) / (m + 1.0f), s2 = s * s;
  float p = 1.0f / 13.0f;
  p = p * s2 + 1.0f / 11.0f;
  p = p * s2 + 1.0f / 9.0f;
  p = p * s2 + 1.0f / 7.0f;
  p = p * s2 + 1.0f / 5.0f;
  p = p * s2 + 1.0f / 3.0f;
  return (float)e * 0.69314718f + 2.0f * (s + s * s2 * p);
}

// sin and cos of 2*pi*t for t in [0, 1): quadrant from 4t, Taylor series on [0, pi/2).
LLRS_HD void sincos_turn(float t, float &sn, float &cs) {
  float q = t * 4.0f;
  int k = (int)q;
  if (k > 3) k = 3;
  float a = (q - (float)k) * 1.57079633f, a2 = a * a;
  float s = 1.0f / 1307674368000.0f;  // 1/15!
  s = s * -a2 + 1.0f / 6227020800.0f;
  s = s * -a2 + 1.0f / 39916800.0f;
  s = s * -a2 + 1.0f / 362880.0f;
  s = s * -a2 + 1.0f / 5040.0f;
  s = s * -a2 + 1.0f / 120.0f;
  s = s * -a2 + 1.0f / 6.0f;
  s = a - a * a2 * s;
  float c = 1.0f / 20922789888000.0f;  // 1/16!
  c = c * -a2 + 1.0f / 87178291200.0f;
  c = c * -a2 + 1.0f / 479001600.0f;
  c = c * -a2 + 1.0f / 3628800.0f;
  c = c * -a2 + 1.0f / 40320.0f;
  c = c * -a2 + 1.0f / 720.0f;
  c = c * -a2 + 1.0f / 24.0f;
  c = c * a2 - 0.5f;
  c = 1.0f + a2 * c;
  switch (k) {
    case 0: sn = s; cs = c; break;
    case 1: sn = c; cs = -s; break;
    case 2: sn = -s; cs = -c; break;
    default: sn = -c; cs = s; break;
  }
}

// Key of tensor `index` of a synthetic model with `seed`.
LLRS_HD uint64_t tensor_key(uint64_t seed, uint64_t index) {
  return mix64(seed + 0x9E3779B97F4A7C15ull * (index + 1));
}

// The pair of N(0,1) samples for flat elements 2p and 2p+1 of a tensor
// (Box-Muller on two 24-bit uniforms from one 64-bit hash).
LLRS_HD void normal_pair(uint64_t key, uint64_t p, float &z0, float &z1) {
  uint64_t h = mix64(key ^ (p * 0xD1B54A32D192ED03ull + 1));
  float u1 = (float)((h >> 40) + 1) * 5.9604644775390625e-8f;       // (0, 1]
  float u2 = (float)((h >> 16) & 0xffffffu) * 5.9604644775390625e-8f;  // [0, 1)
  float r = sqrtf(-2.0f * ln_unit(u1));
  float sn, cs;
  sincos_turn(u2, sn, cs);
  z0 = r * cs;
  z1 = r * sn;
}

// Value of flat element e of a synthetic tensor: std * z (+1 for a norm gain).
LLRS_HD float synth_value(uint64_t key, uint64_t e, float std_dev, bool gain) {
  float z0, z1;
  normal_pair(key, e >> 1, z0, z1);
  float z = (e & 1) ? z1 : z0;
  return gain ? 1.0f + std_dev * z : std_dev * z;
}

}  // namespace enc
}  // namespace llrs
