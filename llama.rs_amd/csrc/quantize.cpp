// Host-side GGML quantizers: QuantTensor::quantize_{q4k,q5_0,q8_0,q6k}
// (src/quant.rs:187-259) and their block encoders (src/quant.rs:650-967),
// which the reference's loader calls for `--quantize q4k|q4km`
// (src/loader.rs:406-447) and which the synthetic-model generator uses.
//
// Rust semantics kept: f32::round rounds half away from zero (roundf),
// f32::max/min ignore NaN (fmaxf/fminf), float -> int `as` casts saturate
// with NaN -> 0, no fused multiply-add (this file is built with
// -ffp-contract=off), sequential f32 sums, f16 encoding round-to-nearest-even.
#include "quantize.h"

#include <cmath>
#include <cstring>

namespace llrs {

uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    return (uint16_t)(sign | 0x7c00u);
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // >= 65520 rounds to inf
  if (ax < 0x38800000u) {                                     // below 2^-14: subnormal f16
    if (ax < 0x33000000u) return (uint16_t)sign;              // <= 2^-25 rounds to zero
    uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t s = 126 - e;
    uint32_t r = m >> s, rem = m & ((1u << s) - 1), halfway = 1u << (s - 1);
    if (rem > halfway || (rem == halfway && (r & 1))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t r = (ax >> 13) - (112u << 10), rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
  return (uint16_t)(sign | r);
}

float f16_bits_to_f32_host(uint16_t h) {
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
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static inline float f16_round(float v) { return f16_bits_to_f32_host(f32_to_f16_bits(v)); }

static inline void put_f16(std::vector<uint8_t> &out, float v) {
  uint16_t h = f32_to_f16_bits(v);
  out.push_back((uint8_t)(h & 0xff));
  out.push_back((uint8_t)(h >> 8));
}

// Rust `as` casts from f32: saturating, NaN -> 0, truncation toward zero.
static inline uint8_t as_u8(float f) {
  if (std::isnan(f) || f <= 0.f) return 0;
  if (f >= 255.f) return 255;
  return (uint8_t)f;
}
static inline int8_t as_i8(float f) {
  if (std::isnan(f)) return 0;
  if (f <= -128.f) return -128;
  if (f >= 127.f) return 127;
  return (int8_t)f;
}
static inline int32_t as_i32(float f) {
  if (std::isnan(f)) return 0;
  if (f <= -2147483648.f) return INT32_MIN;
  if (f >= 2147483648.f) return INT32_MAX;
  return (int32_t)f;
}
static inline float clampf(float v, float lo, float hi) {
  // f32::clamp: NaN passes through (then the cast maps it to 0).
  if (v < lo) v = lo;
  if (v > hi) v = hi;
  return v;
}

// quantize_block_q8_0 (src/quant.rs:650-662).
static void block_q8_0(const float *v, std::vector<uint8_t> &out) {
  float abs_max = 0.f;
  for (int i = 0; i < 32; i++) abs_max = fmaxf(abs_max, fabsf(v[i]));
  float d = abs_max / 127.0f;
  float inv = d == 0.f ? 0.f : 1.0f / d;
  put_f16(out, d);
  for (int i = 0; i < 32; i++) out.push_back((uint8_t)as_i8(clampf(roundf(v[i] * inv), -127.f, 127.f)));
}

// make_qx_quants_16 (src/quant.rs:726-777).
static float make_qx_quants_16(const float *v, uint8_t *codes) {
  float mx = 0.f, abs_max = 0.f;
  for (int i = 0; i < 16; i++)
    if (fabsf(v[i]) > abs_max) {
      abs_max = fabsf(v[i]);
      mx = v[i];
    }
  if (abs_max < 1e-15f) {
    memset(codes, 0, 16);
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

// quantize_block_q6k (src/quant.rs:664-724).
static void block_q6k(const float *v, std::vector<uint8_t> &out) {
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
    out.insert(out.end(), 210, 0);
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
  uint8_t low[128], high[64];
  for (int half = 0; half < 2; half++) {
    int base = half * 128;
    for (int lane = 0; lane < 32; lane++) {
      uint8_t q1 = codes[base + lane], q2 = codes[base + 32 + lane], q3 = codes[base + 64 + lane],
              q4 = codes[base + 96 + lane];
      low[half * 64 + lane] = (uint8_t)((q1 & 0x0f) | ((q3 & 0x0f) << 4));
      low[half * 64 + 32 + lane] = (uint8_t)((q2 & 0x0f) | ((q4 & 0x0f) << 4));
      high[half * 32 + lane] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
    }
  }
  out.insert(out.end(), low, low + 128);
  out.insert(out.end(), high, high + 64);
  for (int g = 0; g < 16; g++) out.push_back((uint8_t)scale_codes[g]);
  put_f16(out, d);
}

// quantize_block_q5_0 (src/quant.rs:779-807).
static void block_q5_0(const float *v, std::vector<uint8_t> &out) {
  float max_value = 0.f, abs_max = 0.f;
  for (int i = 0; i < 32; i++)
    if (fabsf(v[i]) > abs_max) {
      abs_max = fabsf(v[i]);
      max_value = v[i];
    }
  float d = abs_max == 0.f ? 0.f : max_value / -16.0f;
  float inv = d == 0.f ? 0.f : 1.0f / d;
  put_f16(out, d);
  size_t qh_pos = out.size();
  out.insert(out.end(), 4, 0);
  uint32_t high = 0;
  for (int j = 0; j < 16; j++) {
    uint8_t q0 = as_u8(clampf(floorf(v[j] * inv + 16.5f), 0.f, 31.f));
    uint8_t q1 = as_u8(clampf(floorf(v[j + 16] * inv + 16.5f), 0.f, 31.f));
    out.push_back((uint8_t)((q0 & 0x0f) | ((q1 & 0x0f) << 4)));
    high |= (((uint32_t)q0 >> 4) & 1) << j;
    high |= (((uint32_t)q1 >> 4) & 1) << (j + 16);
  }
  for (int k = 0; k < 4; k++) out[qh_pos + k] = (uint8_t)(high >> (8 * k));
}

// make_qkx2_quants (src/quant.rs:892-967).
static float make_qkx2_quants(const float *v, const float *w, uint8_t *codes, float *out_min,
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
    memset(codes, 0, 32);
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
        memcpy(codes, aux, 32);
        best_error = err;
        scale = cs;
        mn = cm;
      }
    }
  }
  *out_min = -mn;
  return scale;
}

// quantize_block_q4k (src/quant.rs:809-890).
static void block_q4k(const float *v, std::vector<uint8_t> &out) {
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
  put_f16(out, dmin);
  out.insert(out.end(), scales, scales + 12);
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
      out.push_back((uint8_t)(codes[pair * 64 + i] | (codes[pair * 64 + 32 + i] << 4)));
}

uint32_t quantize_rows(uint32_t requested, const float *values, size_t rows, size_t cols,
                       std::vector<uint8_t> &out) {
  uint32_t ty = requested;
  // Fallback rules of quantize_q4k / quantize_q6k / quantize_q5_0 / quantize_q8_0.
  if (ty == LLRS_Q4_K && cols % 256) ty = LLRS_Q5_0;
  if (ty == LLRS_Q6_K && cols % 256) ty = LLRS_Q8_0;
  if ((ty == LLRS_Q5_0 || ty == LLRS_Q8_0) && cols % 32) ty = LLRS_F32;
  out.clear();
  if (ty == LLRS_F32) {
    out.resize(rows * cols * 4);
    memcpy(out.data(), values, rows * cols * 4);
    return ty;
  }
  out.reserve(row_bytes(ty, cols) * rows);
  for (size_t r = 0; r < rows; r++) {
    const float *row = values + r * cols;
    switch (ty) {
      case LLRS_Q4_K: for (size_t c = 0; c < cols; c += 256) block_q4k(row + c, out); break;
      case LLRS_Q6_K: for (size_t c = 0; c < cols; c += 256) block_q6k(row + c, out); break;
      case LLRS_Q5_0: for (size_t c = 0; c < cols; c += 32) block_q5_0(row + c, out); break;
      case LLRS_Q8_0: for (size_t c = 0; c < cols; c += 32) block_q8_0(row + c, out); break;
      default: break;
    }
  }
  return ty;
}

}  // namespace llrs

extern "C" int llrs_quantize(uint32_t ggml_type, const float *values, size_t rows, size_t cols,
                             void *out, size_t out_capacity, size_t *out_nbytes,
                             uint32_t *out_type) {
  using namespace llrs;
  clear_error();
  if (ggml_type != LLRS_Q4_K && ggml_type != LLRS_Q5_0 && ggml_type != LLRS_Q8_0 &&
      ggml_type != LLRS_Q6_K)
    return set_error(LLRS_E_UNSUPPORTED, "llrs_quantize supports Q4_K, Q5_0, Q8_0 and Q6_K");
  if (!values && rows * cols) return set_error(LLRS_E_INVALID, "values is NULL");
  uint32_t ty = ggml_type;
  if (ty == LLRS_Q4_K && cols % 256) ty = LLRS_Q5_0;
  if (ty == LLRS_Q6_K && cols % 256) ty = LLRS_Q8_0;
  if ((ty == LLRS_Q5_0 || ty == LLRS_Q8_0) && cols % 32) ty = LLRS_F32;
  size_t need = ty == LLRS_F32 ? rows * cols * 4 : row_bytes(ty, cols) * rows;
  if (out_nbytes) *out_nbytes = need;
  if (out_type) *out_type = ty;
  if (!out) return LLRS_OK;
  if (out_capacity < need)
    return set_error(LLRS_E_INVALID, "output capacity %zu < %zu", out_capacity, need);
  std::vector<uint8_t> buf;
  quantize_rows(ggml_type, values, rows, cols, buf);
  memcpy(out, buf.data(), need);
  return LLRS_OK;
}
