// Generic batch-1 dequant-GEMV for every GGML type the reference supports,
// and the bit-exact row dequantizer.
//
// y[r] = sum_c W[r, c] * x[c], the contract of KernelBackend::matvec
// (src/backend.rs:143-162) over dot_row_scalar (src/quant.rs:458-648).
//
// Layout: one wave64 per output row; lane l handles the 32-element units
// l, l+64, ... of the row (a unit is a Q4_0..Q8_0 block, a K-quant sub-block,
// or 32 consecutive F32/F16/BF16 elements), decodes them in registers and
// accumulates in f32; DPP moves and permlane swaps reduce the wave.  This path covers
// all types and shapes; the hot types of the decode step use the tuned
// kernels in gemv_fast.hip.
#include <hip/hip_runtime.h>

#include "common.h"
#include "gemv.h"
#include "quant_dev.h"
#include "wave_dev.h"

namespace llrs {

__device__ __forceinline__ float wave_sum(float v) { return wave_total(v); }

__device__ __forceinline__ float dot32(const float (&w)[32], const float *x) {
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  float a = 0.f;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    float4 v = x4[k];
    a += w[4 * k] * v.x + w[4 * k + 1] * v.y + w[4 * k + 2] * v.z + w[4 * k + 3] * v.w;
  }
  return a;
}

// Decodes the 32 weights of unit u of `row` into w[].
template <uint32_t TY>
__device__ __forceinline__ void decode_unit(const uint8_t *row, int u, float (&w)[32]) {
  if constexpr (TY == LLRS_Q4_0 || TY == LLRS_Q4_1) {
    constexpr int BS = TY == LLRS_Q4_0 ? 18 : 20, QO = TY == LLRS_Q4_0 ? 2 : 4;
    const uint8_t *b = row + (size_t)u * BS;
    float d = ld_f16(b);
    float m = TY == LLRS_Q4_1 ? ld_f16(b + 2) : 0.f;
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      uint16_t p = ld_u16(b + QO + j);
      int q0 = p & 0xff, q1 = p >> 8;
      if constexpr (TY == LLRS_Q4_0) {
        w[j] = d * ((float)(q0 & 15) - 8.f);
        w[j + 1] = d * ((float)(q1 & 15) - 8.f);
        w[j + 16] = d * ((float)(q0 >> 4) - 8.f);
        w[j + 17] = d * ((float)(q1 >> 4) - 8.f);
      } else {
        w[j] = d * (float)(q0 & 15) + m;
        w[j + 1] = d * (float)(q1 & 15) + m;
        w[j + 16] = d * (float)(q0 >> 4) + m;
        w[j + 17] = d * (float)(q1 >> 4) + m;
      }
    }
  } else if constexpr (TY == LLRS_Q5_0 || TY == LLRS_Q5_1) {
    constexpr int BS = TY == LLRS_Q5_0 ? 22 : 24, HO = TY == LLRS_Q5_0 ? 2 : 4,
                  QO = TY == LLRS_Q5_0 ? 6 : 8;
    const uint8_t *b = row + (size_t)u * BS;
    float d = ld_f16(b);
    float m = TY == LLRS_Q5_1 ? ld_f16(b + 2) : 0.f;
    uint32_t qh = (uint32_t)ld_u16(b + HO) | ((uint32_t)ld_u16(b + HO + 2) << 16);
#pragma unroll
    for (int j = 0; j < 16; j += 2) {
      uint16_t p = ld_u16(b + QO + j);
#pragma unroll
      for (int t = 0; t < 2; t++) {
        int byte = (p >> (8 * t)) & 0xff;
        int q0 = (byte & 15) | (((qh >> (j + t)) & 1) << 4);
        int q1 = (byte >> 4) | (((qh >> (j + t + 16)) & 1) << 4);
        if constexpr (TY == LLRS_Q5_0) {
          w[j + t] = d * ((float)q0 - 16.f);
          w[j + t + 16] = d * ((float)q1 - 16.f);
        } else {
          w[j + t] = d * (float)q0 + m;
          w[j + t + 16] = d * (float)q1 + m;
        }
      }
    }
  } else if constexpr (TY == LLRS_Q8_0) {
    const uint8_t *b = row + (size_t)u * 34;
    float d = ld_f16(b);
#pragma unroll
    for (int j = 0; j < 32; j += 2) {
      uint16_t p = ld_u16(b + 2 + j);
      w[j] = d * (float)(int8_t)(p & 0xff);
      w[j + 1] = d * (float)(int8_t)(p >> 8);
    }
  } else if constexpr (TY == LLRS_Q4_K || TY == LLRS_Q5_K) {
    constexpr int BS = TY == LLRS_Q4_K ? 144 : 176, QO = TY == LLRS_Q4_K ? 16 : 48;
    const uint8_t *b = row + (size_t)(u >> 3) * BS;
    int g = u & 7, sc, mn;
    float d = ld_f16(b), dmin = ld_f16(b + 2);
    scale_min_k4(g, b + 4, sc, mn);
    float ds = d * (float)sc, dm = dmin * (float)mn;
    const uint4 *qs = reinterpret_cast<const uint4 *>(b + QO + (g >> 1) * 32);
    uint4 v0 = qs[0], v1 = qs[1];
    uint32_t words[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t hw[8];
    if constexpr (TY == LLRS_Q5_K) {
      const uint4 *qh = reinterpret_cast<const uint4 *>(b + 16);
      uint4 h0 = qh[0], h1 = qh[1];
      hw[0] = h0.x; hw[1] = h0.y; hw[2] = h0.z; hw[3] = h0.w;
      hw[4] = h1.x; hw[5] = h1.y; hw[6] = h1.z; hw[7] = h1.w;
    }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      uint32_t wd = (g & 1) ? (words[k] >> 4) : words[k];
#pragma unroll
      for (int t = 0; t < 4; t++) {
        int q = (wd >> (8 * t)) & 15;
        if constexpr (TY == LLRS_Q5_K) q += ((hw[k] >> (8 * t + g)) & 1) << 4;
        w[4 * k + t] = ds * (float)q - dm;
      }
    }
  } else if constexpr (TY == LLRS_Q6_K) {
    const uint8_t *b = row + (size_t)(u >> 3) * 210;
    int t = u & 7, half = t >> 2, quarter = t & 3;
    float d = ld_f16(b + 208);
    const uint8_t *ql = b + half * 64 + (quarter & 1) * 32;
    const uint8_t *qh = b + 128 + half * 32;
    float s0 = d * (float)(int8_t)b[192 + half * 8 + quarter * 2];
    float s1 = d * (float)(int8_t)b[192 + half * 8 + quarter * 2 + 1];
#pragma unroll
    for (int j = 0; j < 32; j += 2) {
      uint16_t l = ld_u16(ql + j), h = ld_u16(qh + j);
#pragma unroll
      for (int e = 0; e < 2; e++) {
        int lb = (l >> (8 * e)) & 0xff, hb = (h >> (8 * e)) & 0xff;
        int lo = quarter < 2 ? (lb & 15) : (lb >> 4);
        int q = (lo | (((hb >> (2 * quarter)) & 3) << 4)) - 32;
        w[j + e] = (j < 16 ? s0 : s1) * (float)q;
      }
    }
  }
}

template <uint32_t TY>
__device__ __forceinline__ float float_elem(const uint8_t *row, int c) {
  if constexpr (TY == LLRS_F32) return reinterpret_cast<const float *>(row)[c];
  else if constexpr (TY == LLRS_F16) return ld_f16(row + 2 * c);
  else return bf16_bits_to_f32(ld_u16(row + 2 * c));
}

template <uint32_t TY>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const uint8_t *__restrict__ W,
                                                           size_t row_bytes, int rows, int cols,
                                                           const float *__restrict__ x,
                                                           float *__restrict__ y,
                                                           const float *__restrict__ bias,
                                                           int accumulate) {
  int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const uint8_t *row = W + (size_t)r * row_bytes;
  float acc = 0.f;
  if constexpr (TY == LLRS_F32 || TY == LLRS_F16 || TY == LLRS_BF16) {
    for (int c = lane; c < cols; c += 64) acc += float_elem<TY>(row, c) * x[c];
  } else {
    int units = cols / 32;
    for (int u = lane; u < units; u += 64) {
      float w[32];
      decode_unit<TY>(row, u, w);
      acc += dot32(w, x + 32 * u);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    if (bias) acc += bias[r];
    y[r] = accumulate ? y[r] + acc : acc;
  }
}

// F32 / F16 / BF16 rows whose length is a multiple of one 16-byte load
// (4 or 8 elements): each wave owns R consecutive rows, its lanes take the
// row's 16-byte chunks l, l + 64, ..., and every chunk of x (read once per
// wave from L2) serves the R rows.  The loop is unrolled so that several
// chunks' loads are in flight per lane.
template <uint32_t TY, int R>
__global__ __launch_bounds__(256) void gemv_float_kernel(const uint8_t *__restrict__ W, size_t row_bytes,
                                                         int rows, int cols, const float *__restrict__ x,
                                                         float *__restrict__ y,
                                                         const float *__restrict__ bias, int accumulate) {
  constexpr int E = TY == LLRS_F32 ? 4 : 8;  // elements per 16-byte load
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (r0 >= rows) return;
  const int chunks = cols / E;
  float acc[R];
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = 0.f;
#pragma unroll 4
  for (int c = lane; c < chunks; c += 64) {
    uint4 w[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int r = min(r0 + i, rows - 1);  // rows past the end: a valid read, not stored
      w[i] = *reinterpret_cast<const uint4 *>(W + (size_t)r * row_bytes + (size_t)c * 16);
    }
    float xv[E];
#pragma unroll
    for (int k = 0; k < E / 4; k++) {
      const float4 v = *reinterpret_cast<const float4 *>(x + (size_t)c * E + 4 * k);
      xv[4 * k] = v.x;
      xv[4 * k + 1] = v.y;
      xv[4 * k + 2] = v.z;
      xv[4 * k + 3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
      const uint32_t u[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
      for (int e = 0; e < E; e++) {
        float wv;
        if constexpr (TY == LLRS_F32) wv = __uint_as_float(u[e]);
        else if constexpr (TY == LLRS_F16) wv = f16_bits_to_f32((uint16_t)(u[e >> 1] >> (16 * (e & 1))));
        else wv = bf16_bits_to_f32((uint16_t)(u[e >> 1] >> (16 * (e & 1))));
        acc[i] += wv * xv[e];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < R; i++) {
    const float a = wave_sum(acc[i]);
    if (lane == 0 && r0 + i < rows) {
      const float v = bias ? a + bias[r0 + i] : a;
      y[r0 + i] = accumulate ? y[r0 + i] + v : v;
    }
  }
}

__global__ void dequant_row_kernel(const uint8_t *__restrict__ row, uint32_t ty, int cols,
                                   float *__restrict__ out) {
  int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c < cols) out[c] = value_dev(row, ty, (uint32_t)c);
}

int launch_gemv_generic(const llrs_tensor *w, const float *x, float *y, const float *bias,
                        bool accumulate, hipStream_t s) {
  if (w->rows == 0) return LLRS_OK;
  dim3 grid((unsigned)((w->rows + 3) / 4)), block(256);
  int rows = (int)w->rows, cols = (int)w->cols;
  int acc = accumulate ? 1 : 0;
  const bool is_float = w->type == LLRS_F32 || w->type == LLRS_F16 || w->type == LLRS_BF16;
  const int per_load = w->type == LLRS_F32 ? 4 : 8;
  if (is_float && cols % per_load == 0 && w->row_bytes % 16 == 0 &&
      reinterpret_cast<uintptr_t>(w->dev) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
    // Four rows per wave for tall matrices; one otherwise, so that short
    // wide ones still spread over the whole chip.
    const bool four = rows >= 8192;
    const dim3 g((unsigned)((rows + (four ? 15 : 3)) / (four ? 16 : 4)));
#define F(T)                                                                                         \
  case T:                                                                                            \
    if (four)                                                                                        \
      hipLaunchKernelGGL((gemv_float_kernel<T, 4>), g, block, 0, s, w->dev, w->row_bytes, rows, cols, \
                         x, y, bias, acc);                                                           \
    else                                                                                             \
      hipLaunchKernelGGL((gemv_float_kernel<T, 1>), g, block, 0, s, w->dev, w->row_bytes, rows, cols, \
                         x, y, bias, acc);                                                           \
    break;
    switch (w->type) {
      F(LLRS_F32) F(LLRS_F16) F(LLRS_BF16)
      default: break;
    }
#undef F
    LLRS_HIP(hipGetLastError());
    return LLRS_OK;
  }
#define L(T)                                                                                    \
  case T:                                                                                       \
    hipLaunchKernelGGL(gemv_generic_kernel<T>, grid, block, 0, s, w->dev, w->row_bytes, rows, \
                       cols, x, y, bias, acc);                                                  \
    break;
  switch (w->type) {
    L(LLRS_F32) L(LLRS_F16) L(LLRS_BF16) L(LLRS_Q4_0) L(LLRS_Q4_1) L(LLRS_Q5_0) L(LLRS_Q5_1)
    L(LLRS_Q8_0) L(LLRS_Q4_K) L(LLRS_Q5_K) L(LLRS_Q6_K)
    default: return set_error(LLRS_E_UNSUPPORTED, "unsupported GGML type %u", w->type);
  }
#undef L
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_dequant_row(const llrs_tensor *w, size_t row, float *out_dev, hipStream_t s) {
  dim3 block(256), grid((unsigned)((w->cols + 255) / 256));
  hipLaunchKernelGGL(dequant_row_kernel, grid, block, 0, s, w->dev + row * w->row_bytes, w->type,
                     (int)w->cols, out_dev);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

}  // namespace llrs
