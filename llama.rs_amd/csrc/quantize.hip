// Synthetic-weight generation + quantization and load-time encoding on the
// GPU (the host side is quantize_host.cpp).  Both use the shared encoders and
// RNG of quant_encode.h; this file is compiled with -ffp-contract=off for
// host and device, so both sides emit identical bytes.
#include <hip/hip_runtime.h>

#include <cstring>

#include "common.h"
#include "quant_encode.h"
#include "quantize.h"

namespace llrs {

// One thread per GGML block: generate its values from the tensor's RNG key
// and encode them.  ty is a quantized type (or F32 for one value per thread).
template <uint32_t TY>
__global__ __launch_bounds__(64) void synth_encode_kernel(uint64_t key, uint64_t rows, uint64_t cols,
                                                          float sd, int gain, uint8_t *out,
                                                          uint64_t rbytes) {
  constexpr int BS = TY == LLRS_Q4_K || TY == LLRS_Q6_K ? 256 : TY == LLRS_F32 ? 1 : 32;
  constexpr int TS = TY == LLRS_Q4_K ? 144 : TY == LLRS_Q6_K ? 210 : TY == LLRS_Q5_0 ? 22
                     : TY == LLRS_Q8_0 ? 34 : 4;
  uint64_t per_row = cols / BS, total = rows * per_row;
  for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < total;
       b += (uint64_t)gridDim.x * blockDim.x) {
    uint64_t r = b / per_row, j = b % per_row;
    uint64_t e0 = r * cols + j * BS;
    uint8_t *dst = out + r * rbytes + j * TS;
    if constexpr (TY == LLRS_F32) {
      float v = enc::synth_value(key, e0, sd, gain != 0);
      memcpy(dst, &v, 4);
    } else {
      float v[BS];
      for (int i = 0; i < BS; i++) v[i] = enc::synth_value(key, e0 + i, sd, gain != 0);
      if constexpr (TY == LLRS_Q4_K) enc::block_q4k(v, dst);
      else if constexpr (TY == LLRS_Q6_K) enc::block_q6k(v, dst);
      else if constexpr (TY == LLRS_Q5_0) enc::block_q5_0(v, dst);
      else enc::block_q8_0(v, dst);
    }
  }
}

// Quantizes device f32 rows with the encoders (GPU load-time quantization).
template <uint32_t TY>
__global__ __launch_bounds__(64) void encode_kernel(const float *__restrict__ vals, uint64_t rows,
                                                    uint64_t cols, uint8_t *out, uint64_t rbytes) {
  constexpr int BS = TY == LLRS_Q4_K || TY == LLRS_Q6_K ? 256 : 32;
  constexpr int TS = TY == LLRS_Q4_K ? 144 : TY == LLRS_Q6_K ? 210 : TY == LLRS_Q5_0 ? 22 : 34;
  uint64_t per_row = cols / BS, total = rows * per_row;
  for (uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; b < total;
       b += (uint64_t)gridDim.x * blockDim.x) {
    uint64_t r = b / per_row, j = b % per_row;
    float v[BS];
    for (int i = 0; i < BS; i++) v[i] = vals[r * cols + j * BS + i];
    uint8_t *dst = out + r * rbytes + j * TS;
    if constexpr (TY == LLRS_Q4_K) enc::block_q4k(v, dst);
    else if constexpr (TY == LLRS_Q6_K) enc::block_q6k(v, dst);
    else if constexpr (TY == LLRS_Q5_0) enc::block_q5_0(v, dst);
    else enc::block_q8_0(v, dst);
  }
}

// F16 / BF16 values widened to f32 with the host loader's conversions (a
// bf16 NaN gets the quiet bit, as the host path sets it).
__global__ void widen_kernel(uint32_t ty, const uint16_t *__restrict__ src, uint64_t n,
                             float *__restrict__ dst) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint16_t h = src[i];
    if (ty == LLRS_F16) {
      dst[i] = enc::f16_to_f32(h);
    } else {
      uint32_t b = (uint32_t)h << 16;
      if ((h & 0x7fffu) > 0x7f80u) b |= 0x00400000u;
      dst[i] = enc::u2f(b);
    }
  }
}

static dim3 grid_for(uint64_t n) {
  uint64_t g = (n + 63) / 64;
  if (g > 65536) g = 65536;
  if (g == 0) g = 1;
  return dim3((unsigned)g);
}

int launch_synth_encode(uint32_t ty, uint64_t key, size_t rows, size_t cols, float sd, bool gain,
                        uint8_t *out, size_t rbytes, hipStream_t s) {
  uint64_t n = ty == LLRS_F32 ? rows * cols : rows * (cols / (size_t)block_size(ty));
  dim3 g = grid_for(n), b(64);
  int gi = gain ? 1 : 0;
  switch (ty) {
    case LLRS_F32: hipLaunchKernelGGL(synth_encode_kernel<LLRS_F32>, g, b, 0, s, key, rows, cols, sd, gi, out, rbytes); break;
    case LLRS_Q4_K: hipLaunchKernelGGL(synth_encode_kernel<LLRS_Q4_K>, g, b, 0, s, key, rows, cols, sd, gi, out, rbytes); break;
    case LLRS_Q6_K: hipLaunchKernelGGL(synth_encode_kernel<LLRS_Q6_K>, g, b, 0, s, key, rows, cols, sd, gi, out, rbytes); break;
    case LLRS_Q5_0: hipLaunchKernelGGL(synth_encode_kernel<LLRS_Q5_0>, g, b, 0, s, key, rows, cols, sd, gi, out, rbytes); break;
    case LLRS_Q8_0: hipLaunchKernelGGL(synth_encode_kernel<LLRS_Q8_0>, g, b, 0, s, key, rows, cols, sd, gi, out, rbytes); break;
    default: return set_error(LLRS_E_UNSUPPORTED, "cannot synthesize %s", type_name(ty));
  }
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_encode(uint32_t ty, const float *vals, size_t rows, size_t cols, uint8_t *out,
                  size_t rbytes, hipStream_t s) {
  uint64_t n = rows * (cols / (size_t)block_size(ty));
  dim3 g = grid_for(n), b(64);
  switch (ty) {
    case LLRS_Q4_K: hipLaunchKernelGGL(encode_kernel<LLRS_Q4_K>, g, b, 0, s, vals, rows, cols, out, rbytes); break;
    case LLRS_Q6_K: hipLaunchKernelGGL(encode_kernel<LLRS_Q6_K>, g, b, 0, s, vals, rows, cols, out, rbytes); break;
    case LLRS_Q5_0: hipLaunchKernelGGL(encode_kernel<LLRS_Q5_0>, g, b, 0, s, vals, rows, cols, out, rbytes); break;
    case LLRS_Q8_0: hipLaunchKernelGGL(encode_kernel<LLRS_Q8_0>, g, b, 0, s, vals, rows, cols, out, rbytes); break;
    default: return set_error(LLRS_E_UNSUPPORTED, "cannot encode %s", type_name(ty));
  }
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_widen(uint32_t ty, const void *src, size_t n, float *dst, hipStream_t s) {
  if (ty != LLRS_F16 && ty != LLRS_BF16) return set_error(LLRS_E_UNSUPPORTED, "cannot widen %s", type_name(ty));
  uint64_t g = (n + 255) / 256;
  g = g > 8192 ? 8192 : g ? g : 1;
  hipLaunchKernelGGL(widen_kernel, dim3((unsigned)g), dim3(256), 0, s, ty, (const uint16_t *)src,
                     (uint64_t)n, dst);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

}  // namespace llrs
