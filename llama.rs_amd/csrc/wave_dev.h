// Lane exchanges within a wave of 64 on gfx950 that stay in the VALU.
//
// __shfl_xor compiles to ds_bpermute_b32, a trip through the LDS unit per
// exchange, and the reduction trees of the decode step chain five or six of
// them.  DPP moves within 16-lane rows and v_permlane16_swap /
// v_permlane32_swap across rows cost VALU latency instead.
//
// lane_partner(v, b) returns the value of lane `lane ^ p(b)`, for a single
// bit b of the lane index: p(1) = 1 and p(2) = 2 (DPP quad_perm), p(4) = 7
// (row_half_mirror: lane 7 - i within each 8), p(8) = 15 (row_mirror: lane
// 15 - i within each 16), p(16) = 16 and p(32) = 32 (the permlane swaps).
// p(b) flips bit b and no bit above it, so a reduce-scatter that handles
// bits from high to low (each level keeping the half its own bit b selects
// and adding the partner's copy of it) pairs lanes that agree on the bits
// already handled; and p(1) .. p(32) span the lane index, so a full sum or
// max over these partners reaches every lane once.  Results land in the
// same lanes as with xor partners; only the order of the additions differs.
// Partners compute a + b and b + a, so every lane of a full sum holds the
// same bits.
#pragma once

#include <hip/hip_runtime.h>

namespace llrs {

namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// The value of lane lane ^ 16: v_permlane16_swap with both operands v
// returns (rows 0, 0, 2, 2) and (rows 1, 1, 3, 3) of v.
__device__ __forceinline__ float lane_swap16(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 16) ? p[0] : p[1]);
}

// The value of lane lane ^ 32: v_permlane32_swap with both operands v
// returns (low half, low half) and (high half, high half) of v.
__device__ __forceinline__ float lane_swap32(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v), __builtin_bit_cast(unsigned, v),
                                                  false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? p[0] : p[1]);
}

// b: 1, 2, 4, 8, 16 or 32 (a compile-time constant once the caller's loop
// is unrolled).
__device__ __forceinline__ float lane_partner(float v, int b) {
  if (b == 1) return dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  if (b == 2) return dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  if (b == 4) return dpp_mov<0x141>(v);  // row_half_mirror
  if (b == 8) return dpp_mov<0x140>(v);  // row_mirror
  if (b == 16) return lane_swap16(v);
  return lane_swap32(v);
}

// Sum and max over the whole wave, in every lane.
__device__ __forceinline__ float wave_total(float v) {
#pragma unroll
  for (int b = 1; b < 64; b <<= 1) v += lane_partner(v, b);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int b = 1; b < 64; b <<= 1) v = fmaxf(v, lane_partner(v, b));
  return v;
}

}  // namespace

}  // namespace llrs
