// Device-side decoders for the GGML block formats (gfx950).
//
// value_dev() restates value_at (src/quant.rs:349-456) element by element and
// is bit-exact with it: every product in a dequantized value (f16 scale x
// <= 8-bit scale x <= 6-bit code) is exact in f32, so only the final add or
// subtract rounds, in the same order as the reference.  Contraction is
// switched off in these functions anyway so the compiler cannot reassociate.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llrs {

// threadIdx.x, read afresh at each call.  The persistent decode kernel runs
// every phase of a layer inside one loop over the layers; values derived from
// the (loop-invariant) thread index would otherwise be hoisted out of that
// loop and held in registers for all phases at once.
__device__ __forceinline__ int thread_x() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  // v_cvt_f32_f16: exact widening, f16 subnormals preserved (gfx9 default mode).
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  uint32_t bits = (uint32_t)h << 16;
  if ((h & 0x7fffu) > 0x7f80u) bits |= 0x00400000u;  // quiet NaN, as the `half` crate does
  return __builtin_bit_cast(float, bits);
}
__device__ __forceinline__ uint16_t ld_u16(const uint8_t *p) {
  // All GGML block sizes are even, so every 2-byte field is 2-byte aligned.
  return *reinterpret_cast<const uint16_t *>(p);
}
__device__ __forceinline__ float ld_f16(const uint8_t *p) { return f16_bits_to_f32(ld_u16(p)); }

// scale_min_k4 (src/quant.rs:338-347).
__device__ __forceinline__ void scale_min_k4(int i, const uint8_t *s, int &sc, int &mn) {
  if (i < 4) {
    sc = s[i] & 63;
    mn = s[i + 4] & 63;
  } else {
    sc = (s[i + 4] & 0x0f) | ((s[i - 4] >> 6) << 4);
    mn = (s[i + 4] >> 4) | ((s[i] >> 6) << 4);
  }
}

__device__ inline float value_dev(const uint8_t *row, uint32_t ty, uint32_t col) {
#pragma clang fp contract(off)
  switch (ty) {
    case 0: return *reinterpret_cast<const float *>(row + (size_t)col * 4);
    case 1: return ld_f16(row + (size_t)col * 2);
    case 30: return bf16_bits_to_f32(ld_u16(row + (size_t)col * 2));
    case 2: {  // Q4_0
      const uint8_t *b = row + (size_t)(col / 32) * 18;
      uint32_t j = col % 32;
      int q = j < 16 ? (b[2 + j] & 0x0f) : (b[2 + j - 16] >> 4);
      return ld_f16(b) * ((float)q - 8.0f);
    }
    case 3: {  // Q4_1
      const uint8_t *b = row + (size_t)(col / 32) * 20;
      uint32_t j = col % 32;
      int q = j < 16 ? (b[4 + j] & 0x0f) : (b[4 + j - 16] >> 4);
      return ld_f16(b) * (float)q + ld_f16(b + 2);
    }
    case 6:
    case 7: {  // Q5_0 / Q5_1
      uint32_t bsz = ty == 6 ? 22 : 24, qh_off = ty == 6 ? 2 : 4, qs_off = ty == 6 ? 6 : 8;
      const uint8_t *b = row + (size_t)(col / 32) * bsz;
      uint32_t j = col % 32;
      int lo = j < 16 ? (b[qs_off + j] & 0x0f) : (b[qs_off + j - 16] >> 4);
      int hi = (b[qh_off + j / 8] >> (j % 8)) & 1;
      int q = lo | (hi << 4);
      if (ty == 6) return ld_f16(b) * ((float)q - 16.0f);
      return ld_f16(b) * (float)q + ld_f16(b + 2);
    }
    case 8: {  // Q8_0
      const uint8_t *b = row + (size_t)(col / 32) * 34;
      return ld_f16(b) * (float)(int8_t)b[2 + col % 32];
    }
    case 12: {  // Q4_K
      const uint8_t *b = row + (size_t)(col / 256) * 144;
      uint32_t j = col % 256;
      int g = (int)(j / 32), sc, mn;
      scale_min_k4(g, b + 4, sc, mn);
      uint8_t p = b[16 + (g / 2) * 32 + j % 32];
      int q = (g % 2 == 0) ? (p & 0x0f) : (p >> 4);
      return ld_f16(b) * (float)sc * (float)q - ld_f16(b + 2) * (float)mn;
    }
    case 13: {  // Q5_K
      const uint8_t *b = row + (size_t)(col / 256) * 176;
      uint32_t j = col % 256;
      int g = (int)(j / 32), sc, mn;
      scale_min_k4(g, b + 4, sc, mn);
      uint8_t p = b[48 + (g / 2) * 32 + j % 32];
      int lo = (g % 2 == 0) ? (p & 0x0f) : (p >> 4);
      int hi = (b[16 + j % 32] & (1 << g)) ? 16 : 0;
      return ld_f16(b) * (float)sc * (float)(lo + hi) - ld_f16(b + 2) * (float)mn;
    }
    case 14: {  // Q6_K
      const uint8_t *b = row + (size_t)(col / 256) * 210;
      uint32_t j = col % 256;
      uint32_t half = j / 128, within = j % 128, lane = within % 32, quarter = within / 32;
      uint8_t lb = b[half * 64 + (quarter & 1) * 32 + lane];
      int ql = quarter < 2 ? (lb & 0x0f) : (lb >> 4);
      int qh = (b[128 + half * 32 + lane] >> (quarter * 2)) & 3;
      float q = (float)((ql | (qh << 4)) - 32);
      float scale = (float)(int8_t)b[192 + half * 8 + quarter * 2 + lane / 16];
      return ld_f16(b + 208) * scale * q;
    }
    default: return 0.0f;
  }
}

// Loads and stores of activations.  With COH (the persistent decode kernel,
// where producer and consumer run in the same launch on different XCDs) they
// are device-scope relaxed atomics, which go through to memory; otherwise
// plain accesses (kernel boundaries order them).
template <bool COH> __device__ __forceinline__ float ld_act(const float *p) {
  if constexpr (COH)
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    return *p;
}
template <bool COH> __device__ __forceinline__ void st_act(float *p, float v) {
  if constexpr (COH)
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *p = v;
}
template <bool COH> __device__ __forceinline__ float4 ld_act4(const float *p) {
  if constexpr (COH)
    return make_float4(ld_act<true>(p), ld_act<true>(p + 1), ld_act<true>(p + 2), ld_act<true>(p + 3));
  else
    return *reinterpret_cast<const float4 *>(p);
}
template <bool COH> __device__ __forceinline__ uint4 ld_u4(const uint8_t *p) {
  if constexpr (COH) {
    uint32_t *q = reinterpret_cast<uint32_t *>(const_cast<uint8_t *>(p));
    return make_uint4(__hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                      __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                      __hip_atomic_load(q + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                      __hip_atomic_load(q + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  } else {
    return *reinterpret_cast<const uint4 *>(p);
  }
}
template <bool COH> __device__ __forceinline__ void st_u4(uint8_t *p, uint4 v) {
  if constexpr (COH) {
    uint32_t *q = reinterpret_cast<uint32_t *>(p);
    __hip_atomic_store(q, v.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, v.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 2, v.z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 3, v.w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    *reinterpret_cast<uint4 *>(p) = v;
  }
}

// A value with its tag in one single-copy-atomic 64-bit word: producers and
// consumers in one launch (the persistent decode kernel, the attention merge)
// meet without counters.  A consumer reads the word with a device-scope load
// until the high half is the step's tag; no value is ever seen with another
// step's tag.
__device__ __forceinline__ void store_tagged(unsigned long long *p, float v, unsigned tag) {
  __hip_atomic_store(p, ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_tagged(const unsigned long long *p, unsigned tag, bool &ok) {
  const unsigned long long w =
      __hip_atomic_load(const_cast<unsigned long long *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ok = ok && (unsigned)(w >> 32) == tag;
  return __uint_as_float((unsigned)w);
}

// Whether a wait for tagged words has gone on for ~20 ms (the 100 MHz wall
// clock); then *err is set and the waiter goes on with what it read.
__device__ __forceinline__ bool tagged_wait_over(unsigned long long &t0, unsigned *err) {
  const unsigned long long t = wall_clock64();
  if (!t0) t0 = t;
  if (t - t0 < 2000000ull) return false;
  if (err && (thread_x() & 63) == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// A uniform pointer moved into scalar registers (for scalar-memory polls of
// words in uncached device memory).
__device__ __forceinline__ const unsigned *uniform_ptr(const unsigned *p) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(p);
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)a);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(a >> 32));
  return reinterpret_cast<const unsigned *>(((unsigned long long)hi << 32) | lo);
}


typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

// Nine dwords from the dword holding p (p 2-byte aligned): raw[0..8].
__device__ __forceinline__ void load9(const uint8_t *p, uint32_t (&raw)[9], uint32_t &sh) {
  // The aligned pointer is derived from p itself (not from an integer) so the
  // compiler keeps it in the global address space: global_load, not flat_load.
  sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3);  // byte shift for v_alignbyte_b32 (0 or 2)
  const uint32_t *base = reinterpret_cast<const uint32_t *>(p - sh);
  u32x4a4 v0 = *reinterpret_cast<const u32x4a4 *>(base);
  u32x4a4 v1 = *reinterpret_cast<const u32x4a4 *>(base + 4);
  raw[0] = v0.x; raw[1] = v0.y; raw[2] = v0.z; raw[3] = v0.w;
  raw[4] = v1.x; raw[5] = v1.y; raw[6] = v1.z; raw[7] = v1.w;
  raw[8] = base[8];
}
__device__ __forceinline__ uint32_t realign(const uint32_t (&raw)[9], int k, uint32_t sh) {
  return __builtin_amdgcn_alignbyte(raw[k + 1], raw[k], sh);
}

}  // namespace llrs
