// Device side of the tuned batch-1 dequant-GEMV for the decode step's weight
// types (Q4_K, Q6_K, Q8_0, Q5_0) with fused prologue (RMSNorm) and epilogues
// (bias, residual add, SiLU(gate)*up, LM-head logits + greedy argmax): the
// per-type decoders, the streaming loop and one launch's work (GemvPhase),
// shared by the GEMV kernel and the persistent decode kernel.
//
// y[r] = sum_c W[r, c] * x[c] (KernelBackend::matvec, src/backend.rs:143-162;
// dot_row_scalar, src/quant.rs:458-648).
//
// Activation digits.  Each workgroup converts x (optionally x * norm_gain) to
// int8 "digits" in LDS: per 16-element block b with scale s_b = max|x|/127,
//     x_j ~= s_b / 128 * X_j,   X_j = 128 d1_j + d2_j,
// d1 in [-127, 127], d2 in [-64, 64] (|error| <= 1/256 of s_b, 3.1e-5 of the
// block maximum).  Weight codes stay in their native GGUF blocks and are
// multiplied with the digits by v_dot4_i32_i8 (4 int8 MACs per instruction,
// exact int32 accumulation, Horner over the two planes); per-block f16 scales
// and x-block scales are applied in f32.  Mins/offsets use the exact integer
// sums of X per block.  In LDS, x-block b lives at slot (b % 4) * (nb / 4) +
// b / 4, so the lanes of a wave read consecutive 16-byte slots.
//
// Work split.  Workgroup w owns whole row quads [w*Q/G, (w+1)*Q/G); each wave
// takes one quad at a time, its 64 lanes splitting the row's blocks ("units"),
// so a lane's digits serve four rows.  The raw weight loads of the next
// (quad, unit) step are issued before the current step is computed.
// Q8_0/Q5_0/Q6_K blocks have even but not 4-byte-aligned offsets: their
// fields are loaded as aligned dwords and realigned with v_alignbyte_b32.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"
#include "gemv.h"
#include "quant_dev.h"
#include "wave_dev.h"

namespace llrs {

namespace {


struct Lds {
  const int8_t *dig;  // [2][cols] digit planes, x-blocks permuted by slot()
  const float *xs;    // [nb] s_b / 128 (slot order)
  const int *sx;      // [nb] sum of X over the block (slot order)
  const float *xsum32;  // [cols/32] sum of reconstructed x per 32 columns
  int cols, nb4;        // nb4 = number of x-blocks / 4
};

// LDS bytes of the digitised activation: 2 digit planes, per-block scales and
// sums, per-32 sums.
__host__ __device__ constexpr size_t fast_gemv_digit_bytes(int cols) {
  return (size_t)2 * cols + (size_t)(cols >> 4) * 8 + (size_t)(cols >> 5) * 4;
}
constexpr size_t kMaxLds = 160 * 1024;

__device__ __forceinline__ int slot(int b, int nb4) { return (b & 3) * nb4 + (b >> 2); }

__device__ __forceinline__ int sdot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}
// Digits (2 planes) of x-block b for the lane, as 4 dwords each.
__device__ __forceinline__ void dig_block(const Lds &L, int b, uint4 (&d)[2]) {
  int s = slot(b, L.nb4) * 16;
#pragma unroll
  for (int p = 0; p < 2; p++) d[p] = *reinterpret_cast<const uint4 *>(L.dig + p * L.cols + s);
}

// sum_j q_j X_j over one x-block (16 weights packed as 4 dwords of int8
// codes): Horner over the digit planes, X = 128 d1 + d2, exact in int32.
__device__ __forceinline__ int block_dot(int q0, int q1, int q2, int q3, const uint4 (&d)[2]) {
  int a = sdot4(q0, (int)d[0].x, 0);
  a = sdot4(q1, (int)d[0].y, a);
  a = sdot4(q2, (int)d[0].z, a);
  a = sdot4(q3, (int)d[0].w, a);
  a = sdot4(q0, (int)d[1].x, a << 7);
  a = sdot4(q1, (int)d[1].y, a);
  a = sdot4(q2, (int)d[1].z, a);
  return sdot4(q3, (int)d[1].w, a);
}

// ------------------------------------------------------------------ per type
// Traits<TY>: units per row; Raw = raw loads of one row for one unit; load();
// Dig = the lane's digits of one unit; digits(); dot() = contribution of one
// row's unit.

template <uint32_t TY> struct Traits;

// scale_min_k4 (src/quant.rs:338-347) of groups 2p, 2p+1 of a K-quant
// header (d, dmin, 12 scale bytes) as byte pairs: groups < 4 keep 6 bits of
// scales[g] / scales[g+4]; groups >= 4 join the nibbles of scales[g+4] with
// the top two bits of scales[g-4] / scales[g].  Both forms are computed and
// blended by a lane mask (a branch would run both sides under exec masking).
__device__ __forceinline__ void k4_scales(const uint4 &hdr, int p, uint32_t &sc, uint32_t &mn) {
  const int sh = (p & 1) * 16;
  const uint32_t Y = hdr.y >> sh, Z = hdr.z >> sh, W = hdr.w >> sh;
  const uint32_t hi_g = 0u - (uint32_t)(p >> 1);  // all ones for groups >= 4
  sc = ((Y & 0x3f3fu) & ~hi_g) | (((W & 0x0f0fu) | ((Y >> 2) & 0x3030u)) & hi_g);
  mn = ((Z & 0x3f3fu) & ~hi_g) | ((((W >> 4) & 0x0f0fu) | ((Z >> 2) & 0x3030u)) & hi_g);
}

// Bits 0..3 of t -> bit 4 of bytes 0..3 (a Q5 block's high bits of four
// consecutive weights).
__device__ __forceinline__ uint32_t spread4(uint32_t t) {
  return ((t & 15u) * 0x00204081u & 0x01010101u) << 4;
}

// Q4_K: unit u = block u/4, sub-block pair p = u%4 (groups 2p, 2p+1 = 64
// weights, x-blocks 4u .. 4u+3).  y += d*sc_g * sum(q x) - dmin*m_g * sum(x).
template <> struct Traits<LLRS_Q4_K> {
  static constexpr int kColsPerUnit = 64;
  struct Raw { uint4 hdr, q0, q1; };
  struct Dig { uint4 g[4][2]; float xs[4]; float xsum[2]; };
  static __device__ __forceinline__ void load(const uint8_t *row, int u, Raw &r) {
    const uint8_t *blk = row + (size_t)(u >> 2) * 144;
    int p = u & 3;
    r.hdr = *reinterpret_cast<const uint4 *>(blk);
    r.q0 = *reinterpret_cast<const uint4 *>(blk + 16 + p * 32);
    r.q1 = *reinterpret_cast<const uint4 *>(blk + 32 + p * 32);
  }
  static __device__ __forceinline__ void digits(const Lds &L, int u, Dig &D) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      dig_block(L, 4 * u + j, D.g[j]);
      D.xs[j] = L.xs[slot(4 * u + j, L.nb4)];
    }
    D.xsum[0] = L.xsum32[2 * u];
    D.xsum[1] = L.xsum32[2 * u + 1];
  }
  static __device__ __forceinline__ float dot(const Raw &r, int u, const Dig &D) {
    const int p = u & 3;
    const float d = f16_bits_to_f32((uint16_t)(r.hdr.x & 0xffff));
    const float dmin = f16_bits_to_f32((uint16_t)(r.hdr.x >> 16));
    uint32_t sc, mn;
    k4_scales(r.hdr, p, sc, mn);
    // Blocks: group 2p = low nibbles of q0 then q1, group 2p+1 = high nibbles.
    const uint32_t m4 = 0x0f0f0f0fu;
    const int a0 = block_dot(r.q0.x & m4, r.q0.y & m4, r.q0.z & m4, r.q0.w & m4, D.g[0]);
    const int a1 = block_dot(r.q1.x & m4, r.q1.y & m4, r.q1.z & m4, r.q1.w & m4, D.g[1]);
    const int a2 = block_dot((r.q0.x >> 4) & m4, (r.q0.y >> 4) & m4, (r.q0.z >> 4) & m4,
                             (r.q0.w >> 4) & m4, D.g[2]);
    const int a3 = block_dot((r.q1.x >> 4) & m4, (r.q1.y >> 4) & m4, (r.q1.z >> 4) & m4,
                             (r.q1.w >> 4) & m4, D.g[3]);
    const float s0 = (float)a0 * D.xs[0] + (float)a1 * D.xs[1];
    const float s1 = (float)a2 * D.xs[2] + (float)a3 * D.xs[3];
    const float t = (float)(sc & 0xff) * s0 + (float)(sc >> 8) * s1;
    const float m = (float)(mn & 0xff) * D.xsum[0] + (float)(mn >> 8) * D.xsum[1];
    return d * t - dmin * m;
  }
};

// Q6_K: unit u = block u/4, half h = (u%4)/2, j = u%2: quarters j and j+2 of
// that half (64 weights sharing 32 ql bytes and the half's 32 qh bytes).
template <> struct Traits<LLRS_Q6_K> {
  static constexpr int kColsPerUnit = 64;
  struct Raw { uint32_t ql[9], qh[9]; uint32_t shl, shh; uint32_t sc; uint16_t d; };
  struct Dig { uint4 g[4][2]; float xs[4]; int sx[4]; };
  static __device__ __forceinline__ int xb(int u, int i) {  // x-block i of unit u
    int h = (u & 3) >> 1, j = u & 1;
    return (u >> 2) * 16 + h * 8 + j * 2 + (i >> 1) * 4 + (i & 1);
  }
  static __device__ __forceinline__ void load(const uint8_t *row, int u, Raw &r) {
    const uint8_t *blk = row + (size_t)(u >> 2) * 210;
    int h = (u & 3) >> 1, j = u & 1;
    load9(blk + h * 64 + j * 32, r.ql, r.shl);
    load9(blk + 128 + h * 32, r.qh, r.shh);
    r.sc = (uint32_t)ld_u16(blk + 192 + h * 8 + 2 * j) |
           ((uint32_t)ld_u16(blk + 192 + h * 8 + 2 * j + 4) << 16);
    r.d = ld_u16(blk + 208);
  }
  static __device__ __forceinline__ void digits(const Lds &L, int u, Dig &D) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int b = xb(u, i), s = slot(b, L.nb4);
      dig_block(L, b, D.g[i]);
      D.xs[i] = L.xs[s];
      D.sx[i] = L.sx[s];
    }
  }
  static __device__ __forceinline__ float dot(const Raw &r, int u, const Dig &D) {
    const int j = u & 1, sh_a = 2 * j, sh_b = 2 * j + 4;
    int qa[8], qb[8];  // 6-bit codes of quarters j and j+2, 4 per dword
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t ql = realign(r.ql, k, r.shl), qh = realign(r.qh, k, r.shh);
      qa[k] = (int)((ql & 0x0f0f0f0fu) | (((qh >> sh_a) & 0x03030303u) << 4));
      qb[k] = (int)(((ql >> 4) & 0x0f0f0f0fu) | (((qh >> sh_b) & 0x03030303u) << 4));
    }
    const int acc[4] = {block_dot(qa[0], qa[1], qa[2], qa[3], D.g[0]),
                        block_dot(qa[4], qa[5], qa[6], qa[7], D.g[1]),
                        block_dot(qb[0], qb[1], qb[2], qb[3], D.g[2]),
                        block_dot(qb[4], qb[5], qb[6], qb[7], D.g[3])};
    float y = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // (q - 32) * X summed = sum q*X - 32 * sum X, exact in int32.
      const int I = acc[i] - 32 * D.sx[i];
      const int s8 = (int)(int8_t)((r.sc >> (8 * i)) & 0xff);  // i: j/0, j/1, j+2/0, j+2/1
      y += (float)s8 * ((float)I * D.xs[i]);
    }
    return f16_bits_to_f32(r.d) * y;
  }
};

// Q8_0: unit u = block u (32 weights, x-blocks 2u, 2u+1).
template <> struct Traits<LLRS_Q8_0> {
  static constexpr int kColsPerUnit = 32;
  struct Raw { uint32_t q[9]; uint32_t sh; uint16_t d; };
  struct Dig { uint4 g[2][2]; float xs[2]; };
  static __device__ __forceinline__ void load(const uint8_t *row, int u, Raw &r) {
    const uint8_t *blk = row + (size_t)u * 34;
    load9(blk + 2, r.q, r.sh);
    r.d = ld_u16(blk);
  }
  static __device__ __forceinline__ void digits(const Lds &L, int u, Dig &D) {
#pragma unroll
    for (int e = 0; e < 2; e++) {
      dig_block(L, 2 * u + e, D.g[e]);
      D.xs[e] = L.xs[slot(2 * u + e, L.nb4)];
    }
  }
  static __device__ __forceinline__ float dot(const Raw &r, int, const Dig &D) {
    int q[8];
#pragma unroll
    for (int k = 0; k < 8; k++) q[k] = (int)realign(r.q, k, r.sh);
    const int a0 = block_dot(q[0], q[1], q[2], q[3], D.g[0]);
    const int a1 = block_dot(q[4], q[5], q[6], q[7], D.g[1]);
    return f16_bits_to_f32(r.d) * ((float)a0 * D.xs[0] + (float)a1 * D.xs[1]);
  }
};

// Q5_0: unit u = block u (32 weights): d, qh (32 high bits), 16 bytes of nibbles.
template <> struct Traits<LLRS_Q5_0> {
  static constexpr int kColsPerUnit = 32;
  struct Raw { uint32_t w[6]; uint32_t sh; uint16_t d; };
  struct Dig { uint4 g[2][2]; float xs[2]; int sx[2]; };
  static __device__ __forceinline__ void load(const uint8_t *row, int u, Raw &r) {
    const uint8_t *blk = row + (size_t)u * 22;
    r.sh = (uint32_t)(reinterpret_cast<uintptr_t>(blk + 2) & 3);
    const uint32_t *base = reinterpret_cast<const uint32_t *>(blk + 2 - r.sh);
    u32x4a4 v0 = *reinterpret_cast<const u32x4a4 *>(base);
    r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
    r.w[4] = base[4];
    r.w[5] = base[5];
    r.d = ld_u16(blk);
  }
  static __device__ __forceinline__ void digits(const Lds &L, int u, Dig &D) {
#pragma unroll
    for (int e = 0; e < 2; e++) {
      int s = slot(2 * u + e, L.nb4);
      dig_block(L, 2 * u + e, D.g[e]);
      D.xs[e] = L.xs[s];
      D.sx[e] = L.sx[s];
    }
  }
  static __device__ __forceinline__ float dot(const Raw &r, int, const Dig &D) {
    const uint32_t qh = __builtin_amdgcn_alignbyte(r.w[1], r.w[0], r.sh);
    int qa[4], qb[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t v = __builtin_amdgcn_alignbyte(r.w[k + 2], r.w[k + 1], r.sh);
      qa[k] = (int)((v & 0x0f0f0f0fu) | spread4(qh >> (4 * k)));
      qb[k] = (int)(((v >> 4) & 0x0f0f0f0fu) | spread4(qh >> (16 + 4 * k)));
    }
    // d * (q - 16) summed against x.
    const int I0 = block_dot(qa[0], qa[1], qa[2], qa[3], D.g[0]) - 16 * D.sx[0];
    const int I1 = block_dot(qb[0], qb[1], qb[2], qb[3], D.g[1]) - 16 * D.sx[1];
    return f16_bits_to_f32(r.d) * ((float)I0 * D.xs[0] + (float)I1 * D.xs[1]);
  }
};

// Q4_0: unit u = block u (32 weights): d, 16 bytes of nibbles (weight j < 16
// the low nibble of byte j, weight 16 + j its high nibble); d * (q - 8).
template <> struct Traits<LLRS_Q4_0> {
  static constexpr int kColsPerUnit = 32;
  struct Raw { uint32_t w[5]; uint32_t sh; uint16_t d; };
  struct Dig { uint4 g[2][2]; float xs[2]; int sx[2]; };
  static __device__ __forceinline__ void load(const uint8_t *row, int u, Raw &r) {
    const uint8_t *blk = row + (size_t)u * 18;
    r.sh = (uint32_t)(reinterpret_cast<uintptr_t>(blk + 2) & 3);
    const uint32_t *base = reinterpret_cast<const uint32_t *>(blk + 2 - r.sh);
    u32x4a4 v0 = *reinterpret_cast<const u32x4a4 *>(base);
    r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
    r.w[4] = base[4];
    r.d = ld_u16(blk);
  }
  static __device__ __forceinline__ void digits(const Lds &L, int u, Dig &D) {
#pragma unroll
    for (int e = 0; e < 2; e++) {
      int s = slot(2 * u + e, L.nb4);
      dig_block(L, 2 * u + e, D.g[e]);
      D.xs[e] = L.xs[s];
      D.sx[e] = L.sx[s];
    }
  }
  static __device__ __forceinline__ float dot(const Raw &r, int, const Dig &D) {
    const uint32_t m4 = 0x0f0f0f0fu;
    int qa[4], qb[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t v = __builtin_amdgcn_alignbyte(r.w[k + 1], r.w[k], r.sh);
      qa[k] = (int)(v & m4);
      qb[k] = (int)((v >> 4) & m4);
    }
    const int I0 = block_dot(qa[0], qa[1], qa[2], qa[3], D.g[0]) - 8 * D.sx[0];
    const int I1 = block_dot(qb[0], qb[1], qb[2], qb[3], D.g[1]) - 8 * D.sx[1];
    return f16_bits_to_f32(r.d) * ((float)I0 * D.xs[0] + (float)I1 * D.xs[1]);
  }
};

// Q4_1 (20-byte blocks) and Q5_1 (24): unit u = block u (32 weights): d, m,
// for Q5_1 32 high bits, then 16 bytes of nibbles; d * q + m.  The blocks and
// so the rows are 4-byte aligned: fields load as dwords.
template <uint32_t TY> struct TraitsQx1 {
  static constexpr bool kQ5 = TY == LLRS_Q5_1;
  static constexpr int kColsPerUnit = 32, kBytes = kQ5 ? 24 : 20;
  struct Raw { uint32_t dm, qh, q[4]; };
  struct Dig { uint4 g[2][2]; float xs[2]; float xsum; };
  static __device__ __forceinline__ void load(const uint8_t *row, int u, Raw &r) {
    const uint32_t *blk = reinterpret_cast<const uint32_t *>(row + (size_t)u * kBytes);
    r.dm = blk[0];
    r.qh = kQ5 ? blk[1] : 0u;
    u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(blk + (kQ5 ? 2 : 1));
    r.q[0] = v.x; r.q[1] = v.y; r.q[2] = v.z; r.q[3] = v.w;
  }
  static __device__ __forceinline__ void digits(const Lds &L, int u, Dig &D) {
#pragma unroll
    for (int e = 0; e < 2; e++) {
      dig_block(L, 2 * u + e, D.g[e]);
      D.xs[e] = L.xs[slot(2 * u + e, L.nb4)];
    }
    D.xsum = L.xsum32[u];
  }
  static __device__ __forceinline__ float dot(const Raw &r, int, const Dig &D) {
    const uint32_t m4 = 0x0f0f0f0fu;
    int qa[4], qb[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      qa[k] = (int)(r.q[k] & m4);
      qb[k] = (int)((r.q[k] >> 4) & m4);
      if constexpr (kQ5) {
        qa[k] |= (int)spread4(r.qh >> (4 * k));
        qb[k] |= (int)spread4(r.qh >> (16 + 4 * k));
      }
    }
    const int I0 = block_dot(qa[0], qa[1], qa[2], qa[3], D.g[0]);
    const int I1 = block_dot(qb[0], qb[1], qb[2], qb[3], D.g[1]);
    const float d = f16_bits_to_f32((uint16_t)(r.dm & 0xffff));
    const float m = f16_bits_to_f32((uint16_t)(r.dm >> 16));
    return d * ((float)I0 * D.xs[0] + (float)I1 * D.xs[1]) + m * D.xsum;
  }
};
template <> struct Traits<LLRS_Q4_1> : TraitsQx1<LLRS_Q4_1> {};
template <> struct Traits<LLRS_Q5_1> : TraitsQx1<LLRS_Q5_1> {};

// Q5_K: as Q4_K with a plane of high bits: qh byte l holds bit g of weight l
// of group g.  Unit u = block u/4, pair p = u%4: the pair's 32 nibble bytes
// and all 32 qh bytes (both groups' bits).
template <> struct Traits<LLRS_Q5_K> {
  static constexpr int kColsPerUnit = 64;
  struct Raw { uint4 hdr, q0, q1, h0, h1; };
  struct Dig { uint4 g[4][2]; float xs[4]; float xsum[2]; };
  static __device__ __forceinline__ void load(const uint8_t *row, int u, Raw &r) {
    const uint8_t *blk = row + (size_t)(u >> 2) * 176;
    const int p = u & 3;
    r.hdr = *reinterpret_cast<const uint4 *>(blk);
    r.h0 = *reinterpret_cast<const uint4 *>(blk + 16);
    r.h1 = *reinterpret_cast<const uint4 *>(blk + 32);
    r.q0 = *reinterpret_cast<const uint4 *>(blk + 48 + p * 32);
    r.q1 = *reinterpret_cast<const uint4 *>(blk + 64 + p * 32);
  }
  static __device__ __forceinline__ void digits(const Lds &L, int u, Dig &D) {
    Traits<LLRS_Q4_K>::Dig d4;
    Traits<LLRS_Q4_K>::digits(L, u, d4);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      D.g[j][0] = d4.g[j][0];
      D.g[j][1] = d4.g[j][1];
      D.xs[j] = d4.xs[j];
    }
    D.xsum[0] = d4.xsum[0];
    D.xsum[1] = d4.xsum[1];
  }
  static __device__ __forceinline__ float dot(const Raw &r, int u, const Dig &D) {
    const int p = u & 3, ga = 2 * p, gb = 2 * p + 1;
    const float d = f16_bits_to_f32((uint16_t)(r.hdr.x & 0xffff));
    const float dmin = f16_bits_to_f32((uint16_t)(r.hdr.x >> 16));
    uint32_t sc, mn;
    k4_scales(r.hdr, p, sc, mn);
    const uint32_t m4 = 0x0f0f0f0fu, b1 = 0x01010101u;
    auto lo = [&](uint32_t q, uint32_t h) { return (int)((q & m4) | (((h >> ga) & b1) << 4)); };
    auto hi = [&](uint32_t q, uint32_t h) { return (int)(((q >> 4) & m4) | (((h >> gb) & b1) << 4)); };
    const int a0 = block_dot(lo(r.q0.x, r.h0.x), lo(r.q0.y, r.h0.y), lo(r.q0.z, r.h0.z), lo(r.q0.w, r.h0.w), D.g[0]);
    const int a1 = block_dot(lo(r.q1.x, r.h1.x), lo(r.q1.y, r.h1.y), lo(r.q1.z, r.h1.z), lo(r.q1.w, r.h1.w), D.g[1]);
    const int a2 = block_dot(hi(r.q0.x, r.h0.x), hi(r.q0.y, r.h0.y), hi(r.q0.z, r.h0.z), hi(r.q0.w, r.h0.w), D.g[2]);
    const int a3 = block_dot(hi(r.q1.x, r.h1.x), hi(r.q1.y, r.h1.y), hi(r.q1.z, r.h1.z), hi(r.q1.w, r.h1.w), D.g[3]);
    const float s0 = (float)a0 * D.xs[0] + (float)a1 * D.xs[1];
    const float s1 = (float)a2 * D.xs[2] + (float)a3 * D.xs[3];
    const float t = (float)(sc & 0xff) * s0 + (float)(sc >> 8) * s1;
    const float m = (float)(mn & 0xff) * D.xsum[0] + (float)(mn >> 8) * D.xsum[1];
    return d * t - dmin * m;
  }
};

__device__ __forceinline__ float wave_sum(float v) { return wave_total(v); }

// The flush's lane exchange: lane_partner's DPP moves and permlane swaps,
// or, with LDSX, ds_bpermute to the same partner lane (same bits either
// way).  ds_bpermute goes through the LDS unit and waits on its round trip,
// but leaves the VALU free: a GEMV whose waves stream many steps (the LM
// head: ~37 four-row steps per wave) keeps its VALU busy with the next
// step's dot products meanwhile, where one or two steps per wave wait on
// the exchange's latency.
template <bool LDSX>
__device__ __forceinline__ float flush_partner(float v, int b) {
  if constexpr (LDSX)
    return __shfl_xor(v, b == 4 ? 7 : b == 8 ? 15 : b);
  else
    return lane_partner(v, b);
}

// Sum of each of four per-lane values over the wave: returns the total of
// row ((lane >> 5) << 1 | (lane >> 4) & 1) in lanes 0, 16, 32, 48.
template <bool LDSX = false>
__device__ __forceinline__ float wave_sum4(const float (&v)[4], int lane) {
  bool hi = lane & 32;
  float s0 = hi ? v[0] : v[2], s1 = hi ? v[1] : v[3];
  float k0 = hi ? v[2] : v[0], k1 = hi ? v[3] : v[1];
  k0 += flush_partner<LDSX>(s0, 32);
  k1 += flush_partner<LDSX>(s1, 32);
  bool hb = lane & 16;
  float k = (hb ? k1 : k0) + flush_partner<LDSX>(hb ? k0 : k1, 16);
#pragma unroll
  for (int b = 8; b > 0; b >>= 1) k += flush_partner<LDSX>(k, b);
  return k;
}

// The two digit planes of one 16-element block, its scale s_b / 128 and the
// integer sum of X = 128 d1 + d2.
__device__ __forceinline__ void digit_block(const float (&v)[16], uint4 &d1, uint4 &d2, float &scale,
                                            int &sum) {
  float m = 0.f;
#pragma unroll
  for (int j = 0; j < 16; j++) m = fmaxf(m, fabsf(v[j]));
  uint32_t p1[4] = {0, 0, 0, 0}, p2[4] = {0, 0, 0, 0};
  sum = 0;
  scale = 0.f;
  if (m > 0.f) {
    float is = 127.0f / m;
    scale = (m / 127.0f) * (1.0f / 128.0f);
#pragma unroll
    for (int j = 0; j < 16; j++) {
      float t = v[j] * is;
      float a1 = rintf(t);
      float a2 = rintf((t - a1) * 128.0f);
      int i1 = (int)a1, i2 = (int)a2;
      sum += i1 * 128 + i2;
      p1[j >> 2] |= (uint32_t)(i1 & 0xff) << (8 * (j & 3));
      p2[j >> 2] |= (uint32_t)(i2 & 0xff) << (8 * (j & 3));
    }
  }
  d1 = make_uint4(p1[0], p1[1], p1[2], p1[3]);
  d2 = make_uint4(p2[0], p2[1], p2[2], p2[3]);
}

// An activation digitised by the kernel that produced it (layout of the LDS
// image below: [2][cols] digit planes, xs[nb], sx[nb], all in slot order),
// copied to LDS; the per-32 sums follow from xs and sx.  With more than two
// 16-byte chunks per thread, a thread issues up to kDigitLoads loads before
// its first LDS store, so the copy takes one memory round trip where a
// load-store loop takes one per chunk (2,960 chunks at 18,944 columns: six
// per thread of 512); at one or two chunks per thread the plain loop
// measured faster.
constexpr int kDigitLoads = 6;
template <bool COH>
__device__ void load_digits(const uint8_t *__restrict__ src, int cols, uint8_t *smem) {
  const int nb = cols >> 4, nb4 = nb >> 2, nt = blockDim.x;
  const int n16 = (2 * cols + 8 * nb) >> 4;  // 16-byte chunks (cols is a multiple of 64)
  if (n16 > 2 * nt) {
    for (int i0 = thread_x(); i0 < n16; i0 += kDigitLoads * nt) {
      uint4 r[kDigitLoads];
#pragma unroll
      for (int k = 0; k < kDigitLoads; k++)
        if (i0 + k * nt < n16) r[k] = ld_u4<COH>(src + 16 * (size_t)(i0 + k * nt));
#pragma unroll
      for (int k = 0; k < kDigitLoads; k++)
        if (i0 + k * nt < n16) reinterpret_cast<uint4 *>(smem)[i0 + k * nt] = r[k];
    }
  } else {
    for (int i = thread_x(); i < n16; i += nt)
      reinterpret_cast<uint4 *>(smem)[i] = ld_u4<COH>(src + 16 * (size_t)i);
  }
  __syncthreads();
  const float *xs = reinterpret_cast<const float *>(smem + 2 * cols);
  const int *sx = reinterpret_cast<const int *>(xs + nb);
  float *xsum32 = reinterpret_cast<float *>(smem + 2 * cols + 8 * nb);
  for (int g = thread_x(); g < (nb >> 1); g += blockDim.x) {
    const int s0 = slot(2 * g, nb4), s1 = slot(2 * g + 1, nb4);
    xsum32[g] = xs[s0] * (float)sx[s0] + xs[s1] * (float)sx[s1];
  }
  __syncthreads();
}

// x (times the RMSNorm gain when given) as digits in LDS; returns
// 1/sqrt(mean(x^2) + eps) with a gain, 1 without.  One pass over x.
// REV: the blocks go to the highest threads first.  The waves without rows
// in a small phase are the highest ones (rows go to waves in order), and they
// have no weight loads in flight: a wave's loads complete in issue order, so
// x loads issued behind prefetched weights would wait for them.
template <bool COH, bool REV = false>
__device__ float digitize(const float *__restrict__ x, const float *__restrict__ gain, float eps,
                          int cols, uint8_t *smem, float *red) {
  const int nt = blockDim.x, tid = thread_x(), nb = cols >> 4, nb4 = nb >> 2;
  const int t0 = REV ? nt - 1 - tid : tid;
  int8_t *dig = reinterpret_cast<int8_t *>(smem);
  float *xs = reinterpret_cast<float *>(smem + 2 * cols);
  int *sx = reinterpret_cast<int *>(xs + nb);
  float *xsum32 = reinterpret_cast<float *>(sx + nb);
  float ss = 0.f;
  // nb is a multiple of 4 and nt of 64, so the lanes b and b^1 of one wave
  // always hold the two x-blocks of a 32-column group (nt - 1 is odd).
  for (int b = t0; b < nb; b += nt) {
    float v[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float4 a = ld_act4<COH>(x + b * 16 + q * 4);
      v[4 * q] = a.x; v[4 * q + 1] = a.y; v[4 * q + 2] = a.z; v[4 * q + 3] = a.w;
    }
    if (gain) {
#pragma unroll
      for (int j = 0; j < 16; j++) ss += v[j] * v[j];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        float4 g = *reinterpret_cast<const float4 *>(gain + b * 16 + q * 4);
        v[4 * q] *= g.x; v[4 * q + 1] *= g.y; v[4 * q + 2] *= g.z; v[4 * q + 3] *= g.w;
      }
    }
    uint4 d1, d2;
    float scale;
    int sum;
    digit_block(v, d1, d2, scale, sum);
    int s = slot(b, nb4);
    *reinterpret_cast<uint4 *>(dig + s * 16) = d1;
    *reinterpret_cast<uint4 *>(dig + cols + s * 16) = d2;
    xs[s] = scale;
    sx[s] = sum;
    float part = scale * (float)sum;
    float pair = lane_partner(part, 1);
    if ((b & 1) == 0) xsum32[b >> 1] = part + pair;
  }
  if (gain) {
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
  }
  __syncthreads();
  float inv = 1.0f;
  if (gain) {
    float t = 0.f;
    for (int i = 0; i < (nt >> 6); i++) t += red[i];
    inv = 1.0f / sqrtf(t / (float)cols + eps);
  }
  return inv;
}

__device__ __forceinline__ uint32_t total_order_key(float f) {
  int32_t b = __float_as_int(f);
  b ^= (int32_t)((uint32_t)(b >> 31) >> 1);
  return (uint32_t)b ^ 0x80000000u;
}

// Sum of each of two per-lane values over the wave: the total of row
// (lane >> 5) ends up in lanes 0 and 32.
template <bool LDSX = false>
__device__ __forceinline__ float wave_sum2(float v0, float v1, int lane) {
  bool hi = lane & 32;
  float k = (hi ? v1 : v0) + flush_partner<LDSX>(hi ? v0 : v1, 32);
#pragma unroll
  for (int b = 16; b > 0; b >>= 1) k += flush_partner<LDSX>(k, b);
  return k;
}

// The same within each 32-lane half of the wave (packed rows): half_sum4
// returns the half's total of v[(lane >> 3) & 3], half_sum2 of
// v[(lane >> 4) & 1].
__device__ __forceinline__ float half_sum4(const float (&v)[4], int lane) {
  bool a = lane & 16;
  float s0 = a ? v[0] : v[2], s1 = a ? v[1] : v[3];
  float k0 = a ? v[2] : v[0], k1 = a ? v[3] : v[1];
  k0 += lane_partner(s0, 16);
  k1 += lane_partner(s1, 16);
  bool b = lane & 8;
  float k = (b ? k1 : k0) + lane_partner(b ? k0 : k1, 8);
#pragma unroll
  for (int o = 4; o > 0; o >>= 1) k += lane_partner(k, o);
  return k;
}
__device__ __forceinline__ float half_sum2(float v0, float v1, int lane) {
  bool a = lane & 16;
  float k = (a ? v1 : v0) + lane_partner(a ? v0 : v1, 16);
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) k += lane_partner(k, o);
  return k;
}

// The balanced split runs while a segment has fewer than this many row groups
// per wave; its LDS holds kBalMaxGroupsPerWave * nw groups x nw waves x R
// (at most 4) partials.
constexpr int kBalMaxGroupsPerWave = 2;
__host__ __device__ constexpr size_t bal_slot_bytes(int nw) {
  return (size_t)kBalMaxGroupsPerWave * nw * nw * 4 * sizeof(float);
}
// The row results' LDS (after the digits), rounded to 16 bytes.
__host__ __device__ constexpr size_t fast_gemv_ybuf_bytes(int rows) { return ((size_t)rows * 4 + 15) & ~(size_t)15; }

// Rows per wave step for a type (kept small enough to double-buffer the raw
// loads in registers); dual gate/up steps hold two rows of each matrix.
template <uint32_t TY, bool DUAL> struct RowsPerStep { static constexpr int value = DUAL ? 2 : 4; };
template <> struct RowsPerStep<LLRS_Q6_K, false> { static constexpr int value = 2; };
template <> struct RowsPerStep<LLRS_Q5_K, false> { static constexpr int value = 2; };

// All dots of this wave's rows of one segment (and of `U` for SwiGLU),
// streamed as (row group, unit-iteration) steps whose raw loads run one step
// ahead of the arithmetic.  Row groups are R rows at row_lo + (first + k *
// stride) * R.  begin() issues the first step's loads (it may run before
// the activation digits exist); run() streams the rest; `emit(row_in_range,
// y, y_up)` runs in one lane per row.
//
// Packed rows: when a row has at most 32 units (e.g. 1,536 columns of Q4_K,
// 24 units), a group is 2R rows and each 32-lane half of the wave takes R of
// them, lane & 31 being the unit: twice the rows per step, at the same
// registers, where otherwise most lanes would idle.
// BAL: the balanced split may run (the standalone GEMV only: in the decode
// step its partial-sum pass cost more than the idle waves it fills, and its
// state costs the persistent kernel registers).
// LDSX: whole-wave row sums exchange through ds_bpermute (flush_partner).
template <uint32_t TY, bool DUAL, bool BAL = false, bool LDSX = false>
struct SegStream {
  using T = Traits<TY>;
  static constexpr int R = RowsPerStep<TY, DUAL>::value;
  static_assert(R <= 4, "bal_slot_bytes holds 4 partials per (group, wave)");
  FastSeg S, U;
  int row_lo, row_hi, first, stride, units, iters, steps, lane, gsz;
  bool packed;
  // Balanced split (single-matrix streams): when the row groups do not
  // divide among the waves and a row takes several unit iterations (long
  // rows over few rows, e.g. a 3,584 x 18,944 GEMV), the wave takes the
  // contiguous range of the (group, iteration) steps starting at group g0,
  // iteration it0, and leaves its per-group partial sums in
  // slots[(group * nw + wave) * R + row]; the caller sums them over the
  // waves, in wave order, after the streaming.
  bool bal;
  int g0, it0, wave, nw;
  float *slots;
  typename T::Raw cur[R], nxt[R], cu[DUAL ? R : 1], nu[DUAL ? R : 1];

  // First row of this wave's g-th row group (of gsz rows: R, or 2R packed).
  __device__ __forceinline__ int group_row(int g) const { return row_lo + (first + g * stride) * gsz; }
  // First row of this lane's part of group g, and its unit at iteration it.
  __device__ __forceinline__ int lane_row(int g) const { return group_row(g) + (packed ? (lane >> 5) * R : 0); }
  __device__ __forceinline__ int lane_unit(int it) const { return packed ? (lane & 31) : it * 64 + lane; }
  // Loads are branch-free (indices past the segment are clamped onto its last
  // row and unit and their products discarded), so the compiler can count the
  // outstanding loads statically and wait only for the current step's.
  __device__ __forceinline__ void load(int g, int it, typename T::Raw (&dst)[R],
                                       typename T::Raw (&dstu)[DUAL ? R : 1]) {
    const int u = min(lane_unit(it), units - 1);
    const int r0 = lane_row(g);
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int r = min(r0 + i, row_hi - 1) - row_lo;
      T::load(S.w + (size_t)r * S.row_bytes, u, dst[i]);
      if constexpr (DUAL) T::load(U.w + (size_t)r * U.row_bytes, u, dstu[i]);
    }
  }
  // first_ / stride_: this wave and the wave count.  slots_: LDS for the
  // balanced split's partial sums (null: whole row groups per wave).
  __device__ __forceinline__ void begin(const FastSeg &S_, const FastSeg &U_, int lo, int hi,
                                        int first_, int stride_, int cols, int lane_,
                                        float *slots_ = nullptr) {
    S = S_;
    U = U_;
    row_lo = lo;
    row_hi = hi;
    first = first_;
    stride = stride_;
    lane = lane_;
    wave = first_;
    nw = stride_;
    slots = slots_;
    units = cols / T::kColsPerUnit;
    packed = units <= 32;
    iters = packed ? 1 : (units + 63) / 64;
    gsz = packed ? 2 * R : R;
    const int ngroups = (row_hi - row_lo + gsz - 1) / gsz;
    bal = BAL && !DUAL && slots_ && iters > 1 && ngroups % nw != 0 && ngroups < kBalMaxGroupsPerWave * nw;
    g0 = it0 = 0;
    if (bal) {
      const int T_ = ngroups * iters, sb = wave * T_ / nw, se = (wave + 1) * T_ / nw;
      steps = se - sb;
      g0 = sb / iters;
      it0 = sb % iters;
      first = 0;
      stride = 1;
    } else {
      int nmine = first < ngroups ? (ngroups - first + stride - 1) / stride : 0;
      steps = __builtin_amdgcn_readfirstlane(nmine) * iters;
    }
    if (steps > 0) load(g0, it0, cur, cu);
  }
  template <class Emit>
  __device__ __forceinline__ void run(const Lds &L, Emit &&emit);
};

template <uint32_t TY, bool DUAL, bool BAL, bool LDSX>
template <class Emit>
__device__ __forceinline__ void SegStream<TY, DUAL, BAL, LDSX>::run(const Lds &L, Emit &&emit) {
  using Raw = typename T::Raw;
  constexpr int RU = DUAL ? R : 1;
  float acc[R], acc2[R];
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = acc2[i] = 0.f;
  int g = g0, it = it0;  // the current step's row group and unit iteration
  // A complete row's sum goes to emit; in the balanced split every partial
  // goes to the wave's slot of its group.
  auto out = [&](int r, float t, float up) {
    if (BAL && !DUAL && bal) {
      const int gg = (r - row_lo) / gsz, i = (r - row_lo) % gsz;
      slots[(gg * nw + wave) * R + i] = t;
    } else {
      emit(r - row_lo, t, up);
    }
  };
  // One step on buffers (c, cu_); when `more` (a compile-time flag, so the
  // loads stay branch-free and their waits exact) the next step's loads go
  // to (n, nu_) first.
  auto step = [&](auto more, Raw (&c)[R], Raw (&cu_)[RU], Raw (&n)[R], Raw (&nu_)[RU]) {
    int gn = g, itn = it + 1;
    if (itn == iters) {
      itn = 0;
      gn = g + 1;
    }
    if constexpr (decltype(more)::value) load(gn, itn, n, nu_);
    const int u0 = lane_unit(it);
    const int u = min(u0, units - 1);
    const int r0 = lane_row(g);
    typename T::Dig D;
    T::digits(L, u, D);
#pragma unroll
    for (int i = 0; i < R; i++) {
      const bool live = u0 < units && r0 + i < row_hi;
      float d = T::dot(c[i], u, D);
      acc[i] += live ? d : 0.f;
      if constexpr (DUAL) {
        float d2 = T::dot(cu_[i], u, D);
        acc2[i] += live ? d2 : 0.f;
      }
    }
    // The row group is complete, or (balanced split) the wave's range ends.
    const bool flush = itn == 0 || (BAL && bal && !decltype(more)::value);
    if (flush && packed) {  // per-half sums
      if constexpr (DUAL) {
        // gate rows 0, 1 in lane groups 0/8, up rows in 16/24 of each half.
        float v[4] = {acc[0], acc[1], acc2[0], acc2[1]};
        float t = half_sum4(v, lane);
        float up = lane_partner(t, 16);
        if ((lane & 23) == 0) {  // lanes 0, 8, 32, 40
          int r = r0 + ((lane >> 3) & 1);
          if (r < row_hi) out(r, t, up);
        }
      } else if constexpr (R == 4) {
        float t = half_sum4(acc, lane);
        if ((lane & 7) == 0) {
          int r = r0 + ((lane >> 3) & 3);
          if (r < row_hi) out(r, t, 0.f);
        }
      } else {
        float t = half_sum2(acc[0], acc[1], lane);
        if ((lane & 15) == 0) {
          int r = r0 + ((lane >> 4) & 1);
          if (r < row_hi) out(r, t, 0.f);
        }
      }
#pragma unroll
      for (int i = 0; i < R; i++) acc[i] = acc2[i] = 0.f;
    } else if (flush) {
      if constexpr (DUAL) {
        // rows 0, 1 of gate and of up: gate sums land in lanes 0/16, up in 32/48.
        float v[4] = {acc[0], acc[1], acc2[0], acc2[1]};
        float t = wave_sum4<LDSX>(v, lane);
        float up = flush_partner<LDSX>(t, 32);
        if ((lane & 47) == 0) {  // lanes 0 and 16
          int r = r0 + ((lane >> 4) & 1);
          if (r < row_hi) out(r, t, up);
        }
      } else if constexpr (R == 4) {
        float t = wave_sum4<LDSX>(acc, lane);
        if ((lane & 15) == 0) {
          int r = r0 + (((lane >> 5) << 1) | ((lane >> 4) & 1));
          if (r < row_hi) out(r, t, 0.f);
        }
      } else {
        float t = wave_sum2<LDSX>(acc[0], acc[1], lane);
        if ((lane & 31) == 0) {
          int r = r0 + (lane >> 5);
          if (r < row_hi) out(r, t, 0.f);
        }
      }
#pragma unroll
      for (int i = 0; i < R; i++) acc[i] = acc2[i] = 0.f;
    }
    g = gn;
    it = itn;
  };
  // Unrolled by two with the buffers swapping roles: no register copies, so
  // the in-flight loads never have to be waited for early.  The last step
  // loads nothing (the phase's closing barrier would wait for such loads).
  using More = std::true_type;
  using Last = std::false_type;
  int s = 0;
  for (; s + 2 < steps; s += 2) {
    step(More{}, cur, cu, nxt, nu);
    step(More{}, nxt, nu, cur, cu);
  }
  if (s + 2 == steps) {
    step(More{}, cur, cu, nxt, nu);
    step(Last{}, nxt, nu, cur, cu);
  } else if (s + 1 == steps) {
    step(Last{}, cur, cu, nxt, nu);
  }
}

// One GEMV launch's work for workgroup `wg` of `nwg`, in two parts:
// prefetch() picks the workgroup's rows and issues its first weight loads
// (they depend on nothing the previous phase writes); finish() stages the
// activation, streams the rest and runs the epilogue.
template <uint32_t TA, uint32_t TB, bool DUAL, bool COH, bool BALANCED = false, bool LDSX = false>
struct GemvPhase {
  int lane, wave, nw, wg, nwg, wrow0, wrow1, s0, base0;
  bool s0_is_ta;
  // The balanced split's partials (set when a.bal and the workgroup's rows
  // lie in one segment).
  float *slots;
  // The balanced split: its own instantiation of the standalone GEMV, for
  // launches that ask for it (its code costs the others registers).
  static constexpr bool BAL = BALANCED && !COH && !DUAL;
  SegStream<TA, DUAL, BAL, LDSX> A;
#ifdef LLRS_STAMPS
  // Timing build only: wall-clock stamps of this workgroup's phase, [1] when
  // the activation is staged, [2] when the weight streaming ends.
  unsigned long long *stamp = nullptr;
#endif

  static __device__ __forceinline__ FastSeg shifted(FastSeg X, int rows) {
    X.w += (size_t)rows * X.row_bytes;
    return X;
  }
  __device__ __forceinline__ void seg_range(const FastGemvArgs &a, int s, int base, int &lo, int &hi) const {
    lo = max(wrow0, base);
    hi = min(wrow1, base + a.seg[s].rows);
  }

  // smem: the launch's dynamic LDS (only its address is taken here).
  __device__ __forceinline__ void prefetch(const FastGemvArgs &a, int wg_, int nwg_, uint8_t *smem) {
    wg = wg_;
    nwg = nwg_;
    lane = thread_x() & 63;
    wave = __builtin_amdgcn_readfirstlane(thread_x() >> 6);
    nw = blockDim.x >> 6;
    fast_gemv_rows(a, wg, nwg, wrow0, wrow1);
    // The workgroup's first segment; when it streams with type TA its first
    // weight loads are issued now.
    s0 = 0;
    base0 = 0;
    while (s0 + 1 < a.nseg && wrow0 >= base0 + a.seg[s0].rows) base0 += a.seg[s0++].rows;
    s0_is_ta = DUAL || TA == TB || s0 + 1 < a.nseg;
    const bool one_seg = wrow1 <= base0 + a.seg[s0].rows;
    slots = BAL && a.bal && one_seg
                ? reinterpret_cast<float *>(smem + fast_gemv_digit_bytes(a.cols) + fast_gemv_ybuf_bytes(wrow1 - wrow0))
                : nullptr;
    if (s0_is_ta) {
      int lo, hi;
      seg_range(a, s0, base0, lo, hi);
      const FastSeg Sw = shifted(a.seg[s0], lo - base0);
      const FastSeg Uw = DUAL ? shifted(a.seg[1], lo - base0) : Sw;
      A.begin(Sw, Uw, lo, max(lo, hi), wave, nw, a.cols, lane, slots);
    }
  }

  // Row results of a balanced stream: the partials of row i's group summed
  // over the waves in order (slots the waves did not write are zero).
  template <class SS, class Emit>
  __device__ __forceinline__ void bal_reduce(Emit &&emit) const {
    for (int i = thread_x(); i < wrow1 - wrow0; i += blockDim.x) {
      const float *sl = slots + (i / SS::R) * nw * SS::R + i % SS::R;
      float t = 0.f;
      for (int w = 0; w < nw; w++) t += sl[w * SS::R];
      emit(i, t, 0.f);
    }
  }

  // The activation (x or its digits) and the residual are read with ordinary
  // loads: every buffer a phase reads was written before any workgroup of the
  // launch first read it, so no cache holds a stale copy.
  __device__ void finish(const FastGemvArgs &a, uint8_t *smem, float *red) {
    // The balanced split's partials start at zero (ordered before the
    // streaming by the staging's workgroup barrier).
    if (BAL && slots)
      for (int i = thread_x(); i < (int)(bal_slot_bytes(nw) / 4); i += blockDim.x) slots[i] = 0.f;
    float inv = 1.0f;
    if (a.dig_in)
      load_digits<false>(a.dig_in, a.cols, smem);
    else
      inv = digitize<false, COH>(a.x, a.norm, a.eps, a.cols, smem, red);
#ifdef LLRS_STAMPS
    if (stamp && thread_x() == 0) stamp[1] = wall_clock64();
#endif
    Lds L;
    L.cols = a.cols;
    L.nb4 = a.cols >> 6;
    L.dig = reinterpret_cast<const int8_t *>(smem);
    L.xs = reinterpret_cast<const float *>(smem + 2 * a.cols);
    L.sx = reinterpret_cast<const int *>(L.xs + (a.cols >> 4));
    L.xsum32 = reinterpret_cast<const float *>(L.sx + (a.cols >> 4));

    // Row results wait in LDS (x inv_rms, SiLU(gate)*up applied) until the
    // streaming is over, so no epilogue memory access stalls the weight loads.
    float *ybuf = reinterpret_cast<float *>(smem + fast_gemv_digit_bytes(a.cols));
    const int r0 = wrow0;
    auto emitter = [&](int lo) {
      return [&, lo](int r, float v, float v2) {
        v *= inv;
        if constexpr (DUAL) v = (v / (1.0f + expf(-v))) * (v2 * inv);
        ybuf[lo - r0 + r] = v;
      };
    };
    // Segments of type TA (all of them unless the last one has type TB); the
    // first one's loads are already in flight.  Dual launches have one segment.
    const int nseg_a = (DUAL || TA == TB) ? a.nseg : a.nseg - 1;
    int base = base0;
    bool bal_a = false, bal_b = false;
    for (int s = s0; s < nseg_a; s++) {
      const FastSeg &S = a.seg[s];
      int lo, hi;
      seg_range(a, s, base, lo, hi);
      if (lo < hi) {
        if (!DUAL && s != s0) {
          const FastSeg Sw = shifted(S, lo - base);
          A.begin(Sw, Sw, lo, hi, wave, nw, a.cols, lane, slots);
        }
        A.run(L, emitter(lo));
        bal_a = A.bal;
      }
      base += S.rows;
    }
    if constexpr (!DUAL && TA != TB) {
      const int s = a.nseg - 1;
      if (s >= s0) {
        const FastSeg &S = a.seg[s];
        int lo, hi;
        seg_range(a, s, base, lo, hi);
        if (lo < hi) {
          const FastSeg Sw = shifted(S, lo - base);
          SegStream<TB, false, BAL, LDSX> B;
          B.begin(Sw, Sw, lo, hi, wave, nw, a.cols, lane, slots);
          B.run(L, emitter(lo));
          bal_b = B.bal;
        }
      }
    }
    __syncthreads();
    // bal_a / bal_b are the same in every wave (they depend on the
    // workgroup's rows only), so the barrier below is uniform.
    if constexpr (BAL) {
      if (bal_a || bal_b) {
        if (bal_a)
          bal_reduce<SegStream<TA, false, true>>(emitter(wrow0));
        else
          bal_reduce<SegStream<TB, false, true>>(emitter(wrow0));
        __syncthreads();
      }
    }
#ifdef LLRS_STAMPS
    if (stamp && thread_x() == 0) stamp[2] = wall_clock64();
#endif

    // Epilogue over the workgroup's rows, coalesced.
    unsigned long long best = 0;
    for (int g = wrow0 + thread_x(); g < wrow1; g += blockDim.x) {
      int s = 0, rs = g;
      while (s + 1 < a.nseg && rs >= a.seg[s].rows) rs -= a.seg[s++].rows;
      const FastSeg &S = a.seg[s];
      const float v = ybuf[g - wrow0];
      switch (a.epi) {
        case kEpiStore: st_act<COH>(S.out + rs, S.bias ? v + S.bias[rs] : v); break;
        case kEpiAdd: st_act<COH>(S.out + rs, (a.res_in ? a.res_in[rs] : S.out[rs]) + v); break;
        case kEpiSwiGlu: st_act<COH>(a.seg[2].out + rs, v); break;
        default: {
          st_act<COH>(S.out + rs, v);
          unsigned long long key = ((unsigned long long)total_order_key(v) << 32) | (uint32_t)rs;
          best = key > best ? key : best;
        }
      }
    }
    if (a.dig_out) {
      // The consumer's activation, digitised once here: this workgroup owns
      // whole 16-row blocks of the output (part == 16).
      __syncthreads();
      const int nb = a.rows >> 4, nb4 = nb >> 2, b0 = wrow0 >> 4;
      for (int t = thread_x(); t < ((wrow1 - wrow0) >> 4); t += blockDim.x) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = ybuf[16 * t + j];
        uint4 d1, d2;
        float scale;
        int sum;
        digit_block(v, d1, d2, scale, sum);
        const int sl = slot(b0 + t, nb4);
        st_u4<COH>(a.dig_out + sl * 16, d1);
        st_u4<COH>(a.dig_out + a.rows + sl * 16, d2);
        st_act<COH>(reinterpret_cast<float *>(a.dig_out + 2 * a.rows) + sl, scale);
        st_act<COH>(reinterpret_cast<float *>(a.dig_out + 2 * a.rows + 4 * nb) + sl,
                    __int_as_float(sum));
      }
    }
    if (a.epi == kEpiLogits) {
      // Max under total_cmp, last index on ties (src/engine.rs:233-241): keys
      // order by (value, index), reduced per block then across blocks.
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        unsigned long long other = __shfl_xor(best, o, 64);
        best = other > best ? other : best;
      }
      __shared__ unsigned long long wbest[16];
      if (lane == 0) wbest[wave] = best;
      __syncthreads();
      if (thread_x() == 0) {
        for (int i = 1; i < nw; i++) best = wbest[i] > best ? wbest[i] : best;
        atomicMax(a.amax_key, best);
        __threadfence();
        unsigned done = atomicAdd(a.done, 1u);
        if (done == (unsigned)nwg - 1) {  // last block: publish the token, advance the position
          __threadfence();
          unsigned long long k = atomicMax(a.amax_key, 0ull);
          uint32_t tok = (uint32_t)(k & 0xffffffffu);
          int p = *a.pos + 1;
          if (p > a.max_pos) p = a.max_pos;  // never index past the context
          *a.pos = p;
          a.tok_by_pos[p] = tok;
          *a.next_token = tok;
          *a.amax_key = 0ull;  // ready for the next step
          *a.done = 0u;
        }
      }
    }
  }
};

}  // namespace

}  // namespace llrs
