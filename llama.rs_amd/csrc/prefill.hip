// Multi-token prefill kernels: the prompt goes through each layer as a
// T-row batch (CausalModel::prefill, src/architecture.rs:60-77, computed the
// way Qwen2Model::forward_impl, src/model.rs:135-271, computes one token).
//
// The weight matrices run as MFMA dequant-GEMMs: a workgroup owns a 64- or
// 128-token x 128-row output tile (of one K range when K is split).  It
// dequantizes its 128 weight rows 64 columns at a time from the native GGUF
// blocks (value_at, src/quant.rs:349-456) into LDS, stages the matching
// activation tile, and accumulates v_mfma_f32_16x16x32_f16 products in f32.
// Eight waves share a tile (prefill_gemm8_kernel; the four-wave form is kept
// for comparison): four stage the weights, four the activations, and each
// multiplies BM/2 tokens x 32 rows.  The raw
// weight blocks and activations of the next 64 columns are loaded into
// registers before the current ones are multiplied, so the loads' latency
// hides behind the MFMAs.  Causal attention runs on f32 MFMA
// (attention_tile_kernel).
//
// Precision: f32 operands are carried as f16 pairs, v = hi + lo with hi =
// f16(v) and lo = f16(v - hi) (22 significant bits), and each product is
// hi*hi + hi*lo + lo*hi (the lo*lo term is below f32 rounding of the sum), so
// the GEMM is close to an f32 GEMM rather than an f16 one.  Q4_K weights take
// prefill_gemm_k4_kernel instead: their integer codes are exact f16 values,
// so one weight plane and two MFMAs per product suffice.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "common.h"
#include "wave_dev.h"
#include "prefill.h"
#include "quant_dev.h"

namespace llrs {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BN = 128, KC = 64, LS = KC + 8;
// Weight-row tiles from which 128-token tiles are used (at 256+ tokens);
// split K makes up the workgroups the larger tiles leave out.
constexpr int kTile128Rows = 16;  // weight rows per tile; LS: LDS row stride in halves

// The 32 values of `row` at columns [k0, k0 + 32) (k0 a multiple of 32), as
// value_at computes them, in two stages: load() issues the loads of the raw
// block bytes, decode() turns them into values once they have arrived.
template <uint32_t TY> struct Deq {
  struct Raw { const uint8_t *row; uint32_t ty; };
  static __device__ __forceinline__ void load(const uint8_t *row, uint32_t ty, int, Raw &r) {
    r.row = row;
    r.ty = ty;
  }
  static __device__ __forceinline__ void decode(const Raw &r, int k0, float (&v)[32]) {
#pragma unroll
    for (int j = 0; j < 32; j++) v[j] = value_dev(r.row, r.ty, (uint32_t)(k0 + j));
  }
};

// Byte i of the little-endian words w.
__device__ __forceinline__ int byte_of(const uint32_t *w, int i) { return (int)((w[i >> 2] >> (8 * (i & 3))) & 0xff); }

template <> struct Deq<LLRS_Q4_K> {
  struct Raw { uint4 hdr, q0, q1; };  // d, dmin, 12 scale bytes; the sub-block's 32 quant bytes
  static __device__ __forceinline__ void load(const uint8_t *row, uint32_t, int k0, Raw &r) {
    const uint8_t *b = row + (size_t)(k0 >> 8) * 144;
    const int g = (k0 & 255) >> 5;
    r.hdr = *reinterpret_cast<const uint4 *>(b);
    r.q0 = *reinterpret_cast<const uint4 *>(b + 16 + (g >> 1) * 32);
    r.q1 = *reinterpret_cast<const uint4 *>(b + 32 + (g >> 1) * 32);
  }
  static __device__ __forceinline__ void decode(const Raw &r, int k0, float (&v)[32]) {
#pragma clang fp contract(off)
    const int g = (k0 & 255) >> 5;
    const uint32_t s[3] = {r.hdr.y, r.hdr.z, r.hdr.w};
    int sc, mn;  // scale_min_k4 (src/quant.rs:338-347) on the scale bytes in registers
    if (g < 4) {
      sc = byte_of(s, g) & 63;
      mn = byte_of(s, g + 4) & 63;
    } else {
      sc = (byte_of(s, g + 4) & 0x0f) | ((byte_of(s, g - 4) >> 6) << 4);
      mn = (byte_of(s, g + 4) >> 4) | ((byte_of(s, g) >> 6) << 4);
    }
    const float ds = f16_bits_to_f32((uint16_t)(r.hdr.x & 0xffff)) * (float)sc;
    const float dm = f16_bits_to_f32((uint16_t)(r.hdr.x >> 16)) * (float)mn;
    const uint32_t w[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const int shift = (g & 1) * 4;
#pragma unroll
    for (int j = 0; j < 32; j++) {
      const int q = (int)((w[j >> 2] >> (8 * (j & 3) + shift)) & 15);
      v[j] = ds * (float)q - dm;
    }
  }
};

template <> struct Deq<LLRS_Q6_K> {
  struct Raw { uint32_t ql[9], qh[9], shl, shh; uint16_t s2, d; };
  static __device__ __forceinline__ void load(const uint8_t *row, uint32_t, int k0, Raw &r) {
    const uint8_t *b = row + (size_t)(k0 >> 8) * 210;
    const int j0 = k0 & 255, half = j0 >> 7, quarter = (j0 >> 5) & 3;
    load9(b + half * 64 + (quarter & 1) * 32, r.ql, r.shl);
    load9(b + 128 + half * 32, r.qh, r.shh);
    r.s2 = ld_u16(b + 192 + half * 8 + quarter * 2);
    r.d = ld_u16(b + 208);
  }
  static __device__ __forceinline__ void decode(const Raw &r, int k0, float (&v)[32]) {
#pragma clang fp contract(off)
    const int quarter = (k0 >> 5) & 3;
    const float d = f16_bits_to_f32(r.d);
    const float sc0 = d * (float)(int8_t)(r.s2 & 0xff), sc1 = d * (float)(int8_t)(r.s2 >> 8);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t l = realign(r.ql, k, r.shl), h = realign(r.qh, k, r.shh);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int lb = (int)((l >> (8 * e)) & 0xff);
        const int lo = quarter < 2 ? (lb & 15) : (lb >> 4);
        const int hi = (int)((h >> (8 * e + 2 * quarter)) & 3);
        const int j = 4 * k + e;
        v[j] = (j < 16 ? sc0 : sc1) * (float)((lo | (hi << 4)) - 32);
      }
    }
  }
};

template <> struct Deq<LLRS_Q8_0> {
  struct Raw { uint32_t q[9], sh; uint16_t d; };
  static __device__ __forceinline__ void load(const uint8_t *row, uint32_t, int k0, Raw &r) {
    const uint8_t *b = row + (size_t)(k0 >> 5) * 34;
    load9(b + 2, r.q, r.sh);
    r.d = ld_u16(b);
  }
  static __device__ __forceinline__ void decode(const Raw &r, int, float (&v)[32]) {
    const float d = f16_bits_to_f32(r.d);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const uint32_t w = realign(r.q, k, r.sh);
#pragma unroll
      for (int e = 0; e < 4; e++) v[4 * k + e] = d * (float)(int8_t)((w >> (8 * e)) & 0xff);
    }
  }
};

template <> struct Deq<LLRS_Q5_0> {
  struct Raw { uint32_t r[9], sh; uint16_t d; };  // qh (4 bytes) then 16 bytes of nibbles
  static __device__ __forceinline__ void load(const uint8_t *row, uint32_t, int k0, Raw &r) {
    const uint8_t *b = row + (size_t)(k0 >> 5) * 22;
    load9(b + 2, r.r, r.sh);
    r.d = ld_u16(b);
  }
  static __device__ __forceinline__ void decode(const Raw &r, int, float (&v)[32]) {
#pragma clang fp contract(off)
    const uint32_t qh = realign(r.r, 0, r.sh);
    const float d = f16_bits_to_f32(r.d);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t w = realign(r.r, k + 1, r.sh);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int j = 4 * k + e;
        const int lo = (int)((w >> (8 * e)) & 15), hi = (int)((w >> (8 * e + 4)) & 15);
        v[j] = d * ((float)(lo | (int)(((qh >> j) & 1) << 4)) - 16.0f);
        v[j + 16] = d * ((float)(hi | (int)(((qh >> (j + 16)) & 1) << 4)) - 16.0f);
      }
    }
  }
};

__device__ __forceinline__ void split_f16(float v, f16 &hi, f16 &lo) {
  hi = (f16)v;
  lo = (f16)(v - (float)hi);
}

// A wave's MI x NJ accumulator blocks of 16 x 16 (tokens tb + 16 i + ..., rows
// nb + 16 j + ...; D layout: lane holds row (lane & 15) and tokens
// 4 * (lane >> 4) + e) into C: C (=|+=) acc (+ bias), or with K split the
// split's partial tile into `part` (split_reduce_kernel adds them up).
template <int MI, int NJ>
__device__ __forceinline__ void store_tile(const PrefillGemmArgs &g, const f32x4 (&acc)[MI][NJ], int nb, int tb,
                                           int lane) {
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int n = nb + 16 * j + (lane & 15);
      if (n >= g.n) continue;
      const float bias = (!g.accumulate && g.bias) ? g.bias[n] : 0.f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int t = tb + 16 * i + 4 * (lane >> 4) + e;
        if (t >= g.t) continue;
        if (g.ksplit > 1) {
          g.part[((size_t)blockIdx.z * g.t + t) * g.n + n] = acc[i][j][e];
        } else {
          float *c = g.c + (size_t)t * g.ldc + n;
          *c = g.accumulate ? *c + acc[i][j][e] : acc[i][j][e] + bias;
        }
      }
    }
}

// BM tokens x BN weight rows per workgroup (BM = 64 or 128).
template <uint32_t TY, int BM>
__global__ __launch_bounds__(256) void prefill_gemm_kernel(PrefillGemmArgs g) {
  constexpr int MI = BM / 32;    // 16-token MFMA blocks per wave
  constexpr int APT = BM / 4;    // activation halves per thread and plane
  constexpr int TPR = 64 / APT;  // threads per activation row
  extern __shared__ __align__(16) f16 lds[];
  f16 *As = lds, *Al = As + BM * LS, *Ws = Al + BM * LS, *Wl = Ws + BN * LS;
  const int n0 = blockIdx.x * BN, t0 = blockIdx.y * BM;
  // This workgroup's K range (split K: whole KC chunks per split).
  const int per = ((g.k + KC - 1) / KC + g.ksplit - 1) / g.ksplit * KC;
  const int kb = blockIdx.z * per, ke = min(g.k, kb + per);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // the wave's (BM/2)-token x 64-row quarter
  f32x4 acc[MI][4];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Staging roles: activations BM rows x TPR runs of APT halves, weights 128
  // rows x 2 runs of 32 values.  Rows past the tile's end read row 0 and are
  // zeroed on their way into LDS.
  const int ar = tid / TPR, ac = (tid % TPR) * APT;
  const int wr = tid >> 1, wc = (tid & 1) * 32;
  const bool a_ok = t0 + ar < g.t, w_ok = n0 + wr < g.n;
  const size_t aoff = (size_t)(a_ok ? t0 + ar : 0) * g.lda + ac;
  const uint8_t *wrow = g.w + (size_t)(w_ok ? n0 + wr : 0) * g.row_bytes;
  half8 ah[APT / 8], alo[APT / 8];
  typename Deq<TY>::Raw raw;
  auto load_chunk = [&](int k0) {
    const int kk = min(k0 + ac, ke - APT);  // columns past the range: a valid read, zeroed below
#pragma unroll
    for (int h = 0; h < APT / 8; h++) {
      ah[h] = *reinterpret_cast<const half8 *>(g.a + aoff - ac + kk + 8 * h);
      alo[h] = *reinterpret_cast<const half8 *>(g.a_lo + aoff - ac + kk + 8 * h);
    }
    Deq<TY>::load(wrow, g.type, min(k0 + wc, ke - 32), raw);
  };
  // A split whose range is empty (rounding of the per-split chunk count)
  // loads nothing and writes zero partials.
  if (kb < ke) load_chunk(kb);
  for (int k0 = kb; k0 < ke; k0 += KC) {
    const int kc = min(KC, ke - k0);  // 32 or 64
    __syncthreads();  // the previous chunk's MFMAs have read LDS
    {
      const bool in = a_ok && ac < kc;
      const half8 z = half8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int h = 0; h < APT / 8; h++) {
        *reinterpret_cast<half8 *>(As + ar * LS + ac + 8 * h) = in ? ah[h] : z;
        *reinterpret_cast<half8 *>(Al + ar * LS + ac + 8 * h) = in ? alo[h] : z;
      }
    }
    {
      float v[32];
      Deq<TY>::decode(raw, min(k0 + wc, ke - 32), v);  // the columns load_chunk read
      const bool in = w_ok && wc < kc;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        half8 h, l;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          f16 a, b;
          split_f16(in ? v[8 * q + e] : 0.f, a, b);
          h[e] = a;
          l[e] = b;
        }
        *reinterpret_cast<half8 *>(Ws + wr * LS + wc + 8 * q) = h;
        *reinterpret_cast<half8 *>(Wl + wr * LS + wc + 8 * q) = l;
      }
    }
    __syncthreads();
    if (k0 + KC < ke) load_chunk(k0 + KC);  // in flight during the MFMAs below
    for (int ks = 0; ks < kc; ks += 32) {
      half8 af[MI], al[MI], bf[4], bl[4];
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const int o = (wm * (BM / 2) + 16 * i + (lane & 15)) * LS + ks + 8 * (lane >> 4);
        af[i] = *reinterpret_cast<const half8 *>(As + o);
        al[i] = *reinterpret_cast<const half8 *>(Al + o);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int o = (wn * 64 + 16 * j + (lane & 15)) * LS + ks + 8 * (lane >> 4);
        bf[j] = *reinterpret_cast<const half8 *>(Ws + o);
        bl[j] = *reinterpret_cast<const half8 *>(Wl + o);
      }
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bf[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bl[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }
  }
  store_tile<MI, 4>(g, acc, n0 + wn * 64, t0 + wm * (BM / 2), lane);
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// One staging thread's 32 Q6_K weights of a row (columns col .. col + 31, within
// one 32-column quarter of a 128-column half) on their integer codes.  A Q6_K
// weight is d * sc * (q - 32) (value_at, src/quant.rs:349-456): q a 6-bit
// code, sc an int8 per 16 columns, d per 256-column block.  sc * (q - 32) is
// an integer of magnitude at most 4,096: hi = its f16 rounding and lo = the
// remainder (-1, 0 or 1, exact), from packed f16 arithmetic on 1024 + q (the
// bit pattern 0x6400 | q): q - 32 is exact, hi one product, lo one fma.  d is
// applied to the accumulators per 256-column block (`first`: this thread
// keeps the row's unit u and publishes the block's rescale d_prev / d and the
// unit; a block with d = 0 is staged as zeros and keeps the unit), as in
// prefill_gemm_k4_kernel.  The three MFMAs per product stay (lo*x_hi is needed
// where |sc * (q - 32)| > 2,048); the staging drops from ~14 VALU operations
// per weight to ~3 per two.
__device__ __forceinline__ void stage_q6k_codes(const Deq<LLRS_Q6_K>::Raw &r, int col, bool w_ok, bool first,
                                                float &u, float *ratio, float *unit, f16 *ws, f16 *wl) {
#pragma clang fp contract(off)
  const float d = f16_bits_to_f32(r.d);
  const bool live = d != 0.f;  // NaN d is live and makes the row NaN, as in f32
  if (first) {
    *ratio = live ? u / d : 1.f;
    if (live) u = d;
    *unit = u;
  }
  const int quarter = (col >> 5) & 3;
  const bool use = w_ok && live;
  const f16 s0 = (f16)(float)(use ? (int)(int8_t)(r.s2 & 0xff) : 0);
  const f16 s1 = (f16)(float)(use ? (int)(int8_t)(r.s2 >> 8) : 0);
  const half2v off = {(f16)-1056.f, (f16)-1056.f};
#pragma unroll
  for (int k2 = 0; k2 < 4; k2++) {  // columns 8 k2 .. 8 k2 + 7
    half8 hv, lv;
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int k = 2 * k2 + p;  // columns 4k .. 4k + 3
      const uint32_t l = realign(r.ql, k, r.shl), h = realign(r.qh, k, r.shh);
      const uint32_t lo4 = (quarter < 2 ? l : l >> 4) & 0x0f0f0f0fu;
      const uint32_t hi2 = (h >> (2 * quarter)) & 0x03030303u;
      const uint32_t q = lo4 | (hi2 << 4);  // four 6-bit codes, a byte each
      const uint32_t pa = (q & 0xffu) | ((q << 8) & 0xff0000u) | 0x64006400u;
      const uint32_t pb = ((q >> 16) & 0xffu) | ((q >> 8) & 0xff0000u) | 0x64006400u;
      const f16 sc = k < 4 ? s0 : s1;
      const half2v scv = {sc, sc};
      const half2v xa = __builtin_bit_cast(half2v, pa) + off, xb = __builtin_bit_cast(half2v, pb) + off;
      const half2v ha = xa * scv, hb = xb * scv;
      const half2v la = __builtin_elementwise_fma(xa, scv, -ha), lb = __builtin_elementwise_fma(xb, scv, -hb);
      hv[4 * p] = ha[0];
      hv[4 * p + 1] = ha[1];
      hv[4 * p + 2] = hb[0];
      hv[4 * p + 3] = hb[1];
      lv[4 * p] = la[0];
      lv[4 * p + 1] = la[1];
      lv[4 * p + 2] = lb[0];
      lv[4 * p + 3] = lb[1];
    }
    *reinterpret_cast<half8 *>(ws + 8 * k2) = hv;
    *reinterpret_cast<half8 *>(wl + 8 * k2) = lv;
  }
}

// The same tile, products and LDS layout with eight waves, so that two
// workgroups per CU put four waves on each SIMD (the four-wave kernel's two
// leave the matrix cores waiting on the staging chain's latency).  Waves 0-3
// dequantize the weight tile (32 values per thread, as above) while waves
// 4-7 stage the activation tile, so each SIMD holds one wave of each kind;
// all eight run MFMAs, each on BM/2 tokens x 32 rows of the tile.  A thread
// keeps only its role's next-chunk registers (a union), which holds a wave
// to 128 registers.  Each output is the same sequence of MFMAs as in the
// four-wave kernel.  Measured 4-5% faster per product (7B shape, 512
// tokens); LLRS_PREFILL_GEMM=4 selects the four-wave kernel.
template <uint32_t TY, int BM, bool CODES>
__global__ __launch_bounds__(512) void prefill_gemm8_kernel(PrefillGemmArgs g) {
  static_assert(!CODES || TY == LLRS_Q6_K, "integer-code staging is written for Q6_K");
  constexpr int MI = BM / 32;    // 16-token MFMA blocks per wave (BM/2 tokens)
  constexpr int NJ = 2;          // 16-row MFMA blocks per wave (32 rows)
  constexpr int APT = BM / 4;    // activation halves per staging thread and plane
  constexpr int TPR = 64 / APT;  // staging threads per activation row
  extern __shared__ __align__(16) f16 lds[];
  f16 *As = lds, *Al = As + BM * LS, *Ws = Al + BM * LS, *Wl = Ws + BN * LS;
  // CODES: per weight row, the rescale of the current 256-column block and the current unit.
  float *ratio = reinterpret_cast<float *>(Wl + BN * LS), *unit = ratio + BN;
  const int n0 = blockIdx.x * BN, t0 = blockIdx.y * BM;
  const int per = CODES ? ((g.k >> 8) + g.ksplit - 1) / g.ksplit * 256
                        : ((g.k + KC - 1) / KC + g.ksplit - 1) / g.ksplit * KC;
  const int kb = blockIdx.z * per, ke = min(g.k, kb + per);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;  // BM/2 tokens x 32 rows
  const bool wstage = wave < 4;             // weight staging (else activation staging)
  const int st = tid & 255;                 // thread index within the staging group
  f32x4 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ar = st / TPR, ac = (st % TPR) * APT;
  const int wr = st >> 1, wc = (st & 1) * 32;
  const bool a_ok = t0 + ar < g.t, w_ok = n0 + wr < g.n;
  const size_t aoff = (size_t)(a_ok ? t0 + ar : 0) * g.lda + ac;
  const uint8_t *wrow = g.w + (size_t)(w_ok ? n0 + wr : 0) * g.row_bytes;
  union Pre {
    struct { half8 ah[APT / 8], al[APT / 8]; } a;
    typename Deq<TY>::Raw raw;
  } pre;
  auto load_chunk = [&](int k0) {
    if (wstage) {
      Deq<TY>::load(wrow, g.type, min(k0 + wc, ke - 32), pre.raw);
    } else {
      const int kk = min(k0 + ac, ke - APT);  // columns past the range: a valid read, zeroed below
#pragma unroll
      for (int h = 0; h < APT / 8; h++) {
        pre.a.ah[h] = *reinterpret_cast<const half8 *>(g.a + aoff - ac + kk + 8 * h);
        pre.a.al[h] = *reinterpret_cast<const half8 *>(g.a_lo + aoff - ac + kk + 8 * h);
      }
    }
  };
  float u = 1.f;  // CODES: a row's current unit (kept by its wc == 0 staging thread)
  if (kb < ke) load_chunk(kb);
  for (int k0 = kb; k0 < ke; k0 += KC) {
    const int kc = min(KC, ke - k0);  // 32 or 64 (64 with CODES)
    __syncthreads();  // the previous chunk's MFMAs have read LDS
    bool staged = false;
    if constexpr (CODES) {
      if (wstage) {
        stage_q6k_codes(pre.raw, k0 + wc, w_ok, (k0 & 255) == 0 && wc == 0, u, ratio + wr, unit + wr,
                        Ws + wr * LS + wc, Wl + wr * LS + wc);
        staged = true;
      }
    }
    if (staged) {
    } else if (wstage) {
      float v[32];
      Deq<TY>::decode(pre.raw, min(k0 + wc, ke - 32), v);  // the columns load_chunk read
      const bool in = w_ok && wc < kc;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        half8 h, l;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          f16 a, b;
          split_f16(in ? v[8 * q + e] : 0.f, a, b);
          h[e] = a;
          l[e] = b;
        }
        *reinterpret_cast<half8 *>(Ws + wr * LS + wc + 8 * q) = h;
        *reinterpret_cast<half8 *>(Wl + wr * LS + wc + 8 * q) = l;
      }
    } else {
      const bool in = a_ok && ac < kc;
      const half8 z = half8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int h = 0; h < APT / 8; h++) {
        *reinterpret_cast<half8 *>(As + ar * LS + ac + 8 * h) = in ? pre.a.ah[h] : z;
        *reinterpret_cast<half8 *>(Al + ar * LS + ac + 8 * h) = in ? pre.a.al[h] : z;
      }
    }
    __syncthreads();
    if (k0 + KC < ke) load_chunk(k0 + KC);  // in flight during the MFMAs below
    if (CODES && (k0 & 255) == 0) {
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const float r = ratio[wn * 32 + 16 * j + (lane & 15)];
#pragma unroll
        for (int i = 0; i < MI; i++) acc[i][j] *= r;
      }
    }
    for (int ks = 0; ks < kc; ks += 32) {
      half8 af[MI], al[MI], bf[NJ], bl[NJ];
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const int o = (wm * (BM / 2) + 16 * i + (lane & 15)) * LS + ks + 8 * (lane >> 4);
        af[i] = *reinterpret_cast<const half8 *>(As + o);
        al[i] = *reinterpret_cast<const half8 *>(Al + o);
      }
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const int o = (wn * 32 + 16 * j + (lane & 15)) * LS + ks + 8 * (lane >> 4);
        bf[j] = *reinterpret_cast<const half8 *>(Ws + o);
        bl[j] = *reinterpret_cast<const half8 *>(Wl + o);
      }
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bf[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bl[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }
  }
  if (CODES && kb < ke) {
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const float d = unit[wn * 32 + 16 * j + (lane & 15)];
#pragma unroll
      for (int i = 0; i < MI; i++) acc[i][j] *= d;
    }
  }
  store_tile<MI, NJ>(g, acc, n0 + wn * 32, t0 + wm * (BM / 2), lane);
}


// The epilogue of a dual gate/up tile without split K: the waves of the up
// row group (wn = 1) hand their accumulators to the waves of the gate row group
// with the same tokens through LDS (the same lane and register layout), and
// those write silu(g) * u as f16 pairs -- the arithmetic of swiglu_f16_kernel,
// so the values are the same as the separate products followed by it -- and,
// with xso, the 32-column sums of hi + lo (two 16-row blocks of a lane's
// column group, reduced over the 16 lanes of each token quad).
template <int MI, int NJ>
__device__ __forceinline__ void swiglu_tile(const PrefillGemmArgs &g, const f32x4 (&acc)[MI][NJ], float *xch,
                                            int wm, int wn, int tb, int lane) {
#pragma clang fp contract(off)
  __syncthreads();  // every wave is done with the LDS tiles
  float *slot = xch + (size_t)wm * (MI * NJ * 4 * 64);
  if (wn == 1) {
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
      for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) slot[((i * NJ + j) * 4 + e) * 64 + lane] = acc[i][j][e];
  }
  __syncthreads();
  if (wn != 0) return;
  const int f0 = blockIdx.x * 64;  // the tile's first gate/up row
#pragma unroll
  for (int i = 0; i < MI; i++) {
    float xsum[NJ / 2][4];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int f = f0 + 16 * j + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int t = tb + 16 * i + 4 * (lane >> 4) + e;
        const float x = acc[i][j][e], u = slot[((i * NJ + j) * 4 + e) * 64 + lane];
        f16 hi = 0, lo = 0;
        if (f < g.dual_rows && t < g.t) {
          split_f16((x / (1.0f + expf(-x))) * u, hi, lo);
          g.h[(size_t)t * g.ldh + f] = hi;
          g.hl[(size_t)t * g.ldh + f] = lo;
        }
        const float v = (float)hi + (float)lo;
        if (j % 2 == 0) xsum[j / 2][e] = v;
        else xsum[j / 2][e] += v;
      }
    }
    if (g.xso) {
#pragma unroll
      for (int q = 0; q < NJ / 2; q++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float v = xsum[q][e];
#pragma unroll
          for (int b = 1; b < 16; b <<= 1) v += lane_partner(v, b);
          const int t = tb + 16 * i + 4 * (lane >> 4) + e, f = f0 + 32 * q;
          if ((lane & 15) == 0 && t < g.t && f < g.dual_rows)
            split_f16(v, g.xso[(size_t)t * g.ldxso + (f >> 5)], g.xso_lo[(size_t)t * g.ldxso + (f >> 5)]);
        }
    }
  }
}

// The Q4_K product with the weight codes as exact f16 integers.  A Q4_K
// weight is d * sc * q - dmin * m (value_at, src/quant.rs:349-456): q < 16 per
// column, sc and m < 64 per 32-column sub-block s, d and dmin per 256-column
// super-block b.  sc * q <= 945 is an exact f16, so
//   y = sum_b d_b * sum_{j in b} (sc q)_j x_j  -  sum_s (dmin m)_s * xsum_s
// with xsum_s the sum of the activations over sub-block s.  The first sum is
// an MFMA product of one exact weight plane with the activations' hi and lo
// planes: two MFMAs where an f32 weight (hi + lo) needs three, and half the
// weight staging and LDS traffic.  Its accumulators are kept in units of the
// row's current d: at each super-block they are scaled by d_prev / d_b (a
// super-block with d = 0 contributes nothing and keeps the unit), and by the
// last d at the end.  The second sum is a K/32-long product of -dmin * m (an
// exact f32, as hi + lo) with xsum (hi + lo, xsum_f16_kernel), run after the
// first on the same tile, LDS and accumulators, three MFMAs per step.  The
// layout, roles and tiles are those of prefill_gemm8_kernel; K splits into
// whole super-blocks.  Integer and f16 arithmetic on the codes is exact, so
// the result differs from the f32 weights' only in f32 rounding.
template <int BM, int TG, bool DUAL>
__global__ __launch_bounds__(512) void prefill_gemm_k4_kernel(PrefillGemmArgs g) {
  static_assert(!DUAL || TG == 4, "dual tiles pair the two row groups of waves");
  // TG token groups x 8/TG row groups of waves: a wave multiplies TW tokens x RW rows.
  constexpr int TW = BM / TG, RW = BN * TG / 8, MI = TW / 16, NJ = RW / 16;
  constexpr int APT = BM / 4, TPR = 64 / APT;
  extern __shared__ __align__(16) f16 lds[];
  f16 *As = lds, *Al = As + BM * LS, *Ws = Al + BM * LS, *Wl = Ws + BN * LS;
  // Per weight row of the tile: the rescale of the current super-block and the current unit.
  float *ratio = reinterpret_cast<float *>(Wl + BN * LS), *unit = ratio + BN;
  const int n0 = blockIdx.x * BN, t0 = blockIdx.y * BM;
  const int per = ((g.k >> 8) + g.ksplit - 1) / g.ksplit * 256;
  const int kb = blockIdx.z * per, ke = min(g.k, kb + per);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % TG, wn = wave / TG;
  const bool wstage = wave < 4;
  const int st = tid & 255;
  f32x4 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ar = st / TPR, ac = (st % TPR) * APT;
  const int wr = st >> 1, wc = (st & 1) * 32;
  // A segmented product: this tile's segment (boundaries are tile multiples).
  const int seg = g.nseg > 1 ? (n0 >= g.seg_base[1]) + (g.nseg > 2 && n0 >= g.seg_base[2]) : 0;
  const int sbase = g.nseg > 0 ? g.seg_base[seg] : 0;
  const int srows = g.nseg > 0 ? g.seg_base[seg + 1] - sbase : g.n;
  const uint8_t *wmat = g.nseg > 0 ? g.seg_w[seg] : g.w;
  // DUAL: tile rows 0-63 are gate rows blockIdx.x * 64 + wr, rows 64-127 the same up rows.
  const int wrow_i = DUAL ? blockIdx.x * 64 + (wr & 63) : n0 - sbase + wr;
  const bool a_ok = t0 + ar < g.t, w_ok = wrow_i < (DUAL ? g.dual_rows : srows);
  const int arow = a_ok ? t0 + ar : 0;
  const uint8_t *wrow = (DUAL && wr >= 64 ? g.w2 : wmat) + (size_t)(w_ok ? wrow_i : 0) * g.row_bytes;
  union Pre {
    struct { half8 ah[APT / 8], al[APT / 8]; } a;
    struct { uint4 hdr, q0, q1; } w;  // d, dmin, 12 scale bytes; the sub-block pair's 32 code bytes
    uint4 mh[4];                      // the headers of four super-blocks (second sum)
  } pre;

  // ---- First sum: the exact codes, rescaled per super-block ----
  auto load_codes = [&](int k0) {  // k0: a multiple of 64 with k0 + 64 <= ke
    if (wstage) {
      const uint8_t *b = wrow + (size_t)(k0 >> 8) * 144;
      const int pair = (k0 & 255) >> 6;
      pre.w.hdr = *reinterpret_cast<const uint4 *>(b);
      pre.w.q0 = *reinterpret_cast<const uint4 *>(b + 16 + pair * 32);
      pre.w.q1 = *reinterpret_cast<const uint4 *>(b + 32 + pair * 32);
    } else {
      const size_t o = (size_t)arow * g.lda + k0 + ac;
#pragma unroll
      for (int h = 0; h < APT / 8; h++) {
        pre.a.ah[h] = *reinterpret_cast<const half8 *>(g.a + o + 8 * h);
        pre.a.al[h] = *reinterpret_cast<const half8 *>(g.a_lo + o + 8 * h);
      }
    }
  };
  float u = 1.f;  // a row's current unit (kept by its wc == 0 staging thread)
  if (kb < ke) load_codes(kb);
  for (int k0 = kb; k0 < ke; k0 += KC) {
    __syncthreads();  // the previous chunk's MFMAs have read LDS
    if (wstage) {
      const int sub = ((k0 + wc) & 255) >> 5;  // sub < 4 is uniform: k0 is
      const uint32_t s[3] = {pre.w.hdr.y, pre.w.hdr.z, pre.w.hdr.w};
      const int sc = sub < 4 ? (byte_of(s, sub) & 63)
                             : ((byte_of(s, sub + 4) & 0x0f) | ((byte_of(s, sub - 4) >> 6) << 4));
      const float d = f16_bits_to_f32((uint16_t)(pre.w.hdr.x & 0xffff));
      const bool live = d != 0.f;  // NaN d is live and makes the row NaN, as in f32
      if ((k0 & 255) == 0 && wc == 0) {
        ratio[wr] = live ? u / d : 1.f;
        if (live) u = d;
        unit[wr] = u;
      }
      // (1024 + q) from the f16 bit pattern 0x6400 | q, then (1024 + q) * sc -
      // 1024 * sc = sc * q, exact in one fma.
      const f16 sch = (f16)(float)((w_ok && live) ? sc : 0);
      const half2v f = {sch, sch}, c = {(f16)(-1024.f * (float)sch), (f16)(-1024.f * (float)sch)};
      const uint32_t w[8] = {pre.w.q0.x, pre.w.q0.y, pre.w.q0.z, pre.w.q0.w,
                             pre.w.q1.x, pre.w.q1.y, pre.w.q1.z, pre.w.q1.w};
      const int shift = (sub & 1) * 4;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        half8 h;
#pragma unroll
        for (int p = 0; p < 2; p++) {
          const uint32_t v = (w[2 * q + p] >> shift) & 0x0f0f0f0fu;  // four codes, a byte each
          const uint32_t lo = (v & 0xffu) | ((v << 8) & 0xff0000u) | 0x64006400u;
          const uint32_t hi = ((v >> 16) & 0xffu) | ((v >> 8) & 0xff0000u) | 0x64006400u;
          const half2v a = __builtin_elementwise_fma(__builtin_bit_cast(half2v, lo), f, c);
          const half2v b = __builtin_elementwise_fma(__builtin_bit_cast(half2v, hi), f, c);
          h[4 * p] = a[0];
          h[4 * p + 1] = a[1];
          h[4 * p + 2] = b[0];
          h[4 * p + 3] = b[1];
        }
        *reinterpret_cast<half8 *>(Ws + wr * LS + wc + 8 * q) = h;
      }
    } else {
      const half8 z = half8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int h = 0; h < APT / 8; h++) {
        *reinterpret_cast<half8 *>(As + ar * LS + ac + 8 * h) = a_ok ? pre.a.ah[h] : z;
        *reinterpret_cast<half8 *>(Al + ar * LS + ac + 8 * h) = a_ok ? pre.a.al[h] : z;
      }
    }
    __syncthreads();
    if (k0 + KC < ke) load_codes(k0 + KC);  // in flight during the MFMAs below
    if ((k0 & 255) == 0) {
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const float r = ratio[wn * RW + 16 * j + (lane & 15)];
#pragma unroll
        for (int i = 0; i < MI; i++) acc[i][j] *= r;
      }
    }
#pragma unroll
    for (int ks = 0; ks < KC; ks += 32) {
      half8 af[MI], al[MI], bf[NJ];
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const int o = (wm * TW + 16 * i + (lane & 15)) * LS + ks + 8 * (lane >> 4);
        af[i] = *reinterpret_cast<const half8 *>(As + o);
        al[i] = *reinterpret_cast<const half8 *>(Al + o);
      }
#pragma unroll
      for (int j = 0; j < NJ; j++)
        bf[j] = *reinterpret_cast<const half8 *>(Ws + (wn * RW + 16 * j + (lane & 15)) * LS + ks +
                                                 8 * (lane >> 4));
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bf[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }
  }
  if (kb < ke) {
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const float d = unit[wn * RW + 16 * j + (lane & 15)];
#pragma unroll
      for (int i = 0; i < MI; i++) acc[i][j] *= d;
    }
  }

  // ---- Second sum: - (dmin m)_s * xsum_s over this range's sub-blocks ----
  const int mb = kb >> 5, me = ke >> 5;  // multiples of 8
  auto load_mins = [&](int m0) {
    if (wstage) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int s0 = m0 + wc + 8 * i;
        pre.mh[i] = s0 < me ? *reinterpret_cast<const uint4 *>(wrow + (size_t)(s0 >> 3) * 144)
                            : uint4{0, 0, 0, 0};
      }
    } else {
      // Columns up to m0 + 64 <= K/32 + 56 < ldxs: in the buffer; those past
      // the range are zeroed below.
      const size_t o = (size_t)arow * g.ldxs + m0 + ac;
#pragma unroll
      for (int h = 0; h < APT / 8; h++) {
        pre.a.ah[h] = *reinterpret_cast<const half8 *>(g.xs + o + 8 * h);
        pre.a.al[h] = *reinterpret_cast<const half8 *>(g.xs_lo + o + 8 * h);
      }
    }
  };
  if (mb < me) load_mins(mb);
  for (int m0 = mb; m0 < me; m0 += KC) {
    const int mc = min(KC, me - m0);  // a multiple of 8
    __syncthreads();
    if (wstage) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const bool in = w_ok && m0 + wc + 8 * i < me;
        const float dmin = f16_bits_to_f32((uint16_t)(pre.mh[i].x >> 16));
        const uint32_t s[3] = {pre.mh[i].y, pre.mh[i].z, pre.mh[i].w};
        half8 h, l;
#pragma unroll
        for (int e = 0; e < 8; e++) {  // scale_min_k4 (src/quant.rs:338-347), the m half
          const int m = e < 4 ? (byte_of(s, e + 4) & 63) : ((byte_of(s, e + 4) >> 4) | ((byte_of(s, e) >> 6) << 4));
          f16 a, b;
          split_f16(in ? -(dmin * (float)m) : 0.f, a, b);
          h[e] = a;
          l[e] = b;
        }
        *reinterpret_cast<half8 *>(Ws + wr * LS + wc + 8 * i) = h;
        *reinterpret_cast<half8 *>(Wl + wr * LS + wc + 8 * i) = l;
      }
    } else {
      const half8 z = half8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int h = 0; h < APT / 8; h++) {
        const bool in = a_ok && ac + 8 * h < mc;
        *reinterpret_cast<half8 *>(As + ar * LS + ac + 8 * h) = in ? pre.a.ah[h] : z;
        *reinterpret_cast<half8 *>(Al + ar * LS + ac + 8 * h) = in ? pre.a.al[h] : z;
      }
    }
    __syncthreads();
    if (m0 + KC < me) load_mins(m0 + KC);
    for (int ks = 0; ks < mc; ks += 32) {
      half8 af[MI], al[MI], bf[NJ], bl[NJ];
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const int o = (wm * TW + 16 * i + (lane & 15)) * LS + ks + 8 * (lane >> 4);
        af[i] = *reinterpret_cast<const half8 *>(As + o);
        al[i] = *reinterpret_cast<const half8 *>(Al + o);
      }
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const int o = (wn * RW + 16 * j + (lane & 15)) * LS + ks + 8 * (lane >> 4);
        bf[j] = *reinterpret_cast<const half8 *>(Ws + o);
        bl[j] = *reinterpret_cast<const half8 *>(Wl + o);
      }
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bf[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bl[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    }
  }
  if constexpr (DUAL) {
    if (g.ksplit == 1) {
      swiglu_tile<MI, NJ>(g, acc, reinterpret_cast<float *>(lds), wm, wn, t0 + wm * TW, lane);
      return;
    }
  }
  if (g.nseg > 0 && g.ksplit == 1) {  // the segment's own output
    PrefillGemmArgs gs = g;
    gs.c = g.seg_c[seg];
    gs.ldc = g.seg_ldc[seg];
    gs.bias = g.seg_bias[seg];
    gs.n = srows;
    store_tile<MI, NJ>(gs, acc, n0 - sbase + wn * RW, t0 + wm * TW, lane);
    return;
  }
  store_tile<MI, NJ>(g, acc, n0 + wn * RW, t0 + wm * TW, lane);
}

// xs + xs_lo [t][s] = the sum over j < 32 of a[t][32 s + j] + a_lo[t][32 s + j]
// (in that order, in f32), as an f16 pair, for s < nsub.
__global__ void xsum_f16_kernel(const f16 *__restrict__ a, const f16 *__restrict__ a_lo, int lda,
                                int nsub, f16 *__restrict__ xs, f16 *__restrict__ xs_lo, int ldxs) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
  if (s >= nsub) return;
  const half8 *p = reinterpret_cast<const half8 *>(a + (size_t)t * lda + 32 * s);
  const half8 *q = reinterpret_cast<const half8 *>(a_lo + (size_t)t * lda + 32 * s);
  float sum = 0.f;
#pragma unroll
  for (int h = 0; h < 4; h++) {
    const half8 x = p[h], y = q[h];
#pragma unroll
    for (int e = 0; e < 8; e++) sum += (float)x[e] + (float)y[e];
  }
  split_f16(sum, xs[(size_t)t * ldxs + s], xs_lo[(size_t)t * ldxs + s]);
}

__global__ void embed_rows_kernel(const uint8_t *__restrict__ emb, uint32_t ty, size_t row_bytes,
                                  int H, uint32_t vocab, const uint32_t *__restrict__ tok, int T,
                                  float *__restrict__ x) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
  if (c >= H || t >= T) return;
  uint32_t id = tok[t];
  if (id >= vocab) id = vocab - 1;  // validated on the host; never read past the table
  x[(size_t)t * H + c] = value_dev(emb + (size_t)id * row_bytes, ty, (uint32_t)c);
}

// RMSNorm::forward (src/model.rs:65-73) per token row, rounded to f16.
// With xs set (H a multiple of 32), also the activation sums of the output
// that Q4_K products read: xs + xs_lo [row][s] = the sum of (hi + lo) over
// columns 32 s ... 32 s + 31 (a 32-lane half-wave of one pass), as f16 pairs.
__device__ __forceinline__ void half_wave_xsum(float v, int col, f16 *xs, f16 *xs_lo) {
#pragma unroll
  for (int b = 1; b < 32; b <<= 1) v += lane_partner(v, b);
  if ((threadIdx.x & 31) == 0) split_f16(v, xs[col >> 5], xs_lo[col >> 5]);
}

__global__ __launch_bounds__(256) void rmsnorm_rows_f16_kernel(const float *__restrict__ x,
                                                               const float *__restrict__ w,
                                                               f16 *__restrict__ out,
                                                               f16 *__restrict__ out_lo, int H,
                                                               float eps, f16 *__restrict__ xs,
                                                               f16 *__restrict__ xs_lo, int ldxs) {
#pragma clang fp contract(off)
  constexpr int kPer = 32;  // values a thread holds in registers (rows up to 8,192)
  __shared__ float red[4];
  const float *xr = x + (size_t)blockIdx.x * H;
  const bool held = H <= kPer * 256;
  float xv[kPer];
  float s = 0.f;
  if (held) {  // every load issued before the first is used
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int i = k * 256 + threadIdx.x;
      xv[k] = i < H ? xr[i] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < kPer; k++)
      if (k * 256 + threadIdx.x < H) s += xv[k] * xv[k];
  } else {
    for (int i = threadIdx.x; i < H; i += 256) s += xr[i] * xr[i];
  }
  s = wave_total(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  const float tot = red[0] + red[1] + red[2] + red[3];
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
  f16 *o = out + (size_t)blockIdx.x * H, *ol = out_lo + (size_t)blockIdx.x * H;
  auto emit = [&](int i, float xi) {  // i0 + threadIdx.x: whole passes, so the sums' shuffles see every lane
    float v = 0.f;
    if (i < H) {
      f16 h, l;
      split_f16(xi * (inv * w[i]), h, l);
      o[i] = h;
      ol[i] = l;
      v = (float)h + (float)l;
    }
    if (xs && i - (int)(threadIdx.x & 31) < H)
      half_wave_xsum(v, i, xs + (size_t)blockIdx.x * ldxs, xs_lo + (size_t)blockIdx.x * ldxs);
  };
  if (held) {
#pragma unroll
    for (int k = 0; k < kPer; k++)
      if (k * 256 < H) emit(k * 256 + threadIdx.x, xv[k]);
  } else {
    for (int i0 = 0; i0 < H; i0 += 256) emit(i0 + threadIdx.x, i0 + threadIdx.x < H ? xr[i0 + threadIdx.x] : 0.f);
  }
}

// Split-half RoPE (src/model.rs:87-95) of the row's query heads (in place)
// and key heads, and the K/V cache rows of position start + t
// (KVCache::update, src/cache.rs:38-53).
__global__ __launch_bounds__(256) void rope_append_kernel(float *__restrict__ q,
                                                          const float *__restrict__ k,
                                                          const float *__restrict__ v,
                                                          const float *__restrict__ rope, int start,
                                                          int nh, int nkv, int hd,
                                                          float *__restrict__ k_cache,
                                                          float *__restrict__ v_cache) {
  const int t = blockIdx.x, p = start + t, half = hd / 2, kvw = nkv * hd;
  const float *cs = rope + (size_t)p * hd, *sn = cs + half;
  float *qr = q + (size_t)t * nh * hd;
  for (int i = threadIdx.x; i < nh * half; i += blockDim.x) {
    const int h = i / half, j = i % half;
    const float re = qr[h * hd + j], im = qr[h * hd + j + half];
    qr[h * hd + j] = re * cs[j] - im * sn[j];
    qr[h * hd + j + half] = re * sn[j] + im * cs[j];
  }
  const float *kr = k + (size_t)t * kvw;
  float *kd = k_cache + (size_t)p * kvw;
  for (int i = threadIdx.x; i < nkv * half; i += blockDim.x) {
    const int h = i / half, j = i % half;
    const float re = kr[h * hd + j], im = kr[h * hd + j + half];
    kd[h * hd + j] = re * cs[j] - im * sn[j];
    kd[h * hd + j + half] = re * sn[j] + im * cs[j];
  }
  const float *vr = v + (size_t)t * kvw;
  float *vd = v_cache + (size_t)p * kvw;
  for (int i = threadIdx.x; i < kvw; i += blockDim.x) vd[i] = vr[i];
}

// Causal GQA attention (src/model.rs:206-231, softmax_inplace 298-313) for a
// tile of 16 query rows of one head, on f32 matrix cores: fp32 products and
// sums as the scalar loop has them, in another order.  The four waves take
// every fourth 16-key block of the causal range and keep a running max;
// their partial states are merged through LDS at the end.
//
// Both products keep the query index in lane % 16, so neither the scores nor
// the weights move between lanes:
//   S^T (keys x queries) = K Q^T     A = K rows, B = Q rows, contraction over
//                                    the head dims (lane group g holds dims
//                                    g*HD/4 ... g*HD/4 + HD/4 - 1)
//   O^T (dims x queries) = V^T P^T   A = V, B = the lane's own weights (the
//                                    score registers r = key 4g + r)
// and O^T's rows come out as dims (4g + r) * HD/16 + t for tile t: each lane
// ends with HD/4 consecutive dims of its query.  Keys past a query's position
// weigh 0 and their V rows are clamped to rows the tile may read.  The
// uniform fallback applies when no finite positive total remains.
template <int HD>
__global__ __launch_bounds__(256, 3) void attention_tile_kernel(const float *__restrict__ q,
                                                             const float *__restrict__ k_cache,
                                                             const float *__restrict__ v_cache,
                                                             int T, int start, int nh, int nkv,
                                                             float scale, f16 *__restrict__ out,
                                                             f16 *__restrict__ out_lo) {
  constexpr int DPL = HD / 4;  // head dims per lane in S (32 contraction steps at 128)
  constexpr int NT = HD / 16;  // 16-dim output tiles of O^T
  __shared__ float so[4][16][HD + 4];
  __shared__ float sm[4][16], sl[4][16];
  const int q0 = (gridDim.x - 1 - blockIdx.x) * 16;  // the longest tiles start first
  const int h = blockIdx.y, kvh = h / (nh / nkv), kvw = nkv * HD;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  const int pmax = start + min(q0 + 15, T - 1);
  const int pq = start + min(q0 + i, T - 1);  // rows past T mask as the last row
  float qv[DPL];
  {
    const float *qp = q + (size_t)min(q0 + i, T - 1) * nh * HD + h * HD + g * DPL;
#pragma unroll
    for (int d = 0; d < DPL; d += 4) *reinterpret_cast<float4 *>(qv + d) = *reinterpret_cast<const float4 *>(qp + d);
  }
  const float *kc = k_cache + (size_t)kvh * HD + g * DPL;
  const float *vc = v_cache + (size_t)kvh * HD + i * NT;
  f32x4 o[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float M = -INFINITY, L = 0.f;
  const int nb = pmax / 16 + 1;
  // The K rows of a block are loaded as soon as the previous block's scores
  // are computed and its V rows once its output products are issued, so each
  // load's latency overlaps the other half of an iteration.
  float kk[DPL], vv[4][NT];
  auto load_k = [&](int key0) {
    const float *kp = kc + (size_t)min(key0 + i, pmax) * kvw;
#pragma unroll
    for (int d = 0; d < DPL; d += 4) *reinterpret_cast<float4 *>(kk + d) = *reinterpret_cast<const float4 *>(kp + d);
  };
  auto load_v = [&](int key0) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const float *vp = vc + (size_t)min(key0 + 4 * g + s, pmax) * kvw;
#pragma unroll
      for (int t = 0; t < NT; t += (NT >= 4 ? 4 : NT)) {
        if constexpr (NT >= 4)
          *reinterpret_cast<float4 *>(&vv[s][t]) = *reinterpret_cast<const float4 *>(vp + t);
        else if constexpr (NT == 2)
          *reinterpret_cast<float2 *>(&vv[s][t]) = *reinterpret_cast<const float2 *>(vp + t);
        else
          vv[s][t] = vp[t];
      }
    }
  };
  if (wave < nb) {
    load_k(wave * 16);
    load_v(wave * 16);
  }
  for (int b = wave; b < nb; b += 4) {
    const int key0 = b * 16;
    // Two independent chains over the head dims (d mod 2), summed at the end.
    f32x4 sp[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int d = 0; d < DPL; d++) sp[d & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[d], qv[d], sp[d & 1], 0, 0, 0);
    const f32x4 st = sp[0] + sp[1];
    if (b + 4 < nb) load_k(key0 + 64);
    float sc[4], mc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      sc[r] = key0 + 4 * g + r <= pq ? st[r] * scale : -INFINITY;
      mc = fmaxf(mc, sc[r]);
    }
    mc = fmaxf(mc, lane_partner(mc, 16));
    mc = fmaxf(mc, lane_partner(mc, 32));
    const float Mn = fmaxf(M, mc);
    const bool live = Mn != -INFINITY;
    const float alpha = live ? expf(M - Mn) : 1.f;
    float pw[4], ls = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      pw[r] = live ? expf(sc[r] - Mn) : 0.f;
      ls += pw[r];
    }
    L = L * alpha + ls;
    M = Mn;
#pragma unroll
    for (int t = 0; t < NT; t++) {
      o[t] *= alpha;
#pragma unroll
      for (int s = 0; s < 4; s++) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[s][t], pw[s], o[t], 0, 0, 0);
    }
    if (b + 4 < nb) load_v(key0 + 64);
  }
  L += lane_partner(L, 16);
  L += lane_partner(L, 32);
  if (g == 0) {
    sm[wave][i] = M;
    sl[wave][i] = L;
  }
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) so[wave][i][(4 * g + r) * NT + t] = o[t][r];
  __syncthreads();
  // Merge: thread -> query qi, dims c*NT ... c*NT + NT - 1.
  const int qi = threadIdx.x >> 4, c = threadIdx.x & 15;
  if (q0 + qi >= T) return;
  float Mt = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; w++) Mt = fmaxf(Mt, sm[w][qi]);
  float Lt = 0.f, acc[NT];
#pragma unroll
  for (int e = 0; e < NT; e++) acc[e] = 0.f;
#pragma unroll
  for (int w = 0; w < 4; w++) {
    const float mw = sm[w][qi];
    const float f = mw == -INFINITY ? 0.f : expf(mw - Mt);
    Lt += sl[w][qi] * f;
#pragma unroll
    for (int e = 0; e < NT; e++) acc[e] += so[w][qi][c * NT + e] * f;
  }
  const int p = start + q0 + qi;
  const size_t at = (size_t)(q0 + qi) * nh * HD + h * HD + c * NT;
  if (isfinite(Lt) && Lt > 0.f) {
#pragma unroll
    for (int e = 0; e < NT; e++) split_f16(acc[e] / Lt, out[at + e], out_lo[at + e]);
  } else {
    const float *vp = v_cache + (size_t)kvh * HD + c * NT;
    for (int e = 0; e < NT; e++) {
      float vs = 0.f;
      for (int j = 0; j <= p; j++) vs += vp[(size_t)j * kvw + e];
      split_f16(vs / (float)(p + 1), out[at + e], out_lo[at + e]);
    }
  }
}

typedef _Float16 half4v __attribute__((ext_vector_type(4)));

// One layer's cache rows of positions [0, P) as f16 hi/lo planes for
// attention_f16_kernel, in blocks of 16 positions (16 * kvw halves a block
// and plane) laid out so that each MFMA operand load of a 16-key block reads
// one contiguous run:
//   K: [block][dim / 32][position % 16][dim % 32]
//   V: [block][dim][position % 16]      (V transposed within the block)
// Positions P .. P16 - 1 (P16 = P rounded up to 16) are zeros, so every block
// a query tile reads holds finite values.  kvw is a multiple of 32.  A
// workgroup moves one block of 16 positions x 64 dims, V through LDS.
__device__ __forceinline__ size_t kblk_index(int pos, int dim, int kvw) {
  return (size_t)(pos >> 4) * 16 * kvw + (size_t)(dim >> 5) * 512 + (pos & 15) * 32 + (dim & 31);
}
__device__ __forceinline__ size_t vblk_index(int pos, int dim, int kvw) {
  return (size_t)(pos >> 4) * 16 * kvw + (size_t)dim * 16 + (pos & 15);
}

__global__ __launch_bounds__(256) void kv_split_f16_kernel(const float *__restrict__ k,
                                                           const float *__restrict__ v, int kvw, int P,
                                                           f16 *__restrict__ kh, f16 *__restrict__ kl,
                                                           f16 *__restrict__ vh, f16 *__restrict__ vl) {
  __shared__ float tile[16][65];
  const int p0 = blockIdx.x * 16, d0 = blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int pl = ty * 4 + r, pos = p0 + pl, dim = d0 + tx;
    float kx = 0.f, vx = 0.f;
    if (pos < P && dim < kvw) {
      kx = k[(size_t)pos * kvw + dim];
      vx = v[(size_t)pos * kvw + dim];
    }
    if (dim < kvw) {
      const size_t o = kblk_index(pos, dim, kvw);
      split_f16(kx, kh[o], kl[o]);
    }
    tile[pl][tx] = vx;
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 4; r++) {  // 16 consecutive positions of 16 consecutive dims: 512 contiguous bytes
    const int pl = threadIdx.x & 15, dl = r * 16 + (threadIdx.x >> 4), dim = d0 + dl;
    if (dim < kvw) {
      const size_t o = vblk_index(p0 + pl, dim, kvw);
      split_f16(tile[pl][dl], vh[o], vl[o]);
    }
  }
}

// attention_tile_kernel's tiles, order, online softmax and merge with f16
// matrix products: q, K, V and the softmax weights as hi + lo pairs and three
// MFMAs per product (hi*hi, hi*lo, lo*hi), accumulated in f32.  Scores: S^T =
// K Q^T in v_mfma_f32_16x16x32_f16 steps of 32 head dims (K rows from kh/kl);
// output: O^T = V^T P^T in v_mfma_f32_16x16x16_f16 steps of 16 keys (V^T rows
// from vth/vtl, 16 output dims a tile).  One score step covers 32 dims where
// the f32 kernel's covers 4, which moves the kernel off the matrix cores'
// f32 rate.  HD >= 32.
template <int HD>
__global__ __launch_bounds__(256, 3) void attention_f16_kernel(const float *__restrict__ q,
                                                            const f16 *__restrict__ kh,
                                                            const f16 *__restrict__ kl,
                                                            const f16 *__restrict__ vh,
                                                            const f16 *__restrict__ vl,
                                                            const float *__restrict__ v_cache, int T,
                                                            int start, int nh, int nkv, float scale,
                                                            f16 *__restrict__ out, f16 *__restrict__ out_lo) {
  constexpr int NC = HD / 32;  // 32-dim score steps
  constexpr int NT = HD / 16;  // 16-dim output tiles
  __shared__ float so[4][16][HD + 4];
  __shared__ float sm[4][16], sl[4][16];
  const int q0 = (gridDim.x - 1 - blockIdx.x) * 16;  // the longest tiles start first
  const int h = blockIdx.y, kvh = h / (nh / nkv), kvw = nkv * HD;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
  const int pmax = start + min(q0 + 15, T - 1);
  const int pq = start + min(q0 + i, T - 1);  // rows past T mask as the last row
  half8 qh[NC], ql[NC];
  {
    const float *qp = q + (size_t)min(q0 + i, T - 1) * nh * HD + h * HD + 8 * g;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const float4 a = *reinterpret_cast<const float4 *>(qp + 32 * c);
      const float4 b = *reinterpret_cast<const float4 *>(qp + 32 * c + 4);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        f16 hi, lo;
        split_f16(x[e], hi, lo);
        qh[c][e] = hi;
        ql[c][e] = lo;
      }
    }
  }
  // Lane (i, g): K of key 16 b + i, dims 32 c + 8 g ...; V^T row (dim) 16 t + i,
  // keys 16 b + 4 g ... (kv_split_f16_kernel's block layout; 16 * kvw halves a block).
  const size_t ko = (size_t)kvh * (HD / 32) * 512 + i * 32 + 8 * g;
  const size_t vo = (size_t)(kvh * HD + i) * 16 + 4 * g;
  f32x4 o[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float M = -INFINITY, L = 0.f;
  const int nb = pmax / 16 + 1;
  half8 kah[NC], kal[NC];
  half4v vah[NT], val[NT];
  auto load_k = [&](int key0) {
    const size_t r = (size_t)key0 * kvw + ko;  // key0 / 16 blocks of 16 * kvw
#pragma unroll
    for (int c = 0; c < NC; c++) {
      kah[c] = *reinterpret_cast<const half8 *>(kh + r + 512 * c);
      kal[c] = *reinterpret_cast<const half8 *>(kl + r + 512 * c);
    }
  };
  auto load_v = [&](int key0) {
    const size_t r = (size_t)key0 * kvw + vo;
#pragma unroll
    for (int t = 0; t < NT; t++) {
      vah[t] = *reinterpret_cast<const half4v *>(vh + r + 256 * t);
      val[t] = *reinterpret_cast<const half4v *>(vl + r + 256 * t);
    }
  };
  if (wave < nb) {
    load_k(wave * 16);
    load_v(wave * 16);
  }
  for (int b = wave; b < nb; b += 4) {
    const int key0 = b * 16;
    f32x4 s0 = f32x4{0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kal[c], qh[c], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kah[c], ql[c], s1, 0, 0, 0);
      s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kah[c], qh[c], s0, 0, 0, 0);
    }
    const f32x4 st = s0 + s1;
    if (b + 4 < nb) load_k(key0 + 64);
    float sc[4], mc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      sc[r] = key0 + 4 * g + r <= pq ? st[r] * scale : -INFINITY;
      mc = fmaxf(mc, sc[r]);
    }
    mc = fmaxf(mc, lane_partner(mc, 16));
    mc = fmaxf(mc, lane_partner(mc, 32));
    const float Mn = fmaxf(M, mc);
    const bool live = Mn != -INFINITY;
    const float alpha = live ? expf(M - Mn) : 1.f;
    float ls = 0.f;
    half4v ph, pl;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float pw = live ? expf(sc[r] - Mn) : 0.f;
      ls += pw;
      f16 hi, lo;
      split_f16(pw, hi, lo);
      ph[r] = hi;
      pl[r] = lo;
    }
    L = L * alpha + ls;
    M = Mn;
#pragma unroll
    for (int t = 0; t < NT; t++) {
      o[t] *= alpha;
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(val[t], ph, o[t], 0, 0, 0);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(vah[t], pl, o[t], 0, 0, 0);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(vah[t], ph, o[t], 0, 0, 0);
    }
    if (b + 4 < nb) load_v(key0 + 64);
  }
  L += lane_partner(L, 16);
  L += lane_partner(L, 32);
  if (g == 0) {
    sm[wave][i] = M;
    sl[wave][i] = L;
  }
  // D layout of O^T: lane (i, g) holds query i, dims 16 t + 4 g + r.
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) so[wave][i][16 * t + 4 * g + r] = o[t][r];
  __syncthreads();
  // Merge: thread -> query qi, dims c*NT ... c*NT + NT - 1.
  const int qi = threadIdx.x >> 4, c = threadIdx.x & 15;
  if (q0 + qi >= T) return;
  float Mt = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; w++) Mt = fmaxf(Mt, sm[w][qi]);
  float Lt = 0.f, acc[NT];
#pragma unroll
  for (int e = 0; e < NT; e++) acc[e] = 0.f;
#pragma unroll
  for (int w = 0; w < 4; w++) {
    const float mw = sm[w][qi];
    const float f = mw == -INFINITY ? 0.f : expf(mw - Mt);
    Lt += sl[w][qi] * f;
#pragma unroll
    for (int e = 0; e < NT; e++) acc[e] += so[w][qi][c * NT + e] * f;
  }
  const int p = start + q0 + qi;
  const size_t at = (size_t)(q0 + qi) * nh * HD + h * HD + c * NT;
  if (isfinite(Lt) && Lt > 0.f) {
#pragma unroll
    for (int e = 0; e < NT; e++) split_f16(acc[e] / Lt, out[at + e], out_lo[at + e]);
  } else {
    const float *vp = v_cache + (size_t)kvh * HD + c * NT;
    for (int e = 0; e < NT; e++) {
      float vs = 0.f;
      for (int j = 0; j <= p; j++) vs += vp[(size_t)j * kvw + e];
      split_f16(vs / (float)(p + 1), out[at + e], out_lo[at + e]);
    }
  }
}

// With xs set (cols, the row length, a multiple of 32): the activation sums
// of the output as rmsnorm_rows_f16_kernel writes them.
__global__ __launch_bounds__(256) void swiglu_f16_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                                         f16 *__restrict__ out, f16 *__restrict__ out_lo,
                                                         size_t n, int cols, f16 *__restrict__ xs,
                                                         f16 *__restrict__ xs_lo, int ldxs) {
#pragma clang fp contract(off)
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  float v = 0.f;
  if (i < n) {
    const float x = g[i];
    f16 h, l;
    split_f16((x / (1.0f + expf(-x))) * u[i], h, l);
    out[i] = h;
    out_lo[i] = l;
    v = (float)h + (float)l;
  }
  const size_t i32 = i & ~(size_t)31;  // the half-wave's first element: n is a multiple of 32 with xs
  if (xs && i32 < n) {
    const size_t row = i32 / (size_t)cols;
    half_wave_xsum(v, (int)(i32 - row * cols), xs + row * ldxs, xs_lo + row * ldxs);
  }
}

__global__ void set_pos_kernel(int *pos, int value) { *pos = value; }


// C[t][j] = (C[t][j] when accumulating, else bias[j] or 0) + the split-K
// partials of splits 0, 1, ..., ksplit - 1, added in that order.
__global__ void split_reduce_kernel(float *__restrict__ c, int ldc, const float *__restrict__ bias,
                                    const float *__restrict__ part, int n, int t, int ksplit,
                                    int accumulate) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
  if (j >= n || r >= t) return;
  float *cp = c + (size_t)r * ldc + j;
  float v = accumulate ? *cp : (bias ? bias[j] : 0.f);
  for (int z = 0; z < ksplit; z++) v += part[((size_t)z * t + r) * n + j];
  *cp = v;
}

// split_reduce_kernel for a dual gate/up product: row f of gate is virtual
// column (f / 64) * 128 + f % 64, of up that + 64; h + hl [t][f] = silu(g) * u
// of the partial sums (split order), as swiglu_tile writes it, and with xso
// the 32-column sums (half_wave_xsum).
__global__ __launch_bounds__(256) void split_reduce_swiglu_kernel(const float *__restrict__ part, int nv, int t_rows,
                                                                  int ksplit, int rows, f16 *__restrict__ h,
                                                                  f16 *__restrict__ hl, int ldh,
                                                                  f16 *__restrict__ xso, f16 *__restrict__ xso_lo,
                                                                  int ldxso) {
#pragma clang fp contract(off)
  const int f = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
  float v = 0.f;
  if (f < rows) {
    const size_t vg = (size_t)(f >> 6) * 128 + (f & 63), zs = (size_t)t_rows * nv;
    const float *p = part + (size_t)t * nv;
    float x = 0.f, u = 0.f;
    for (int z = 0; z < ksplit; z++) {
      x += p[z * zs + vg];
      u += p[z * zs + vg + 64];
    }
    f16 hi, lo;
    split_f16((x / (1.0f + expf(-x))) * u, hi, lo);
    h[(size_t)t * ldh + f] = hi;
    hl[(size_t)t * ldh + f] = lo;
    v = (float)hi + (float)lo;
  }
  const int f32 = f & ~31;
  if (xso && f32 < rows) half_wave_xsum(v, f32, xso + (size_t)t * ldxso, xso_lo + (size_t)t * ldxso);
}

// split_reduce_kernel for a segmented product: column j of the partials
// belongs to segment i (seg_base[i] <= j < seg_base[i + 1]) and goes to
// seg_c[i] + r * seg_ldc[i] + (j - seg_base[i]), from its bias or 0 (or C
// when accumulating) plus the partials in split order.
struct SegOut {
  float *c[3];
  int ldc[3];
  const float *bias[3];
  int base[4];
  int nseg;
};
__global__ void split_reduce_seg_kernel(SegOut o, const float *__restrict__ part, int n, int t, int ksplit,
                                        int accumulate) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
  if (j >= n || r >= t) return;
  const int s = (o.nseg > 1 && j >= o.base[1]) + (o.nseg > 2 && j >= o.base[2]);
  const int jl = j - o.base[s];
  float *cp = o.c[s] + (size_t)r * o.ldc[s] + jl;
  float v = accumulate ? *cp : (o.bias[s] ? o.bias[s][jl] : 0.f);
  for (int z = 0; z < ksplit; z++) v += part[((size_t)z * t + r) * n + j];
  *cp = v;
}

}  // namespace

namespace {

// Workgroup slots of the device for the GEMM: two workgroups per CU (their
// LDS, 55-74 KB each, allows two).
int gemm_slots() {
  static int slots = 0;
  if (!slots) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    slots = 2 * cus;
  }
  return slots;
}

// The eight-wave kernel unless LLRS_PREFILL_GEMM=4 asks for the four-wave one
// (for comparisons; read at every launch, so a test can switch it).
bool eight_waves() {
  const char *e = getenv("LLRS_PREFILL_GEMM");
  return !(e && strcmp(e, "4") == 0);
}

void launch_tiles(const PrefillGemmArgs &a, int bm, hipStream_t s) {
  const dim3 grid((unsigned)((a.n + BN - 1) / BN), (unsigned)((a.t + bm - 1) / bm), (unsigned)a.ksplit);
  const size_t lds = (size_t)2 * (bm + BN) * LS * sizeof(f16);
  const bool w8 = eight_waves();
  if (a.type == LLRS_Q4_K && a.xs) {
    const size_t lds4 = lds + 2 * BN * sizeof(float);
    if (a.w2 && bm == 128)
      hipLaunchKernelGGL((prefill_gemm_k4_kernel<128, 4, true>), grid, dim3(512), lds4, s, a);
    else if (a.w2)
      hipLaunchKernelGGL((prefill_gemm_k4_kernel<64, 4, true>), grid, dim3(512), lds4, s, a);
    else if (bm == 128)
      hipLaunchKernelGGL((prefill_gemm_k4_kernel<128, 4, false>), grid, dim3(512), lds4, s, a);
    else
      hipLaunchKernelGGL((prefill_gemm_k4_kernel<64, 4, false>), grid, dim3(512), lds4, s, a);
    return;
  }

  if (a.type == LLRS_Q6_K && w8 && prefill_codes_enabled()) {
    const size_t lds6 = lds + 2 * BN * sizeof(float);
    if (bm == 128)
      hipLaunchKernelGGL((prefill_gemm8_kernel<LLRS_Q6_K, 128, true>), grid, dim3(512), lds6, s, a);
    else
      hipLaunchKernelGGL((prefill_gemm8_kernel<LLRS_Q6_K, 64, true>), grid, dim3(512), lds6, s, a);
    return;
  }
#define GEMM(T)                                                                         \
  if (w8 && bm == 128)                                                                  \
    hipLaunchKernelGGL((prefill_gemm8_kernel<T, 128, false>), grid, dim3(512), lds, s, a); \
  else if (w8)                                                                          \
    hipLaunchKernelGGL((prefill_gemm8_kernel<T, 64, false>), grid, dim3(512), lds, s, a);  \
  else if (bm == 128)                                                                   \
    hipLaunchKernelGGL((prefill_gemm_kernel<T, 128>), grid, dim3(256), lds, s, a);     \
  else                                                                                  \
    hipLaunchKernelGGL((prefill_gemm_kernel<T, 64>), grid, dim3(256), lds, s, a);
  switch (a.type) {
    case LLRS_Q4_K: GEMM(LLRS_Q4_K) break;
    case LLRS_Q6_K: GEMM(LLRS_Q6_K) break;
    case LLRS_Q8_0: GEMM(LLRS_Q8_0) break;
    case LLRS_Q5_0: GEMM(LLRS_Q5_0) break;
    default: GEMM(0xffffffffu) break;
  }
#undef GEMM
}

// The tiles of `a` with K split over `ksplit` workgroups, then the
// fixed-order reduction of their partials into C.
int launch_split(PrefillGemmArgs a, int bm, int ksplit, hipStream_t s) {
  a.ksplit = ksplit;
  if (ksplit > 1) {
    if (!a.part || (size_t)ksplit * a.t * a.n > a.part_cap)
      return set_error(LLRS_E_INVALID, "prefill GEMM: split-K scratch of %zu floats is too small (%d x %d x %d)",
                       a.part_cap, ksplit, a.t, a.n);
  }
  launch_tiles(a, bm, s);
  if (ksplit > 1 && a.w2)
    hipLaunchKernelGGL(split_reduce_swiglu_kernel, dim3((unsigned)((a.dual_rows + 255) / 256), (unsigned)a.t),
                       dim3(256), 0, s, a.part, a.n, a.t, ksplit, a.dual_rows, a.h, a.hl, a.ldh, a.xso, a.xso_lo,
                       a.ldxso);
  else if (ksplit > 1 && a.nseg > 0) {
    SegOut o{};
    o.nseg = a.nseg;
    for (int i = 0; i < a.nseg; i++) {
      o.c[i] = a.seg_c[i];
      o.ldc[i] = a.seg_ldc[i];
      o.bias[i] = a.seg_bias[i];
    }
    for (int i = 0; i <= a.nseg; i++) o.base[i] = a.seg_base[i];
    hipLaunchKernelGGL(split_reduce_seg_kernel, dim3((unsigned)((a.n + 255) / 256), (unsigned)a.t), dim3(256), 0,
                       s, o, a.part, a.n, a.t, ksplit, a.accumulate);
  } else if (ksplit > 1)
    hipLaunchKernelGGL(split_reduce_kernel, dim3((unsigned)((a.n + 255) / 256), (unsigned)a.t), dim3(256), 0,
                       s, a.c, a.ldc, a.bias, a.part, a.n, a.t, ksplit, a.accumulate);
  return LLRS_OK;
}

}  // namespace

size_t prefill_split_scratch_floats() { return (size_t)gemm_slots() * BN * 128; }

bool prefill_codes_enabled() {
  const char *e = getenv("LLRS_PREFILL_CODES");
  return eight_waves() && !(e && strcmp(e, "f32") == 0);
}

int launch_xsum_f16(const f16 *a, const f16 *a_lo, int lda, int k, int T, f16 *xs, f16 *xs_lo, int ldxs,
                    hipStream_t s) {
  if (k % 32 || lda % 8 || T <= 0 || ldxs < k / 32)
    return set_error(LLRS_E_UNSUPPORTED, "activation sums over %d columns (lda %d, ldxs %d)", k, lda, ldxs);
  const int nsub = k / 32;
  hipLaunchKernelGGL(xsum_f16_kernel, dim3((unsigned)((nsub + 63) / 64), (unsigned)T), dim3(64), 0, s, a,
                     a_lo, lda, nsub, xs, xs_lo, ldxs);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_prefill_gemm(const PrefillGemmArgs &g, hipStream_t s) {
  if (g.k % 32 || g.lda % 8 || g.n <= 0 || g.k <= 0 || g.t <= 0)
    return set_error(LLRS_E_UNSUPPORTED, "prefill GEMM shape %d x %d (lda %d) is not supported", g.n,
                     g.k, g.lda);
  if (g.xs && (g.type != LLRS_Q4_K || g.k % 256 || g.ldxs % 8 || g.ldxs < g.k / 32 + 56))
    return set_error(LLRS_E_UNSUPPORTED, "prefill GEMM: activation sums (ldxs %d) for a type %u product of %d columns",
                     g.ldxs, g.type, g.k);
  if (g.w2 && (!g.xs || g.dual_rows <= 0 || g.dual_rows % 64 || g.n != 2 * g.dual_rows || !g.h || !g.hl ||
               (g.xso && g.ldxso < g.dual_rows / 32)))
    return set_error(LLRS_E_UNSUPPORTED, "prefill GEMM: dual gate/up product of %d rows is not supported", g.dual_rows);
  // 128-token tiles when there are enough of them (the dequantized weight
  // tile then serves twice the tokens), else 64.  Products with fewer tiles
  // than half the slots split K over up to 8 workgroups (at least 6 K chunks
  // each).  Otherwise whole rounds of tiles run as they are, and a last
  // round that would fill at most half the slots runs as its own launch with
  // K split over the slots.  Split partials are reduced in split order, so C
  // is the same bit for bit on every run.
  const int slots = gemm_slots();
  const int ntiles = (g.n + BN - 1) / BN;
  const int bm = (g.t >= 256 && ntiles >= kTile128Rows) ? 128 : 64;
  const int mt = (g.t + bm - 1) / bm, chunks = (g.k + KC - 1) / KC;
  int ks = 1;
  while (ks < 8 && ntiles * mt * ks * 2 <= slots && chunks / (ks * 2) >= 6) ks *= 2;
  const int per_round = slots / mt;  // row tiles per round of slots
  const int full = (ks == 1 && per_round > 0) ? ntiles / per_round * per_round : 0;
  const int rem = ntiles - full;
  if (g.nseg > 0 && (g.type != LLRS_Q4_K || !g.xs || g.nseg > 3 || g.seg_base[0] != 0 || g.seg_base[g.nseg] != g.n))
    return set_error(LLRS_E_UNSUPPORTED, "prefill GEMM: segmented product of %d segments is not supported", g.nseg);
  for (int i = 1; i < g.nseg; i++)
    if (g.seg_base[i] % BN || g.seg_base[i] <= g.seg_base[i - 1])
      return set_error(LLRS_E_UNSUPPORTED, "prefill GEMM: segment boundary %d is not a multiple of %d", g.seg_base[i], BN);
  if (g.nseg == 0 && full > 0 && rem > 0 && rem * mt * 2 <= slots) {
    PrefillGemmArgs m = g;
    m.n = full * BN;
    m.ksplit = 1;
    if (g.w2) m.dual_rows = full * BN / 2;
    launch_tiles(m, bm, s);
    PrefillGemmArgs r = g;
    r.n = g.n - full * BN;
    if (g.w2) {  // the remaining gate/up rows from full * 64 on
      const size_t f = (size_t)full * BN / 2;
      r.w = g.w + f * (size_t)g.row_bytes;
      r.w2 = g.w2 + f * (size_t)g.row_bytes;
      r.dual_rows = g.dual_rows - (int)f;
      r.h = g.h + f;
      r.hl = g.hl + f;
      if (g.xso) {
        r.xso = g.xso + f / 32;
        r.xso_lo = g.xso_lo + f / 32;
      }
    } else {
      r.w = g.w + (size_t)full * BN * (size_t)g.row_bytes;
      r.c = g.c + (size_t)full * BN;
      r.bias = g.bias ? g.bias + (size_t)full * BN : nullptr;
    }
    LLRS_TRY(launch_split(r, bm, std::max(1, std::min({8, slots / (rem * mt), chunks / 6})), s));
  } else {
    LLRS_TRY(launch_split(g, bm, ks, s));
  }
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_embed_rows(const llrs_tensor *emb, const uint32_t *tok, int T, float *x, hipStream_t s) {
  const int H = (int)emb->cols;
  hipLaunchKernelGGL(embed_rows_kernel, dim3((H + 255) / 256, T), dim3(256), 0, s, emb->dev,
                     emb->type, emb->row_bytes, H, (uint32_t)emb->rows, tok, T, x);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_rmsnorm_rows_f16(const float *x, const float *w, f16 *out, f16 *out_lo, int T, int H,
                            float eps, hipStream_t s, f16 *xs, f16 *xs_lo, int ldxs) {
  if (xs && (H % 32 || ldxs < H / 32))
    return set_error(LLRS_E_UNSUPPORTED, "activation sums over %d columns (ldxs %d)", H, ldxs);
  hipLaunchKernelGGL(rmsnorm_rows_f16_kernel, dim3(T), dim3(256), 0, s, x, w, out, out_lo, H, eps, xs, xs_lo,
                     ldxs);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_rope_append(float *q, const float *k, const float *v, const float *rope, int T, int start,
                       int nh, int nkv, int hd, float *k_cache, float *v_cache, hipStream_t s) {
  hipLaunchKernelGGL(rope_append_kernel, dim3(T), dim3(256), 0, s, q, k, v, rope, start, nh, nkv, hd,
                     k_cache, v_cache);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

bool prefill_attention_f16() {
  const char *e = getenv("LLRS_PREFILL_ATTN");
  return !(e && strcmp(e, "f32") == 0);
}

int launch_attention_rows(const float *q, const float *k_cache, const float *v_cache, int T,
                          int start, int nh, int nkv, int hd, float scale, f16 *out, f16 *out_lo,
                          hipStream_t s, const PrefillKvF16 *kvf) {
  if (T <= 0 || nkv <= 0 || nh % nkv)
    return set_error(LLRS_E_UNSUPPORTED, "attention over %d rows with %d/%d heads", T, nh, nkv);
  const dim3 grid((unsigned)((T + 15) / 16), (unsigned)nh);
  if (kvf && hd >= 32 && prefill_attention_f16()) {
    const int kvw = nkv * hd, P = start + T;
    if (((P + 15) & ~15) > kvf->positions || kvf->kvw != kvw || kvw % 32)
      return set_error(LLRS_E_INVALID, "prefill attention: f16 K/V scratch of %d positions x %d for %d x %d",
                       kvf->positions, kvf->kvw, P, kvw);
    hipLaunchKernelGGL(kv_split_f16_kernel, dim3((unsigned)((P + 15) / 16), (unsigned)((kvw + 63) / 64)),
                       dim3(256), 0, s, k_cache, v_cache, kvw, P, kvf->kh, kvf->kl, kvf->vh, kvf->vl);
#define ATT16(D)                                                                                      \
  hipLaunchKernelGGL(attention_f16_kernel<D>, grid, dim3(256), 0, s, q, kvf->kh, kvf->kl, kvf->vh, kvf->vl, \
                     v_cache, T, start, nh, nkv, scale, out, out_lo)
    switch (hd) {
      case 32: ATT16(32); break;
      case 64: ATT16(64); break;
      case 128: ATT16(128); break;
      default: return set_error(LLRS_E_UNSUPPORTED, "attention head_dim %d is not supported", hd);
    }
#undef ATT16
    LLRS_HIP(hipGetLastError());
    return LLRS_OK;
  }
#define ATT(D)                                                                                   \
  hipLaunchKernelGGL(attention_tile_kernel<D>, grid, dim3(256), 0, s, q, k_cache, v_cache, T, start, \
                     nh, nkv, scale, out, out_lo)
  switch (hd) {
    case 16: ATT(16); break;
    case 32: ATT(32); break;
    case 64: ATT(64); break;
    case 128: ATT(128); break;
    default: return set_error(LLRS_E_UNSUPPORTED, "attention head_dim %d is not supported", hd);
  }
#undef ATT
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_swiglu_f16(const float *g, const float *u, f16 *out, f16 *out_lo, size_t n, int cols, hipStream_t s,
                      f16 *xs, f16 *xs_lo, int ldxs) {
  if (xs && (cols <= 0 || cols % 32 || n % (size_t)cols || ldxs < cols / 32))
    return set_error(LLRS_E_UNSUPPORTED, "activation sums over rows of %d columns (ldxs %d)", cols, ldxs);
  hipLaunchKernelGGL(swiglu_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, out,
                     out_lo, n, cols, xs, xs_lo, ldxs);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_set_pos(int *pos, int value, hipStream_t s) {
  hipLaunchKernelGGL(set_pos_kernel, dim3(1), dim3(1), 0, s, pos, value);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

}  // namespace llrs
