// Per-token decode kernels of Qwen2Model::forward_impl (src/model.rs:135-271)
// other than the weight GEMVs: embedding gather, RMSNorm, fused RoPE + KV
// append + GQA attention, SiLU*up, greedy argmax, position advance.
//
// The token and position live in device memory (tok_by_pos[], *pos), so the
// same launch sequence is captured once into a hipGraph and replayed for
// every decode step with nothing returning to the host.  Every device read
// of *pos is bounded by the context length, so even a corrupted position can
// never index outside the cache.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "common.h"
#include "decode.h"
#include "quant_dev.h"

namespace llrs {

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Block-wide reductions for blockDim.x a multiple of 64 (<= 1024).
__device__ float block_sum(float v, float *sh) {
  v = wave_sum_f(v);
  int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; i++) t += sh[i];
  return t;
}

__device__ __forceinline__ int bounded_pos(const int *pos, int max_seq) {
  int p = *pos;
  return p < 0 ? 0 : p >= max_seq ? max_seq - 1 : p;
}

// embed_tokens.row_into(token) (src/model.rs:170-171): bit-exact dequant.
__global__ void embed_kernel(const uint8_t *__restrict__ emb, uint32_t ty, size_t row_bytes, int H,
                             uint32_t vocab, const uint32_t *__restrict__ tok_by_pos,
                             const int *__restrict__ pos, int max_seq, float *__restrict__ out) {
  int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= H) return;
  uint32_t tok = tok_by_pos[bounded_pos(pos, max_seq)];
  if (tok >= vocab) tok = vocab - 1;  // tokens are validated on the host; never read past the table
  out[c] = value_dev(emb + (size_t)tok * row_bytes, ty, (uint32_t)c);
}

// RMSNorm::forward (src/model.rs:65-73): out = in * (1/sqrt(mean(in^2)+eps) * w).
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float *__restrict__ in,
                                                       const float *__restrict__ w,
                                                       float *__restrict__ out, int n, float eps) {
#pragma clang fp contract(off)
  __shared__ float sh[16];
  float s = 0.f;
  for (int i = threadIdx.x; i < n; i += blockDim.x) s += in[i] * in[i];
  s = block_sum(s, sh);
  float inv = 1.0f / sqrtf(s / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = in[i] * (inv * w[i]);
}

// ------------------------------------------------------------------ attention
//
// One workgroup per (KV head, chunk of kChunk positions); the chunks past the
// current position exit at once, so one grid (sized for the whole context)
// serves every position of a captured graph.  Per chunk: split-half RoPE
// (src/model.rs:87-95) on the group's query heads, scores q.k * 1/sqrt(hd),
// softmax partials (max, sum of exp) and exp-weighted V sums
// (src/model.rs:206-231, softmax_inplace 298-313).  The chunk holding the
// current position also rotates the new key and appends key and value to
// the cache (KVCache::update, src/cache.rs:38-53).  The last chunk of a KV
// head to finish (atomic counter) merges the partials; if the total is not
// finite and positive the weights fall back to uniform, as softmax_inplace does.

constexpr int kChunk = 64;  // positions per workgroup (one per lane of a wave)

__global__ __launch_bounds__(256) void attention_kernel(AttnArgs a) {
  extern __shared__ __align__(16) float sm[];
  const int G = a.nh / a.nkv, hd = a.hd, half = hd / 2, kvw = a.nkv * hd;
  const int kvh = blockIdx.y, chunk = blockIdx.x;
  const int pos = bounded_pos(a.pos, a.max_seq);
  const int c0 = chunk * kChunk;
  if (c0 > pos) return;
  const int n_active = pos / kChunk + 1;
  const int c1 = min(c0 + kChunk, pos + 1);  // exclusive
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float *qs = sm;                     // [G][hd] rotated queries
  float *e = qs + G * hd;             // [G][kChunk] scores, then exp weights
  __shared__ float mh[16], lh[16];    // per-head chunk max and sum of exp
  const float *cs = a.rope + (size_t)pos * hd, *sn = cs + half;

  for (int t = tid; t < G * half; t += blockDim.x) {
    int h = t / half, i = t % half;
    const float *x = a.q + (size_t)(kvh * G + h) * hd;
    float re = x[i], im = x[i + half];
    qs[h * hd + i] = re * cs[i] - im * sn[i];
    qs[h * hd + i + half] = re * sn[i] + im * cs[i];
  }
  float *kc = a.k_cache, *vc = a.v_cache;
  if (pos >= c0 && pos < c1) {  // this chunk appends the new key (rotated) and value
    float *krow = kc + (size_t)pos * kvw + kvh * hd, *vrow = vc + (size_t)pos * kvw + kvh * hd;
    const float *kx = a.k + kvh * hd, *vx = a.v + kvh * hd;
    for (int i = tid; i < half; i += blockDim.x) {
      float re = kx[i], im = kx[i + half];
      krow[i] = re * cs[i] - im * sn[i];
      krow[i + half] = re * sn[i] + im * cs[i];
    }
    for (int i = tid; i < hd; i += blockDim.x) vrow[i] = vx[i];
  }
  __syncthreads();

  // Scores: 4 lanes per position, each a quarter of the head dimension.
  const float scale = a.scale;
  for (int base = 0; base < kChunk; base += blockDim.x / 4) {
    int pl = base + tid / 4, qd = tid & 3;
    int p = c0 + pl;
    const int dq = hd / 4;
    float part[16];
#pragma unroll
    for (int h = 0; h < 16; h++) part[h] = 0.f;
    if (pl < kChunk && p < c1) {
      const float *kr = kc + (size_t)p * kvw + kvh * hd + qd * dq;
      for (int d = 0; d < dq; d += 4) {
        float4 kv4 = *reinterpret_cast<const float4 *>(kr + d);
#pragma unroll
        for (int h = 0; h < 16; h++) {
          if (h < G) {
            const float *qq = qs + h * hd + qd * dq + d;
            part[h] += qq[0] * kv4.x + qq[1] * kv4.y + qq[2] * kv4.z + qq[3] * kv4.w;
          }
        }
      }
    }
#pragma unroll
    for (int h = 0; h < 16; h++) {
      part[h] += __shfl_xor(part[h], 1, 64);
      part[h] += __shfl_xor(part[h], 2, 64);
    }
    if (pl < kChunk && qd == 0) {
#pragma unroll
      for (int h = 0; h < 16; h++)
        if (h < G) e[h * kChunk + pl] = p < c1 ? part[h] * scale : -INFINITY;
    }
  }
  __syncthreads();

  // Softmax partials: one wave per head, one lane per position.
  const int nw = blockDim.x >> 6;
  for (int h = wave; h < G; h += nw) {
    float s = e[h * kChunk + lane];
    bool valid = c0 + lane < c1;
    float m = wave_max_f(valid ? s : -INFINITY);
    float x = valid ? expf(s - m) : 0.f;
    e[h * kChunk + lane] = x;
    float l = wave_sum_f(x);
    if (lane == 0) {
      mh[h] = m;
      lh[h] = l;
    }
  }
  __syncthreads();

  // Exp-weighted V sums (and plain V sums for the uniform fallback): thread
  // (dv, ps) holds four head dimensions and the positions ps, ps + PS, ...;
  // its V loads are issued together, then partial sums meet in LDS.
  float *part_o = a.scratch + ((size_t)kvh * a.max_chunks + chunk) * a.part_stride;
  const int d4n = hd / 4;                  // float4 columns per head
  const int PS = blockDim.x / d4n;         // position slots
  const int dv = tid % d4n, ps = tid / d4n;
  float4 acc[16];
#pragma unroll
  for (int h = 0; h < 16; h++) acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 vs = make_float4(0.f, 0.f, 0.f, 0.f);
  {
    constexpr int kMaxPer = 16;  // kChunk / PS with PS >= 4 (hd <= 256)
    float4 vv[kMaxPer];
#pragma unroll
    for (int i = 0; i < kMaxPer; i++) {
      int p = c0 + ps + i * PS;
      vv[i] = (ps + i * PS < kChunk && p < c1)
                  ? *reinterpret_cast<const float4 *>(vc + (size_t)p * kvw + kvh * hd + 4 * dv)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < kMaxPer; i++) {
      int pl = ps + i * PS;
      if (pl >= kChunk || c0 + pl >= c1) continue;
      vs.x += vv[i].x; vs.y += vv[i].y; vs.z += vv[i].z; vs.w += vv[i].w;
#pragma unroll
      for (int h = 0; h < 16; h++) {
        if (h >= G) continue;
        float w = e[h * kChunk + pl];
        acc[h].x += w * vv[i].x; acc[h].y += w * vv[i].y;
        acc[h].z += w * vv[i].z; acc[h].w += w * vv[i].w;
      }
    }
  }
  __syncthreads();  // e[] is reused below as the reduction buffer
  float *red = qs;  // [PS][G + 1][hd], fits in the qs + e region
#pragma unroll
  for (int h = 0; h < 16; h++)
    if (h < G) *reinterpret_cast<float4 *>(red + ((size_t)ps * (G + 1) + h) * hd + 4 * dv) = acc[h];
  *reinterpret_cast<float4 *>(red + ((size_t)ps * (G + 1) + G) * hd + 4 * dv) = vs;
  __syncthreads();
  for (int t = tid; t < (G + 1) * hd; t += blockDim.x) {
    float s = 0.f;
    for (int q = 0; q < PS; q++) s += red[(size_t)q * (G + 1) * hd + t];
    part_o[t] = s;  // [G][hd] exp-weighted sums, then [hd] plain sums
  }
  if (tid < G) {
    part_o[G * hd + hd + tid] = mh[tid];
    part_o[G * hd + hd + G + tid] = lh[tid];
  }

  // The last chunk of this KV head merges all partials.
  __threadfence();
  __syncthreads();
  __shared__ int last;
  if (tid == 0) last = atomicAdd(a.counters + kvh, 1u) == (unsigned)(n_active - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  const float *base = a.scratch + (size_t)kvh * a.max_chunks * a.part_stride;
  float *wsm = qs;  // [n_active][G] rescale weights, then [G] totals
  for (int t = tid; t < n_active * G; t += blockDim.x)
    wsm[t] = base[(size_t)(t / G) * a.part_stride + G * hd + hd + (t % G)];
  __syncthreads();
  __shared__ float Lh[16];
  if (tid < G) {
    float M = -INFINITY;
    for (int c = 0; c < n_active; c++) M = fmaxf(M, wsm[c * G + tid]);
    float L = 0.f;
    for (int c = 0; c < n_active; c++) {
      float w = expf(wsm[c * G + tid] - M);
      L += w * base[(size_t)c * a.part_stride + G * hd + hd + G + tid];
      wsm[c * G + tid] = w;
    }
    Lh[tid] = L;
  }
  __syncthreads();
  for (int t = tid; t < G * hd; t += blockDim.x) {
    int h = t / hd, dd = t % hd;
    float O = 0.f, V = 0.f;
#pragma unroll 8
    for (int c = 0; c < n_active; c++) {
      const float *pc = base + (size_t)c * a.part_stride;
      O += wsm[c * G + h] * pc[h * hd + dd];
      V += pc[G * hd + dd];
    }
    float L = Lh[h];
    float out = (isfinite(L) && L > 0.f) ? O / L : V / (float)(pos + 1);
    a.out[(size_t)(kvh * G + h) * hd + dd] = out;
  }
  if (tid == 0) a.counters[kvh] = 0u;
}

// silu(gate) * up (src/model.rs:251-254).
__global__ void silu_mul_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                float *__restrict__ out, int n) {
#pragma clang fp contract(off)
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    float x = g[i];
    out[i] = (x / (1.0f + expf(-x))) * u[i];
  }
}

// f32::total_cmp order as an unsigned key (larger key = larger under total_cmp).
__device__ __forceinline__ uint32_t total_order_key(float f) {
  int32_t b = __float_as_int(f);
  b ^= (int32_t)((uint32_t)(b >> 31) >> 1);
  return (uint32_t)b ^ 0x80000000u;
}

// argmax_current_logits (src/engine.rs:233-241): max under total_cmp, last
// index among equal maxima.  Advances *pos by `advance` first (the logits
// belong to the token just processed) and writes the winner as the token of
// that position, so the next replay embeds it.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ logits, int n,
                                                      int *__restrict__ pos, int max_seq,
                                                      uint32_t *__restrict__ tok_by_pos,
                                                      uint32_t *__restrict__ next_token,
                                                      int advance) {
  __shared__ unsigned long long sh[16];
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    unsigned long long key = ((unsigned long long)total_order_key(logits[i]) << 32) | (uint32_t)i;
    best = key > best ? key : best;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    unsigned long long other = __shfl_xor(best, o, 64);
    best = other > best ? other : best;
  }
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) best = sh[i] > best ? sh[i] : best;
    uint32_t tok = (uint32_t)(best & 0xffffffffu);
    int p = *pos + advance;
    if (p < 0) p = 0;
    if (p > max_seq) p = max_seq;  // tok_by_pos has max_seq + 1 entries
    *pos = p;
    tok_by_pos[p] = tok;
    *next_token = tok;
  }
}

__global__ void advance_kernel(int *pos, int max_seq) {
  int p = *pos + 1;
  *pos = p > max_seq ? max_seq : p;
}

// ------------------------------------------------------------------ launchers

int launch_embed(const llrs_tensor *emb, const uint32_t *tok_by_pos, const int *pos, int max_seq,
                 float *out, hipStream_t s) {
  int H = (int)emb->cols;
  hipLaunchKernelGGL(embed_kernel, dim3((H + 255) / 256), dim3(256), 0, s, emb->dev, emb->type,
                     emb->row_bytes, H, (uint32_t)emb->rows, tok_by_pos, pos, max_seq, out);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_rmsnorm(const float *in, const float *w, float *out, int n, float eps, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, in, w, out, n, eps);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

size_t attention_scratch_floats(int nh, int nkv, int hd, int max_seq) {
  int G = nh / nkv;
  size_t chunks = (size_t)(max_seq + kChunk - 1) / kChunk;
  size_t stride = (size_t)G * hd + hd + 2 * G;
  return (size_t)nkv * chunks * stride;
}

int launch_attention(const AttnArgs &args, hipStream_t s) {
  int G = args.nh / args.nkv;
  if (args.nh % args.nkv || G > 16 || args.hd > 256 || args.hd % 16 || 256 % args.hd)
    return set_error(LLRS_E_UNSUPPORTED, "attention geometry %d/%d heads, head_dim %d is not supported",
                     args.nh, args.nkv, args.hd);
  // Dynamic LDS: queries + scores; reused as the [PS][G+1][hd] V reduction
  // buffer (PS * hd = 1024 floats per head) and the combine's weights.
  size_t floats = (size_t)G * args.hd + (size_t)G * kChunk;
  floats = std::max(floats, (size_t)1024 * (G + 1));
  floats = std::max(floats, (size_t)args.max_chunks * G);
  size_t lds = floats * sizeof(float);
  if (lds > 160 * 1024)
    return set_error(LLRS_E_UNSUPPORTED, "attention needs %zu bytes of LDS (context too long)", lds);
  dim3 grid((unsigned)args.max_chunks, (unsigned)args.nkv);
  hipLaunchKernelGGL(attention_kernel, grid, dim3(256), lds, s, args);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int attention_chunks(int max_seq) { return (max_seq + kChunk - 1) / kChunk; }

int launch_silu_mul(const float *g, const float *u, float *out, int n, hipStream_t s) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, s, g, u, out, n);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_argmax(const float *logits, int n, int *pos, int max_seq, uint32_t *tok_by_pos,
                  uint32_t *next_token, int advance, hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, logits, n, pos, max_seq, tok_by_pos,
                     next_token, advance);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_advance(int *pos, int max_seq, hipStream_t s) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, pos, max_seq);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

}  // namespace llrs
