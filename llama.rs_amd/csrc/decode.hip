// Per-token decode kernels of Qwen2Model::forward_impl (src/model.rs:135-271)
// other than the weight GEMVs: embedding gather, RMSNorm, RoPE + KV append,
// GQA attention, SiLU*up, greedy argmax, position advance.
//
// The token and position live in device memory (tok_by_pos[], *pos), so the
// same launch sequence can be captured once into a hipGraph and replayed for
// every decode step with nothing returning to the host.
#include <hip/hip_runtime.h>

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
__device__ float block_max(float v, float *sh) {
  v = wave_max_f(v);
  int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  float t = -INFINITY;
  for (int i = 0; i < nw; i++) t = fmaxf(t, sh[i]);
  return t;
}

// embed_tokens.row_into(token) (src/model.rs:170-171): bit-exact dequant.
__global__ void embed_kernel(const uint8_t *__restrict__ emb, uint32_t ty, size_t row_bytes, int H,
                             const uint32_t *__restrict__ tok_by_pos, const int *__restrict__ pos,
                             float *__restrict__ out) {
  int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= H) return;
  uint32_t tok = tok_by_pos[*pos];
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

// Split-half RoPE on every Q and KV head (src/model.rs:87-95, 188-203) with the
// position's cos/sin row, then KVCache::update (src/cache.rs:38-53).
__global__ void rope_kv_kernel(float *__restrict__ q, const float *__restrict__ k,
                               const float *__restrict__ v, const float *__restrict__ rope,
                               const int *__restrict__ pos, float *__restrict__ kc,
                               float *__restrict__ vc, int nh, int nkv, int hd) {
#pragma clang fp contract(off)
  int p = *pos;
  int half = hd / 2, kvw = nkv * hd;
  const float *cs = rope + (size_t)p * hd;  // [cos(half) | sin(half)]
  const float *sn = cs + half;
  float *krow = kc + (size_t)p * kvw, *vrow = vc + (size_t)p * kvw;
  int total = (nh + nkv) * half;
  for (int t = threadIdx.x; t < total; t += blockDim.x) {
    int h = t / half, i = t % half;
    if (h < nh) {
      float *x = q + h * hd;
      float re = x[i], im = x[i + half];
      x[i] = re * cs[i] - im * sn[i];
      x[i + half] = re * sn[i] + im * cs[i];
    } else {
      int kh = h - nh;
      const float *x = k + kh * hd;
      float re = x[i], im = x[i + half];
      krow[kh * hd + i] = re * cs[i] - im * sn[i];
      krow[kh * hd + i + half] = re * sn[i] + im * cs[i];
    }
  }
  for (int t = threadIdx.x; t < kvw; t += blockDim.x) vrow[t] = v[t];
}

// GQA attention for one query head per block (src/model.rs:206-231) with
// softmax_inplace (src/model.rs:298-313), including its uniform fallback.
__global__ __launch_bounds__(256) void attention_kernel(const float *__restrict__ q,
                                                        const float *__restrict__ kc,
                                                        const float *__restrict__ vc,
                                                        const int *__restrict__ pos,
                                                        float *__restrict__ scores_all,
                                                        float *__restrict__ out, int nh, int nkv,
                                                        int hd, int max_seq, float scale) {
#pragma clang fp contract(off)
  __shared__ float sh[16];
  __shared__ float part[1024];
  int h = blockIdx.x;
  int n = *pos + 1;
  int kvh = h / (nh / nkv), kvw = nkv * hd;
  const float *qh = q + h * hd;
  float *sc = scores_all + (size_t)h * max_seq;
  float mx = -INFINITY;
  for (int p = threadIdx.x; p < n; p += blockDim.x) {
    const float *kr = kc + (size_t)p * kvw + kvh * hd;
    float dot = 0.f;
    for (int d = 0; d < hd; d++) dot += qh[d] * kr[d];
    float s = dot * scale;
    sc[p] = s;
    mx = fmaxf(mx, s);
  }
  mx = block_max(mx, sh);
  float sum = 0.f;
  for (int p = threadIdx.x; p < n; p += blockDim.x) {
    float e = expf(sc[p] - mx);
    sc[p] = e;
    sum += e;
  }
  sum = block_sum(sum, sh);
  bool ok = isfinite(sum) && sum > 0.f;
  float uni = 1.0f / (float)n;
  __syncthreads();
  int parts = blockDim.x / hd;  // hd divides 256 for hd in {64, 128, 256}
  int d = threadIdx.x % hd, pi = threadIdx.x / hd;
  float acc = 0.f;
  if (pi < parts)
    for (int p = pi; p < n; p += parts) {
      float wgt = ok ? sc[p] / sum : uni;
      acc += wgt * vc[(size_t)p * kvw + kvh * hd + d];
    }
  part[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x < hd) {
    float t = 0.f;
    for (int i = 0; i < parts; i++) t += part[i * hd + threadIdx.x];
    out[h * hd + threadIdx.x] = t;
  }
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
// index among equal maxima.  Advances *pos by one first (the logits belong
// to the token just processed) and writes the winner as the token of the
// new position, so the next replay embeds it.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ logits, int n,
                                                      int *__restrict__ pos,
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
    *pos = p;
    tok_by_pos[p] = tok;
    *next_token = tok;
  }
}

__global__ void advance_kernel(int *pos) { *pos += 1; }

// ------------------------------------------------------------------ launchers

int launch_embed(const llrs_tensor *emb, const uint32_t *tok_by_pos, const int *pos, float *out,
                 hipStream_t s) {
  int H = (int)emb->cols;
  hipLaunchKernelGGL(embed_kernel, dim3((H + 255) / 256), dim3(256), 0, s, emb->dev, emb->type,
                     emb->row_bytes, H, tok_by_pos, pos, out);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_rmsnorm(const float *in, const float *w, float *out, int n, float eps, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, in, w, out, n, eps);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_rope_kv(float *q, const float *k, const float *v, const float *rope, const int *pos,
                   float *kc, float *vc, int nh, int nkv, int hd, hipStream_t s) {
  hipLaunchKernelGGL(rope_kv_kernel, dim3(1), dim3(512), 0, s, q, k, v, rope, pos, kc, vc, nh, nkv,
                     hd);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_attention(const float *q, const float *kc, const float *vc, const int *pos,
                     float *scores, float *out, int nh, int nkv, int hd, int max_seq,
                     hipStream_t s) {
  if (hd > 256 || 256 % hd)
    return set_error(LLRS_E_UNSUPPORTED, "head_dim %d is not supported (must divide 256)", hd);
  float scale = 1.0f / sqrtf((float)hd);
  hipLaunchKernelGGL(attention_kernel, dim3(nh), dim3(256), 0, s, q, kc, vc, pos, scores, out, nh,
                     nkv, hd, max_seq, scale);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_silu_mul(const float *g, const float *u, float *out, int n, hipStream_t s) {
  hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, s, g, u, out, n);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_argmax(const float *logits, int n, int *pos, uint32_t *tok_by_pos, uint32_t *next_token,
                  int advance, hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, logits, n, pos, tok_by_pos,
                     next_token, advance);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_advance(int *pos, hipStream_t s) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, pos);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

}  // namespace llrs
