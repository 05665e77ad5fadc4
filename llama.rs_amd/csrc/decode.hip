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
#include <type_traits>

#include "common.h"
#include "attention_dev.h"
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


// embed_tokens.row_into(token) (src/model.rs:170-171): bit-exact dequant.
__global__ void embed_kernel(const uint8_t *__restrict__ emb, uint32_t ty, size_t row_bytes, int H,
                             uint32_t vocab, const uint32_t *__restrict__ tok_by_pos,
                             const int *__restrict__ pos, int max_seq, float *__restrict__ out,
                             unsigned *__restrict__ epoch, unsigned *__restrict__ clear,
                             int nclear) {
  int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c == 0) *epoch += 1u;       // a fresh tag for this step's attention partials
  if (c < nclear) clear[c] = 0u;  // the step's barrier counters start at zero
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

template <int HD>
__global__ __launch_bounds__(64 * kTaskItems) void attention_kernel(AttnArgs a) {
  __shared__ __align__(16) float qs[kTaskItems][HD], kn[kTaskItems][HD];
  __shared__ __align__(16) float part[kTaskItems * AttnGeom<HD>::kPart];
  a.tag = *a.epoch * (unsigned)a.nlayers + (unsigned)a.layer;
  // Grid (head, y): block y runs tasks y, y + Y, y + 2Y, .. (Y = gridDim.y,
  // up to kTaskItems / T of them), so the tasks spread over the blocks as
  // the persistent kernel spreads them over its workgroups.  Blocks past the
  // head's tasks exit at once.  A head's last task waits only for tasks
  // that never wait (one waiting block per head), so every wait ends.
  const int pos = bounded_pos(a.pos, a.max_seq);
  const int S = attention_span(pos, a.nh);
  const int n_items = pos / (S * kChunk) + 1, T = attention_task_items(n_items, a.fold_max);
  if ((int)blockIdx.y >= (n_items + T - 1) / T) return;
  const int wave = threadIdx.x >> 6;
  auto slot = [&](int s, int, int n_tasks, int &h, int &task) {
    h = blockIdx.x;
    task = blockIdx.y + s * gridDim.y;
    return task < n_tasks;
  };
  if (S > 1)
    attention_round<HD, false, true>(a, pos, slot, qs[wave], kn[wave], part);
  else
    attention_round<HD, false, false>(a, pos, slot, qs[wave], kn[wave], part);
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

// Plain streaming copy (the calibration copy of llrs_device_copy).
__global__ __launch_bounds__(256) void copy_kernel(uint4 *__restrict__ dst,
                                                   const uint4 *__restrict__ src, size_t n16) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// ------------------------------------------------------------------ launchers

int launch_embed(const llrs_tensor *emb, const uint32_t *tok_by_pos, const int *pos, int max_seq,
                 float *out, unsigned *epoch, hipStream_t s, unsigned *clear, int nclear) {
  int H = (int)emb->cols;
  int n = H > nclear ? H : nclear;
  hipLaunchKernelGGL(embed_kernel, dim3((n + 255) / 256), dim3(256), 0, s, emb->dev, emb->type,
                     emb->row_bytes, H, (uint32_t)emb->rows, tok_by_pos, pos, max_seq, out, epoch,
                     clear, nclear);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_rmsnorm(const float *in, const float *w, float *out, int n, float eps, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, in, w, out, n, eps);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

long attention_part_stride(int hd) { return 2L * hd + 2; }

size_t attention_scratch_words(int nh, int hd, int max_seq) {
  const int chunks = attention_chunks(max_seq);
  return (size_t)nh * (size_t)chunks * (size_t)attention_part_stride(hd);
}

int attention_chunks(int max_seq) { return (max_seq + kChunk - 1) / kChunk; }

int launch_attention(const AttnArgs &args, hipStream_t s) {
  const int hd = args.hd;
  if (args.nkv <= 0 || args.nh % args.nkv || !(hd == 16 || hd == 32 || hd == 64 || hd == 128))
    return set_error(LLRS_E_UNSUPPORTED, "attention geometry %d/%d heads, head_dim %d is not supported",
                     args.nh, args.nkv, hd);
  if (args.part_stride != attention_part_stride(hd) || args.max_chunks != attention_chunks(args.max_seq))
    return set_error(LLRS_E_INVALID, "attention scratch geometry does not match head_dim %d, context %d",
                     hd, args.max_seq);
  const dim3 grid((unsigned)args.nh, (unsigned)attention_blocks(args.max_chunks)), block(64 * kTaskItems);
  switch (hd) {
    case 16: hipLaunchKernelGGL(attention_kernel<16>, grid, block, 0, s, args); break;
    case 32: hipLaunchKernelGGL(attention_kernel<32>, grid, block, 0, s, args); break;
    case 64: hipLaunchKernelGGL(attention_kernel<64>, grid, block, 0, s, args); break;
    default: hipLaunchKernelGGL(attention_kernel<128>, grid, block, 0, s, args); break;
  }
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

int launch_copy(void *dst, const void *src, size_t nbytes, int cu_count, hipStream_t s) {
  const size_t n16 = nbytes / 16;
  size_t grid = (n16 + 255) / 256;
  const size_t cap = (size_t)cu_count * 8;
  if (grid > cap) grid = cap;
  if (grid == 0) return LLRS_OK;
  hipLaunchKernelGGL(copy_kernel, dim3((unsigned)grid), dim3(256), 0, s, static_cast<uint4 *>(dst),
                     static_cast<const uint4 *>(src), n16);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

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
