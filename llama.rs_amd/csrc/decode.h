// Launchers for the per-token decode kernels (decode.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace llrs {

// Decode attention items.
constexpr int kChunk = 32;  // positions per attention sub-chunk (one wave)
// Sub-chunks per attention item at position pos for nh query heads: one
// while the items of all heads fit kItemSlots (the persistent kernel's 256
// workgroups x 8 waves on this part, so every wave takes at most one item),
// then as many as bring them back within it: an item's sub-chunks load one
// after another, but a wave's items do too, with a merge wait each.
constexpr int kItemSlots = 2048;
__host__ __device__ inline int attention_span(int pos, int nh) {
  const long n = (long)(pos / kChunk + 1) * (nh > 0 ? nh : 1);
  return (int)((n + kItemSlots - 1) / kItemSlots);
}
// Attention tasks: T consecutive items of one head, one per wave of a
// workgroup of kTaskItems waves, whose partials meet in LDS; the head's tasks
// then meet through the scratch partials, folded by the head's last task.  T
// (1, 2, 4 or 8): kTaskItems while a head has at most that many items (its
// task alone writes the output), else the smallest that leaves the fold at
// most `fold` partials (AttnArgs::fold_max): larger tasks gather more items
// on one CU, whose loads then queue behind each other.
constexpr int kTaskItems = 8;
__host__ __device__ inline int attention_task_items(int n_items, int fold) {
  if (n_items <= kTaskItems) return kTaskItems;
  int t = 1;
  while (t < kTaskItems && (n_items + t - 1) / t - 1 > fold) t *= 2;
  return t;
}
// The default fold bound: the partials one load round of the fold reads
// (32 / VW, VW = 2 V floats per lane at head_dim 128, else 1).
inline int attention_fold_default(int hd) { return hd >= 128 ? 16 : 32; }
// Workgroups per head of the attention kernel: kTaskItems items each.
__host__ __device__ inline int attention_blocks(int max_chunks) { return (max_chunks + kTaskItems - 1) / kTaskItems; }
// From this position the persistent kernel issues an attention item's key
// rows before the phase barrier and its value rows after it; at earlier
// positions it issues both before the barrier.
constexpr int kSplitLoadsFrom = 1024;

// Fused RoPE + KV append + GQA attention of one layer.
struct AttnArgs {
  const float *q, *k, *v;  // projections of the current token (q, k before RoPE)
  const float *rope;       // [max_seq][hd]: cos of the half, then sin of the half
  const int *pos;
  float *k_cache, *v_cache;  // this layer's [max_seq][kv_width]
  float *out;                // [nh * hd]
  // Task partials per head, attention_scratch_words(nh, hd, max_seq) words:
  // each value with the tag of the (step, layer) that wrote it in the high
  // half.
  unsigned long long *scratch;
  const unsigned *epoch;     // step counter, advanced by the embedding kernel
  unsigned *err;             // set when a merge gave up waiting for a partial
  int layer, nlayers;        // tag = *epoch * nlayers + layer
  unsigned tag;              // filled in on the device
  int nh, nkv, hd, max_seq;
  int max_chunks;            // attention_chunks(max_seq)
  long part_stride;          // attention_part_stride(hd): words per (head, task) partial
  int fold_max;              // attention_task_items' fold bound
  float scale;               // 1/sqrt(hd)
};

// Also advances *epoch (the attention partials' tag) and zeroes
// clear[0 .. nclear) (the persistent kernel's barrier counters).
int launch_embed(const llrs_tensor *emb, const uint32_t *tok_by_pos, const int *pos, int max_seq,
                 float *out, unsigned *epoch, hipStream_t s, unsigned *clear = nullptr,
                 int nclear = 0);
int launch_rmsnorm(const float *in, const float *w, float *out, int n, float eps, hipStream_t s);
long attention_part_stride(int hd);
size_t attention_scratch_words(int nh, int hd, int max_seq);
int attention_chunks(int max_seq);
int launch_attention(const AttnArgs &args, hipStream_t s);
int launch_silu_mul(const float *g, const float *u, float *out, int n, hipStream_t s);
int launch_argmax(const float *logits, int n, int *pos, int max_seq, uint32_t *tok_by_pos,
                  uint32_t *next_token, int advance, hipStream_t s);
int launch_advance(int *pos, int max_seq, hipStream_t s);
// dst = src over nbytes (16-byte aligned, a multiple of 16).
int launch_copy(void *dst, const void *src, size_t nbytes, int cu_count, hipStream_t s);

}  // namespace llrs
