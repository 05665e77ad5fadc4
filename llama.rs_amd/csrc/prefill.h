// Multi-token prefill (CausalModel::prefill, src/architecture.rs:60-77): the
// prompt's tokens go through each layer together, the weight matrices as
// MFMA dequant-GEMMs.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace llrs {

typedef _Float16 f16;

// C[t][n] (=|+=) sum_k A[t][k] * W[n][k] (+ bias[n]) for t < T, n < rows(W).
struct PrefillGemmArgs {
  const f16 *a, *a_lo;  // [T][lda] activations as hi + lo f16 pairs
  int lda;
  const uint8_t *w;  // native GGUF rows
  uint32_t type;
  long row_bytes;
  int n, k;       // rows and cols of W
  float *c;       // [T][ldc]
  int ldc;
  const float *bias;  // [n] or null; ignored when accumulating
  int t;
  int accumulate;
  int ksplit;  // set by launch_prefill_gemm: K ranges whose partial tiles go to `part`
  // Split-K scratch: each K range writes its partial products here ([ksplit][t][n]),
  // and a reduction adds them to C in split order, so results do not depend
  // on the order the workgroups finish in.
  float *part;
  size_t part_cap;  // floats
  // Q4_K weights: when set, the per-sub-block sums of the activations
  // (launch_xsum_f16 of a/a_lo, [T][ldxs], ldxs >= k/32 + 56) and the product
  // runs on the Q4_K codes as exact integers (prefill_codes_enabled()).
  const f16 *xs, *xs_lo;
  int ldxs;
  // Dual product (gate and up, Q4_K on its codes): w are the gate rows, w2 the
  // up rows (same k, type and row bytes), n = 2 * dual_rows virtual rows
  // (each 128-row tile holds 64 gate rows and the same 64 up rows), and the
  // output is silu(gate) * up as f16 pairs h/hl [t][ldh] instead of c; with
  // xso set, also its 32-column sums (for a Q4_K ffn_down).
  const uint8_t *w2;
  int dual_rows;
  f16 *h, *hl;
  int ldh;
  f16 *xso, *xso_lo;
  int ldxso;
  // Segmented product (Q4_K on its codes, e.g. q, k and v of one input): rows
  // [seg_base[i], seg_base[i + 1]) of the n come from seg_w[i] and go to
  // seg_c[i] (row stride seg_ldc[i], bias seg_bias[i] or null); every
  // boundary but the last a multiple of 128.  nseg = 0: w, c, ldc and bias.
  int nseg;
  const uint8_t *seg_w[3];
  float *seg_c[3];
  int seg_ldc[3];
  const float *seg_bias[3];
  int seg_base[4];
};

// Floats of split-K scratch a prefill GEMM may need on this device: one
// 128 x 128 tile per workgroup slot.
size_t prefill_split_scratch_floats();
int launch_prefill_gemm(const PrefillGemmArgs &g, hipStream_t s);
// Whether Q4_K and Q6_K products run on their integer codes (the default;
// LLRS_PREFILL_CODES=f32 or the four-wave GEMM, LLRS_PREFILL_GEMM=4, select
// the f32-weight product).  Read at every call.
bool prefill_codes_enabled();
// xs + xs_lo [t][s] = sum_{j<32} (a + a_lo)[t][32 s + j] as f16 pairs, s < k/32, t < T.
int launch_xsum_f16(const f16 *a, const f16 *a_lo, int lda, int k, int T, f16 *xs, f16 *xs_lo, int ldxs,
                    hipStream_t s);

// x[t][:] = embedding row of tok[t] (bit-exact dequant), t < T.
int launch_embed_rows(const llrs_tensor *emb, const uint32_t *tok, int T, float *x, hipStream_t s);
// out + out_lo [t][:] = x[t] * (1/sqrt(mean(x[t]^2) + eps) * w) as f16 pairs;
// with xs set, also their 32-column sums as launch_xsum_f16 gives them (up
// to f32 summation order).
int launch_rmsnorm_rows_f16(const float *x, const float *w, f16 *out, f16 *out_lo, int T, int H,
                            float eps, hipStream_t s, f16 *xs = nullptr, f16 *xs_lo = nullptr, int ldxs = 0);
// Split-half RoPE of q (in place) and k at positions start + t, and the K/V
// cache rows of those positions.
int launch_rope_append(float *q, const float *k, const float *v, const float *rope, int T, int start,
                       int nh, int nkv, int hd, float *k_cache, float *v_cache, hipStream_t s);
// Scratch for the f16 attention: one layer's K and V rows as hi/lo planes in
// blocks of 16 positions (positions x kvw halves a plane; positions a
// multiple of 16 and at least the rows attended, rounded up to 16).
struct PrefillKvF16 {
  f16 *kh, *kl, *vh, *vl;
  int positions, kvw;
};
// Causal GQA attention of the T query rows (positions start + t) over the
// cache, out + out_lo [T][nh*hd] (f16 pairs).  With kvf (head_dim >= 32 and
// unless LLRS_PREFILL_ATTN=f32) the products run as f16 hi/lo MFMAs on a copy
// of the cache rows in kvf; otherwise as f32 MFMAs on the cache.
int launch_attention_rows(const float *q, const float *k_cache, const float *v_cache, int T,
                          int start, int nh, int nkv, int hd, float scale, f16 *out, f16 *out_lo,
                          hipStream_t s, const PrefillKvF16 *kvf = nullptr);
// out + out_lo [i] = silu(g[i]) * u[i] as f16 pairs, i < n (rows of `cols`);
// with xs set, also their 32-column sums per row.
int launch_swiglu_f16(const float *g, const float *u, f16 *out, f16 *out_lo, size_t n, int cols, hipStream_t s,
                      f16 *xs = nullptr, f16 *xs_lo = nullptr, int ldxs = 0);
int launch_set_pos(int *pos, int value, hipStream_t s);

}  // namespace llrs
