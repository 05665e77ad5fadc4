// Launchers for the per-token decode kernels (decode.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace llrs {

int launch_embed(const llrs_tensor *emb, const uint32_t *tok_by_pos, const int *pos, float *out,
                 hipStream_t s);
int launch_rmsnorm(const float *in, const float *w, float *out, int n, float eps, hipStream_t s);
int launch_rope_kv(float *q, const float *k, const float *v, const float *rope, const int *pos,
                   float *kc, float *vc, int nh, int nkv, int hd, hipStream_t s);
int launch_attention(const float *q, const float *kc, const float *vc, const int *pos,
                     float *scores, float *out, int nh, int nkv, int hd, int max_seq,
                     hipStream_t s);
int launch_silu_mul(const float *g, const float *u, float *out, int n, hipStream_t s);
int launch_argmax(const float *logits, int n, int *pos, uint32_t *tok_by_pos, uint32_t *next_token,
                  int advance, hipStream_t s);
int launch_advance(int *pos, hipStream_t s);

}  // namespace llrs
