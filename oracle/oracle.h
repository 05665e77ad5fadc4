/*
 * CPU ORACLE -- test infrastructure only.
 *
 * A plain-C restatement of the reference's (bernkastel5/llama.rs) scalar CPU
 * path, used as the parity checker for the HIP product path and as the CPU
 * baseline in bench.py.  Nothing in the product library links or calls this
 * code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load liboracle.so.
 *
 * Arithmetic rules (to follow the Rust scalar backend bit-for-bit on x86-64):
 *   - built with -ffp-contract=off, no fast-math: Rust never contracts a*b+c;
 *   - sequential left-to-right f32 accumulation in the reference loop orders;
 *   - Rust's f32 `.sum()` starts from -0.0 (only the sign of an all-zero sum
 *     differs from +0.0), explicit `let mut sum = 0.0` loops start from +0.0;
 *   - libm: powf / sinf / cosf / expf / sqrtf from glibc, as the Rust binary
 *     calls on Linux;
 *   - f16/bf16 -> f32 are exact IEEE widenings (the `half` crate).
 *
 * Pinning status of each part is stated where it is defined (oracle.c,
 * oracle_model.c) and in the tests that pin it.
 */
#ifndef LLRS_ORACLE_H
#define LLRS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids accepted by QuantType::from_ggml_type (src/quant.rs:27-44). */
enum {
  OQ_F32 = 0, OQ_F16 = 1, OQ_Q4_0 = 2, OQ_Q4_1 = 3, OQ_Q5_0 = 6, OQ_Q5_1 = 7,
  OQ_Q8_0 = 8, OQ_Q4_K = 12, OQ_Q5_K = 13, OQ_Q6_K = 14, OQ_BF16 = 30
};

enum { OQ_KERNEL_SCALAR = 0, OQ_KERNEL_AVX2 = 1 };

/* QuantType::block_size / type_size (src/quant.rs:46-67); 0 for unknown ids. */
int oq_block_size(uint32_t ggml_type);
int oq_type_size(uint32_t ggml_type);
/* cols / block * type_size (src/quant.rs:171-173); 0 if cols is not a block multiple. */
size_t oq_row_bytes(uint32_t ggml_type, size_t cols);

float oq_f16_to_f32(uint16_t h);
float oq_bf16_to_f32(uint16_t h);

/* value_at (src/quant.rs:349-456). */
float oq_value_at(const uint8_t *row, uint32_t ggml_type, size_t col);
/* row_into (src/quant.rs:261-272): dequantize one row of `cols` values. */
void oq_dequant_row(const uint8_t *row, uint32_t ggml_type, size_t cols, float *out);
/* dot_row_scalar (src/quant.rs:458-648). */
float oq_dot_row_scalar(const uint8_t *row, uint32_t ggml_type, const float *x, size_t cols);
/* dot_row_avx2 (src/simd.rs:283-311); returns the scalar result if the CPU lacks AVX2+FMA. */
float oq_dot_row_avx2(const uint8_t *row, uint32_t ggml_type, const float *x, size_t cols);
int oq_cpu_has_avx2_fma(void);

/*
 * CpuBackend::matvec (src/backend.rs:143-162): rows run in parallel iff
 * threads > 1 && rows >= 2*threads && rows*cols >= parallel_threshold.
 * threads == 0 means all logical CPUs (src/backend.rs:99-106).
 * Returns 0, or -1 on a shape error.
 */
int oq_matvec(const uint8_t *weight, uint32_t ggml_type, size_t rows, size_t cols,
              const float *x, float *y, int kernel, int threads, size_t parallel_threshold);

/* ---------------------------- model (oracle_model.c) ---------------------------- */

typedef struct oq_model oq_model;
typedef struct oq_state oq_state;

/*
 * GgufLoader::load (src/loader.rs:233-399) with LoadQuantization::None: the
 * GGUF must already hold quantized (or float) tensors, which are used verbatim
 * (src/loader.rs:411-418).  Returns NULL on error; oq_last_error() says why.
 */
oq_model *oq_model_load_gguf(const char *path, int kernel, int threads);
void oq_model_free(oq_model *m);
const char *oq_last_error(void);

/* LlamaConfig fields (src/config.rs:18-55). */
typedef struct {
  size_t hidden_size, intermediate_size, num_attention_heads, num_key_value_heads,
      num_hidden_layers, vocab_size, max_position_embeddings, head_dim, kv_width;
  float rms_norm_eps, rope_theta;
  int tie_word_embeddings;
} oq_config;
void oq_model_config(const oq_model *m, oq_config *out);

/* KVCache::new + InferenceBuffers::new (src/cache.rs:13-36, 80-101). */
oq_state *oq_state_new(const oq_model *m, size_t max_seq_len);
void oq_state_free(oq_state *s);

/* forward_impl (src/model.rs:135-271).  logits_mode: 0 Skip, 1 Compute. */
int oq_forward_token(const oq_model *m, oq_state *s, uint32_t token, size_t pos, int logits_mode);
/* CausalModel::prefill default loop (src/architecture.rs:60-77). */
int oq_prefill(const oq_model *m, oq_state *s, const uint32_t *tokens, size_t n, size_t start_pos);
/* argmax_current_logits (src/engine.rs:233-241): total_cmp order, last index on ties. */
uint32_t oq_argmax(const float *logits, size_t n);
/* benchmark_tokens decode loop (src/engine.rs:205-216): n_steps x (argmax, forward).
 * out_tokens[i] is the token fed at position start_pos + i. */
int oq_decode_greedy(const oq_model *m, oq_state *s, size_t start_pos, size_t n_steps,
                     uint32_t *out_tokens);

/* GgufFile::open + tensor + to_vec_f32 (src/gguf.rs:78-215, src/quant.rs:274-283):
 * dequantized values of one tensor; version, rows and cols reported.  Returns
 * 0, or -1 with oq_last_error() set.  out may be NULL to query the shape. */
int oq_gguf_read_f32(const char *path, const char *name, uint32_t *version, size_t *rows,
                     size_t *cols, float *out, size_t capacity);

/* sample_current_logits (src/engine.rs:253-325) with the uniform draw given:
 * repetition penalty for the tokens in recent[0 .. n_recent), temperature,
 * the descending total_cmp sort (ties: lower index first), top-k, softmax and
 * top-p in sequential f32 sums, then random = uniform * kept_sum decremented
 * by each kept probability until <= 0. */
uint32_t oq_sample(const float *logits, size_t n, float temperature, size_t top_k, float top_p,
                   float repetition_penalty, const uint32_t *recent, size_t n_recent, float uniform);

/* Read access to the state, for tests. */
const float *oq_state_logits(const oq_state *s);
const float *oq_state_residual(const oq_state *s);
const float *oq_state_k_cache(const oq_state *s, size_t layer);
const float *oq_state_v_cache(const oq_state *s, size_t layer);

/* Write access, for tests and the bench's CPU baseline: seeds a state with
 * rows computed elsewhere (the GPU's prefilled cache), so that the oracle can
 * check steps at depths whose own prefill it could not afford.  what: 0 = K
 * rows of `layer`, 1 = V rows of `layer` (n floats from position 0), 2 = the
 * logits (n = vocab).  Returns 0, or -1 on a bad layer / length. */
int oq_state_load(oq_state *s, int what, size_t layer, const float *src, size_t n);

#ifdef __cplusplus
}
#endif
#endif
