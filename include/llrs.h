/*
 * llrs.h -- C ABI of the MI355X (gfx950) HIP backend for llama.rs's batch-1
 * decode path.
 *
 * Conventions: every function returning int returns LLRS_OK (0) on success or
 * a negative LLRS_E_* code; llrs_last_error() then holds a message for the
 * calling thread.  No C++ exception or unwinding crosses this boundary (the
 * reference builds with panic = "abort", Cargo.toml:20).  All pointers are
 * plain host pointers unless a name ends in _dev.  Handles are not
 * thread-safe: one thread drives a backend at a time, as the reference's
 * engine drives its model (src/engine.rs:36-50).
 */
#ifndef LLRS_H
#define LLRS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLRS_OK 0
#define LLRS_E_INVALID -1   /* bad argument, shape or length (anyhow::ensure! in the reference) */
#define LLRS_E_UNSUPPORTED -2 /* unknown GGML type, architecture or option */
#define LLRS_E_HIP -3       /* HIP runtime failure */
#define LLRS_E_OOM -4       /* device or host allocation failure */
#define LLRS_E_IO -5        /* file open / read / write failure */
#define LLRS_E_FORMAT -6    /* malformed GGUF file */

/* GGML tensor type ids: QuantType::from_ggml_type (src/quant.rs:27-44). */
enum llrs_ggml_type {
  LLRS_F32 = 0, LLRS_F16 = 1, LLRS_Q4_0 = 2, LLRS_Q4_1 = 3, LLRS_Q5_0 = 6, LLRS_Q5_1 = 7,
  LLRS_Q8_0 = 8, LLRS_Q4_K = 12, LLRS_Q5_K = 13, LLRS_Q6_K = 14, LLRS_BF16 = 30
};

/* LogitsMode (src/architecture.rs:35-39). */
enum llrs_logits_mode { LLRS_LOGITS_SKIP = 0, LLRS_LOGITS_COMPUTE = 1 };

/* LoadQuantization (src/loader.rs:16-25). */
enum llrs_quantization { LLRS_QUANT_NONE = 0, LLRS_QUANT_Q4K = 1, LLRS_QUANT_Q4KM = 2 };
/* Checkpoint formats ModelLoader::load recognises (src/loader.rs:44-77). */
enum llrs_model_format { LLRS_FORMAT_GGUF = 1, LLRS_FORMAT_SAFETENSORS = 2 };

typedef struct llrs_backend llrs_backend;
typedef struct llrs_tensor llrs_tensor;
typedef struct llrs_model llrs_model;
typedef struct llrs_kv llrs_kv;

/* Thread-local message for the last failed call on this thread ("" if none). */
const char *llrs_last_error(void);

/* ------------------------------------------------------------------------ */
/* Backend: replaces CpuBackend::new / KernelBackend::{name, threads}        */
/* (src/backend.rs:48-65, 67-73, 97-121, 134-141).                           */
/* ------------------------------------------------------------------------ */
typedef struct {
  int device;      /* HIP device ordinal */
  uint32_t flags;  /* reserved, must be 0 */
} llrs_backend_config;

int llrs_backend_create(const llrs_backend_config *cfg, llrs_backend **out);
/* Drop (src/backend.rs's Arc<dyn KernelBackend> going out of scope): releases
 * the caller's handle.  Every tensor, model and KV cache made from the
 * backend holds a counted reference to it, as Qwen2Model holds an Arc of its
 * backend (src/model.rs:117; src/loader.rs:99, 242), so the device state
 * lives until the last of them is freed, in any order. */
void llrs_backend_destroy(llrs_backend *b);
/* KernelBackend::name (src/backend.rs:70): "hip-gfx950". */
const char *llrs_backend_name(const llrs_backend *b);
/* KernelBackend::threads (src/backend.rs:71): the device's compute-unit count. */
size_t llrs_backend_threads(const llrs_backend *b);
/* Blocks the host until all work queued by this backend has finished. */
int llrs_backend_synchronize(llrs_backend *b);

/* ------------------------------------------------------------------------ */
/* Tensors: QuantTensor::from_owned / from_mmap (src/quant.rs:114-157).      */
/* The native GGUF block bytes are copied once to HBM, block layout intact.  */
/* ------------------------------------------------------------------------ */
/* Validates the byte length exactly as QuantTensor::from_data
 * (src/quant.rs:132-157): cols % block_size == 0 and
 * nbytes == rows*cols/block_size*type_size.  rows == 0 is allowed (empty). */
int llrs_tensor_upload(llrs_backend *b, const void *bytes, size_t nbytes, uint32_t ggml_type,
                       size_t rows, size_t cols, llrs_tensor **out);
void llrs_tensor_free(llrs_tensor *t);
int llrs_tensor_info(const llrs_tensor *t, uint32_t *ggml_type, size_t *rows, size_t *cols,
                     size_t *nbytes);
/* Copies the tensor's native bytes back to the host (nbytes must match). */
int llrs_tensor_download(const llrs_tensor *t, void *out, size_t nbytes);

/* KernelBackend::matvec (src/backend.rs:72, 143-162) with validate_matvec's
 * checks (src/quant.rs:303-318): nx == cols, ny == rows, tensor is 2-D.
 * Host input and output; synchronous; y is fully overwritten. */
int llrs_matvec(llrs_backend *b, const llrs_tensor *w, const float *x, size_t nx, float *y,
                size_t ny);
/* The same on device pointers, enqueued on the backend's stream (asynchronous). */
int llrs_matvec_dev(llrs_backend *b, const llrs_tensor *w, const float *x_dev, float *y_dev);
/* QuantTensor::row_into (src/quant.rs:261-272): dequantize row `row` into out[n]
 * (n must equal cols); the bit-exact test hook for value_at. */
int llrs_dequant_row(llrs_backend *b, const llrs_tensor *w, size_t row, float *out, size_t n);

/* Device scratch helpers for the _dev entry points and benchmarks. */
int llrs_device_alloc(llrs_backend *b, size_t nbytes, void **out_dev);
int llrs_device_free(llrs_backend *b, void *dev);
int llrs_copy_h2d(llrs_backend *b, void *dst_dev, const void *src, size_t nbytes);
int llrs_copy_d2h(llrs_backend *b, void *dst, const void *src_dev, size_t nbytes);
/* Device-to-device copy by a plain streaming kernel (16-byte aligned
 * pointers, nbytes a multiple of 16); synchronous.  No counterpart in the
 * reference: it is the known-size copy against which HBM traffic counters of
 * the other kernels are calibrated. */
int llrs_device_copy(llrs_backend *b, void *dst_dev, const void *src_dev, size_t nbytes);

/* Host-side quantizers, QuantTensor::quantize_* (src/quant.rs:187-259,
 * 650-967) including their fallbacks (Q4_K -> Q5_0 -> F32, Q6_K -> Q8_0).
 * ggml_type selects the entry point (LLRS_Q4_K, LLRS_Q5_0, LLRS_Q8_0,
 * LLRS_Q6_K); *out_type receives the type actually produced.  If out is NULL
 * the required size is returned in *out_nbytes. */
int llrs_quantize(uint32_t ggml_type, const float *values, size_t rows, size_t cols, void *out,
                  size_t out_capacity, size_t *out_nbytes, uint32_t *out_type);

/* GgufFile::open + GgufFile::tensor (src/gguf.rs:78-215): reads one tensor of
 * a GGUF v2/v3 file with every header/range check of the reader.  Shape is
 * reported as the reference does ([rows, cols] = [dims[1], dims[0]]; rows = 1
 * for a 1-D tensor).  If out is NULL only the metadata is returned. */
int llrs_gguf_read_tensor(const char *path, const char *name, uint32_t *version,
                          uint32_t *ggml_type, size_t *rows, size_t *cols, void *out,
                          size_t out_capacity, size_t *nbytes);

/* ------------------------------------------------------------------------ */
/* Model: ModelLoader::load_dynamic -> GgufLoader::load (src/loader.rs:37-42, */
/* 233-399), CausalModel (src/architecture.rs:42-78).                        */
/* ------------------------------------------------------------------------ */
/* LlamaConfig (src/config.rs:18-55) as loaded. */
typedef struct {
  size_t hidden_size, intermediate_size, num_attention_heads, num_key_value_heads,
      num_hidden_layers, vocab_size, max_position_embeddings, head_dim, kv_width;
  float rms_norm_eps, rope_theta;
  int tie_word_embeddings;
} llrs_model_config;

/* Loads a GGUF v2/v3 Qwen2 file: metadata -> config, tensors uploaded to HBM
 * verbatim (quantization = LLRS_QUANT_NONE) or quantized at load time with
 * the reference's q4k / q4km recipe when the file holds F32/F16/BF16
 * matrices (src/loader.rs:406-447). */
int llrs_model_load_gguf(llrs_backend *b, const char *path, int quantization, llrs_model **out);
/* SafetensorsLoader::load (src/loader.rs:80-228): a Hugging Face Qwen2
 * checkpoint directory (config.json + model.safetensors, or the shards of
 * model.safetensors.index.json).  F32/F16/BF16 matrices are uploaded as they
 * are (quantization = LLRS_QUANT_NONE) or converted and quantized on the GPU
 * with the q4k / q4km recipe (maybe_quantize, src/loader.rs:406-447); norms
 * and biases become f32 (missing Q/K/V biases: zeros); the LM head is
 * lm_head.weight when present, else the embedding matrix. */
int llrs_model_load_safetensors(llrs_backend *b, const char *model_dir, int quantization,
                                llrs_model **out);
/* ModelLoader::load (src/loader.rs:44-77): a .gguf file, a .safetensors file
 * (its directory is loaded), or a directory holding model.safetensors /
 * model.safetensors.index.json or exactly one .gguf file. */
int llrs_model_load(llrs_backend *b, const char *path, int quantization, llrs_model **out);
/* The format llrs_model_load picks for path (LLRS_FORMAT_*) and what it opens
 * (the GGUF file or the checkpoint directory), without a GPU.  resolved may
 * be NULL. */
int llrs_model_format(const char *path, int *format, char *resolved, size_t capacity);
/* LlamaConfig::from_json + validate (src/config.rs:17-90) on a config.json
 * whose model_type is "qwen2" (src/loader.rs:85-97), without a GPU. */
int llrs_hf_config_read(const char *config_json_path, llrs_model_config *out);
/* SafetensorStore::open + tensor (src/loader.rs:543-645) without a GPU: one
 * F32/F16/BF16 tensor of a checkpoint directory, with every check of the
 * safetensors header.  *ggml_type is LLRS_F32, LLRS_F16 or LLRS_BF16; shape
 * receives *ndim (1 or 2) sizes, outermost first.  If out is NULL only the
 * metadata is returned. */
int llrs_safetensors_read_tensor(const char *model_dir, const char *name, uint32_t *ggml_type,
                                 size_t *shape, size_t *ndim, void *out, size_t out_capacity,
                                 size_t *nbytes);
/* Releases the caller's handle; KV caches made from the model keep it (and
 * its backend) alive until they are freed. */
void llrs_model_free(llrs_model *m);
int llrs_model_config_get(const llrs_model *m, llrs_model_config *out);
/* Bytes of weights the decode step streams per token (all matrices incl.
 * the LM head, plus one embedding row, norms and biases). */
size_t llrs_model_weight_bytes(const llrs_model *m);

/* Synthetic Qwen2 models (random-init from a seed, quantized with a recipe). */
typedef struct {
  size_t hidden_size, intermediate_size, num_attention_heads, num_key_value_heads,
      num_hidden_layers, vocab_size, max_position_embeddings;
  float rms_norm_eps, rope_theta;
  int tie_word_embeddings;
  int recipe;       /* LLRS_QUANT_Q4KM, LLRS_QUANT_Q4K, or LLRS_QUANT_NONE (F32) */
  uint64_t seed;
  float weight_std; /* N(0, weight_std) weights and biases; norm gains 1 + N(0, weight_std) */
  int threads;      /* host threads for generation; 0 = all */
} llrs_synth_config;
/* Writes a GGUF v3 file with the synthetic model (pre-quantized tensors). */
int llrs_synth_write_gguf(const llrs_synth_config *cfg, const char *path);
/* Builds the same model directly in HBM without a file: generated and
 * quantized on the GPU with the same functions, so its tensors hold exactly
 * the bytes llrs_synth_write_gguf writes for the same config. */
int llrs_model_synthetic(llrs_backend *b, const llrs_synth_config *cfg, llrs_model **out);
/* Writes a loaded model back to a GGUF v3 file: matrices in their native
 * block bytes, norms and biases as F32 (as loaded). */
int llrs_model_export_gguf(const llrs_model *m, const char *path);

/* KVCache::new + InferenceBuffers::new (src/cache.rs:13-36, 80-101): a
 * device-resident f32 KV cache, layout [layer][pos][kv_width] as the
 * reference's, plus device activation buffers.  Fails if max_seq_len is 0 or
 * exceeds max_position_embeddings (src/cache.rs:14-19). */
int llrs_kv_create(llrs_model *m, size_t max_seq_len, llrs_kv **out);
/* Frees the cache and releases its reference to the model. */
void llrs_kv_free(llrs_kv *kv);
/* KVCache::reset (src/cache.rs:55-57): the rows are kept (positions are
 * overwritten before they are read); the device's wait flags (below) are
 * cleared. */
int llrs_kv_reset(llrs_kv *kv);
/* Every device-side wait of a decode step is bounded (~20 ms): a barrier of
 * the persistent kernel, or an attention merge waiting for partials.  On
 * expiry the kernel sets a flag and finishes; the next call that checks
 * (forward_token, prefill, decode_greedy: every 64 steps and at the end)
 * returns LLRS_E_HIP and clears the flag, so later calls run normally (the
 * steps since the last check are untrustworthy: prefill the cache again).
 * This hook sets a flag from the host (which: 0 = barrier, 1 = attention
 * merge) so that tests can exercise the reporting path; no counterpart in
 * the reference. */
int llrs_kv_debug_set_wait_flag(llrs_kv *kv, int which);
/* Measurement only, no counterpart in the reference: runs `blocks`
 * workgroups of an LDS access-pattern probe for `iters` iterations and
 * waits for them (mode 0: conflict-free 32-bit reads, 1: 64-bit reads, 2:
 * 128-bit reads, 3: 32-bit reads with every lane in one bank, 4:
 * conflict-free 128-bit writes, 5 and 6: 128-bit MFMA operand reads from
 * rows 144 and 176 bytes apart, 7: 128-bit staging writes to rows 144 bytes
 * apart, 8 and 9: 128-bit reads of 256-byte runs at unaligned and aligned
 * offsets, 10 and 11: chunk-major staging writes with and without a row
 * swizzle), so that the LDS counters can be read against a known bank
 * pattern (bench.py --lds-probe). */
int llrs_debug_lds_probe(llrs_backend *b, int mode, int blocks, int iters);
/* Which implementation runs this state's decode steps: 1 = one persistent
 * launch for all layers (chosen at llrs_kv_create when the model's weight
 * types and head_dim have an instantiation and LLRS_NO_PERSISTENT is unset),
 * 0 = one launch per phase.  Both compute the same values.  No counterpart
 * in the reference (its decode step has one implementation). */
int llrs_kv_decode_path(const llrs_kv *kv);

/* CausalModel::forward_token (src/architecture.rs:47-54; src/model.rs:135-271).
 * Fails if token >= vocab or pos >= max_seq_len (src/model.rs:145-153). */
int llrs_forward_token(llrs_model *m, llrs_kv *kv, uint32_t token, size_t pos, int logits_mode);
/* CausalModel::prefill (src/architecture.rs:60-77): logits only for the last token. */
int llrs_prefill(llrs_model *m, llrs_kv *kv, const uint32_t *tokens, size_t n, size_t start_pos);
/* The decode loop of InferenceEngine::benchmark_tokens (src/engine.rs:205-216):
 * n_steps x { token = argmax(current logits); forward_token(token, start_pos+i) },
 * replayed from one captured hipGraph with token and position kept on the
 * device.  out_tokens[i] receives the token fed at start_pos + i. */
int llrs_decode_greedy(llrs_model *m, llrs_kv *kv, size_t start_pos, size_t n_steps,
                       uint32_t *out_tokens);
/* argmax_current_logits (src/engine.rs:233-241) of the current device logits. */
int llrs_argmax(llrs_kv *kv, uint32_t *out_token);

/* EngineOptions' sampling fields (src/engine.rs:14-31). */
typedef struct llrs_sampling {
  float temperature;        /* 0: greedy (the first candidate of the sorted logits) */
  float top_p;              /* in (0, 1] */
  uint32_t top_k;           /* 0: every token */
  float repetition_penalty; /* > 0; 1: off */
} llrs_sampling;
/* InferenceEngine::sample_current_logits (src/engine.rs:253-325) on the
 * device over the current logits: the repetition penalty for the tokens in
 * recent[0 .. n_recent) (the repeat window, at most 65536), the temperature,
 * the descending sort, top-k, softmax, the top-p cutoff and the draw.  The
 * uniform number in [0, 1) is the caller's (the reference draws
 * rand::thread_rng().gen::<f32>()).  Options are validated as
 * validate_sampling (src/engine.rs:327-338). */
int llrs_sample(llrs_kv *kv, const llrs_sampling *opts, const uint32_t *recent, size_t n_recent,
                float uniform, uint32_t *out_token);
/* llrs_sample without any allocation, on any call: no counterpart in the
 * reference.  For callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc).  It is not for code under stream
 * capture: like llrs_sample it copies the window from host memory,
 * synchronises the stream and reads the token back.  Its
 * scratch (sort keys and indices, the repeat window, the radix sort's
 * temporary storage: 8.3 MB) is one file-scope device array per GPU, held
 * until the process ends, so the vocabulary is limited to 262,144 tokens and
 * the window to 65,536 (larger inputs fail with LLRS_E_INVALID).  Every call
 * on one GPU shares that array: calls that overlap on one GPU (two threads,
 * two streams) race.  Same arguments, validation and results as llrs_sample. */
int llrs_sample_noalloc(llrs_kv *kv, const llrs_sampling *opts, const uint32_t *recent,
                        size_t n_recent, float uniform, uint32_t *out_token);
/* InferenceEngine::generate_with_metrics' token loop (src/engine.rs:115-186)
 * on token ids (the tokenizer stays with the caller): reset the cache, seed
 * the repeat window with the prompt's last repeat_last_n tokens (136-143),
 * prefill, then up to min(max_new_tokens, context - n_prompt) times: sample
 * the current logits (llrs_sample, with uniforms[i] as the i-th draw; unused
 * and may be NULL when temperature is 0), record the token, remember it, stop
 * if it is one of eos_ids (the EOS token is kept, as the reference pushes
 * before checking), else forward it at the next position.  Fails as the
 * reference does on an empty prompt and on a prompt that does not leave a
 * position for decoding ("prompt has N tokens, but context is M").
 * out_tokens holds max_new_tokens ids; result gets the counts and the
 * prefill / decode wall time (InferenceMetrics, src/benchmark.rs:3-34). */
typedef struct llrs_generation {
  size_t prompt_tokens, generated_tokens;
  double prefill_ms, decode_ms;
  int stopped_on_eos;
} llrs_generation;
int llrs_generate(llrs_model *m, llrs_kv *kv, const uint32_t *prompt, size_t n_prompt,
                  const llrs_sampling *opts, size_t repeat_last_n, const uint32_t *eos_ids,
                  size_t n_eos, size_t max_new_tokens, const float *uniforms, uint32_t *out_tokens,
                  llrs_generation *result);
/* find_eos_tokens (src/engine.rs:340-387), host only: generation_config.json's
 * eos_token_id (a number or an array) in the model's directory (the path
 * itself if a directory, else its parent), then the ids of "<|im_end|>" and
 * "<|endoftext|>" in tokenizer.json (added tokens first, then the model's
 * vocabulary, as Tokenizer::token_to_id), sorted and deduplicated.
 * tokenizer.json is required (InferenceEngine::from_path loads it first).
 * *n_out = the count; out may be NULL with capacity 0 to query it. */
int llrs_find_eos_tokens(const char *model_path, uint32_t *out, size_t capacity, size_t *n_out);
/* Readback for tests: InferenceBuffers::logits (src/cache.rs:76) and
 * KVCache::{k,v}_cache[layer][0 .. n) (src/cache.rs:5-7). */
int llrs_read_logits(llrs_kv *kv, float *out, size_t n);
int llrs_read_kv(llrs_kv *kv, size_t layer, int which /*0 = K, 1 = V*/, float *out, size_t n);
/* Readback for tests: the token ids the device holds for positions
 * [start, start + n).  Position p holds the token fed at p; after a step (or
 * a prefill) that computed logits at p, position p + 1 holds their greedy
 * token, written by the LM-head launch (the argmax_current_logits of
 * src/engine.rs:233-241 that the next step consumes).  start + n may reach
 * max_seq_len + 1 (the slot after the context). */
int llrs_read_tokens(llrs_kv *kv, size_t start, size_t n, uint32_t *out);

/* Measurement hook (no reference counterpart; llama-bench times whole steps,
 * src/bin/llama-bench.rs:117-126): times the decode step's launch(es) for one
 * projection group with HIP events on the backend's stream.  `which`: 0 q/k/v
 * (RMSNorm fused), 1 o (+ residual), 2 gate/up (RMSNorm + SiLU*up fused),
 * 3 down (+ residual), 4 LM head (RMSNorm + argmax fused), 5 every layer of
 * the step (the persistent kernel when llrs_kv_decode_path is 1, else the
 * per-phase launches; the embedding runs untimed before each round).  The
 * layer groups rotate over every layer so each launch streams its own
 * weights; the LM head is one matrix.  Runs `iters` rounds and restores the
 * position; returns the mean launch (5: round) time in microseconds and the
 * weight bytes one launch reads. */
int llrs_profile_projection(llrs_model *m, llrs_kv *kv, int which, int iters, double *avg_us,
                            size_t *bytes_per_launch);

#ifdef __cplusplus
}
#endif
#endif
