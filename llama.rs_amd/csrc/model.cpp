// Qwen2 model on the GPU: loader, device KV cache, per-token step, hipGraph
// decode loop (the C ABI model half of include/llrs.h).
//
//   llrs_model_load_gguf   GgufLoader::load (src/loader.rs:233-399) incl.
//                          maybe_quantize (406-447) and load_gguf_* (497-534)
//   llrs_model_load_safetensors  SafetensorsLoader::load (src/loader.rs:80-228)
//                          incl. load_st_* (458-495)
//   llrs_model_load        ModelLoader::load's format detection (src/loader.rs:44-77)
//   llrs_kv_create         KVCache::new + InferenceBuffers::new (src/cache.rs:13-101)
//   llrs_forward_token     Qwen2Model::forward_impl (src/model.rs:135-271)
//   llrs_prefill           CausalModel::prefill (src/architecture.rs:60-77)
//   llrs_decode_greedy     InferenceEngine::benchmark_tokens' decode loop
//                          (src/engine.rs:205-216) + argmax (233-241)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <initializer_list>
#include <thread>
#include <new>
#include <string>
#include <mutex>
#include <vector>

#include "common.h"
#include "decode.h"
#include "decode_persistent.h"
#include "gemv.h"
#include "gguf.h"
#include "prefill.h"
#include "quantize.h"
#include "safetensors.h"
#include "quant_encode.h"
#include "sampling.h"
#include "synth.h"

namespace llrs {

struct DevLayer {
  llrs_tensor *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr, *gate = nullptr,
              *up = nullptr, *down = nullptr;
  float *attn_norm = nullptr, *ffn_norm = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr;
};

// A named model tensor in load order: a matrix, or an f32 vector.
struct TensorRef {
  std::string name;
  llrs_tensor *mat;
  float *vec;
  size_t len;
};

}  // namespace llrs

struct llrs_model {
  llrs_backend *b = nullptr;  // a counted reference (backend_retain)
  // The caller's handle + one per KV cache: a cache keeps its model (and so
  // the backend) alive, as the reference's caches borrow a model that holds
  // an Arc of its backend (src/model.rs:117).
  std::atomic<int> owners{1};
  llrs_model_config cfg{};
  llrs_tensor *embed = nullptr, *lm_head = nullptr;
  float *norm = nullptr;
  std::vector<llrs::DevLayer> layers;
  std::vector<llrs_tensor *> tensors;
  std::vector<void *> vecs;
  std::vector<llrs::TensorRef> refs;
  size_t weight_bytes = 0;
};

struct llrs_kv {
  llrs_model *m = nullptr;
  size_t max_seq_len = 0;
  float *k_cache = nullptr, *v_cache = nullptr;  // [layer][pos][kv_width]
  float *hidden = nullptr, *residual = nullptr, *q = nullptr, *k = nullptr, *v = nullptr,
        *attn = nullptr, *gate = nullptr, *up = nullptr, *act = nullptr, *logits = nullptr,
        *rope = nullptr;
  unsigned long long *scores = nullptr;  // attention chunk partials, tagged words
  unsigned *epoch = nullptr;             // the step's tag, advanced by the embedding
  unsigned *attn_err = nullptr;          // an attention merge gave up waiting
  llrs::SampleScratch sample;            // llrs_sample's buffers, allocated on first use
  int *pos = nullptr;
  uint32_t *tok_by_pos = nullptr, *next_token = nullptr;
  unsigned long long *amax_key = nullptr;  // LM-head argmax accumulator (zero between steps)
  unsigned *done = nullptr;                // LM-head block completion counter
  uint8_t *act_dig = nullptr;              // SiLU*up digitised by gate/up for ffn_down
  // Persistent decode (one launch for every layer), when the model's weight
  // types have an instantiation: per-layer arguments, barrier words, error flag.
  llrs::PersistentLayer *p_layers = nullptr;
  unsigned *p_bar = nullptr, *p_err = nullptr;
  llrs::AttnArgs p_attn{};  // layer 0's attention (per-layer buffers act_stride floats apart)
  long p_act_stride = 0;
  bool p_bar_uc = false;    // p_bar is uncached memory (scalar polls), returned to the pool
  int p_grid = 0;
  size_t p_lds = 0;
  uint32_t p_types[5] = {};
  uint32_t *pinned = nullptr;  // host staging, max_seq_len + 2 words
  // Captured steps: [logits mode + 2 * long] (long: the persistent kernel's
  // instantiation for positions past 2,048).
  hipGraph_t graph[4] = {};
  hipGraphExec_t exec[4] = {};
  std::vector<void *> allocs;
  // Multi-token prefill buffers (allocated on first use, pf_cap token rows).
  size_t pf_cap = 0;
  float *pf_x = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr, *pf_g = nullptr,
        *pf_u = nullptr;
  llrs::f16 *pf_h = nullptr, *pf_hl = nullptr;  // GEMM inputs as f16 hi + lo pairs
  llrs::f16 *pf_xs = nullptr, *pf_xsl = nullptr;  // their 32-column sums (Q4_K products), [pf_cap][pf_ldxs]
  llrs::f16 *pf_xs2 = nullptr, *pf_xsl2 = nullptr;  // the same for ffn_down's input of the dual gate/up product
  int pf_ldxs = 0;
  llrs::PrefillKvF16 pf_kvf{};  // one layer's K/V rows as f16 hi/lo planes (prefill attention)
  float *pf_part = nullptr;                     // split-K partial tiles of the prefill GEMMs
  size_t pf_part_cap = 0;                       // floats
};

namespace llrs {

// Materialises matrix `name` ([rows, cols]) as a device tensor.
using MatFn = std::function<int(const std::string &name, size_t rows, size_t cols, llrs_tensor **out)>;
// Writes vector `name` (length len) as f32 into dst (device); zeros if absent and allowed.
using VecFn = std::function<int(const std::string &name, size_t len, bool zeros_if_missing, float *dst)>;

static int dev_alloc(std::vector<void *> &list, void **p, size_t bytes) {
  LLRS_HIP(hipMalloc(p, bytes ? bytes : 4));
  list.push_back(*p);
  return LLRS_OK;
}

// Uncached device memory (no L2 keeps a copy, so scalar loads see other
// XCDs' atomics) for the persistent kernel's counters.  Once a kernel has read
// such memory it is never freed (freeing it has corrupted later allocations on
// this platform): released blocks return to a process-wide list for reuse.
namespace {
struct UcBlock {
  int device;
  void *ptr;
  size_t bytes;
  bool used;
};
std::mutex uc_mu;
std::vector<UcBlock> uc_blocks;
}  // namespace

static int uc_acquire(int device, size_t bytes, void **out) {
  std::lock_guard<std::mutex> g(uc_mu);
  for (UcBlock &b : uc_blocks)
    if (!b.used && b.device == device && b.bytes >= bytes) {
      b.used = true;
      *out = b.ptr;
      return LLRS_OK;
    }
  LLRS_HIP(hipExtMallocWithFlags(out, bytes, hipDeviceMallocUncached));
  uc_blocks.push_back({device, *out, bytes, true});
  return LLRS_OK;
}

static void uc_release(void *ptr) {
  std::lock_guard<std::mutex> g(uc_mu);
  for (UcBlock &b : uc_blocks)
    if (b.ptr == ptr) b.used = false;
}

// LlamaConfig::validate (src/config.rs:57-89), with head_dim = hidden / heads.
static int validate_config(llrs_model_config &c) {
  if (!c.hidden_size || !c.intermediate_size || !c.num_attention_heads || !c.num_key_value_heads ||
      !c.num_hidden_layers || !c.vocab_size)
    return set_error(LLRS_E_INVALID, "invalid Qwen2 config: dimensions must be non-zero");
  if (c.hidden_size % c.num_attention_heads)
    return set_error(LLRS_E_INVALID, "hidden_size must be divisible by num_attention_heads");
  if (c.num_attention_heads % c.num_key_value_heads)
    return set_error(LLRS_E_INVALID,
                     "num_attention_heads must be divisible by num_key_value_heads");
  c.head_dim = c.hidden_size / c.num_attention_heads;
  c.kv_width = c.num_key_value_heads * c.head_dim;
  if (c.head_dim % 2) return set_error(LLRS_E_INVALID, "Qwen2 RoPE requires an even head_dim");
  if (!std::isfinite(c.rms_norm_eps) || c.rms_norm_eps <= 0)
    return set_error(LLRS_E_INVALID, "rms_norm_eps must be finite and positive");
  if (!std::isfinite(c.rope_theta) || c.rope_theta <= 0)
    return set_error(LLRS_E_INVALID, "rope_theta must be finite and positive");
  return LLRS_OK;
}

// Host staging of a model load: two pinned buffers that the mapped
// checkpoint bytes are copied into by several threads (the page faults of the
// mapping spread over them), and a copy stream (default priority) whose
// transfers overlap the encoding of the previous chunk on the backend stream.
struct LoadStaging {
  static constexpr size_t kCap = 64u << 20;
  llrs_backend *b = nullptr;
  hipStream_t cs = nullptr;
  uint8_t *pin[2] = {nullptr, nullptr};
  hipEvent_t copied[2] = {nullptr, nullptr};
  ~LoadStaging() {
    if (cs) (void)hipStreamSynchronize(cs);
    if (b) (void)hipStreamSynchronize(b->stream);
    for (int i = 0; i < 2; i++) {
      if (pin[i]) (void)hipHostFree(pin[i]);
      if (copied[i]) (void)hipEventDestroy(copied[i]);
    }
    if (cs) (void)hipStreamDestroy(cs);
  }
  int init(llrs_backend *be) {
    b = be;
    LLRS_HIP(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking));
    for (int i = 0; i < 2; i++) {
      LLRS_HIP(hipHostMalloc((void **)&pin[i], kCap, hipHostMallocDefault));
      LLRS_HIP(hipEventCreateWithFlags(&copied[i], hipEventDisableTiming));
    }
    return LLRS_OK;
  }
};

static void parallel_copy(uint8_t *dst, const uint8_t *src, size_t n) {
  const size_t kMinPart = 4u << 20;
  const unsigned nt = (unsigned)std::min<size_t>(8, std::max<size_t>(1, n / kMinPart));
  if (nt == 1) {
    memcpy(dst, src, n);
    return;
  }
  std::vector<std::thread> th;
  const size_t part = (n + nt - 1) / nt;
  for (unsigned i = 0; i < nt; i++) {
    const size_t o = i * part, len = o < n ? std::min(part, n - o) : 0;
    if (len) th.emplace_back([=] { memcpy(dst + o, src + o, len); });
  }
  for (auto &t : th) t.join();
}

// maybe_quantize (src/loader.rs:406-447) on the GPU: the F32/F16/BF16 source
// bytes are uploaded as they are, widened to f32 on the device and encoded
// by the same encoders the host quantizer uses (bit-identical).  want may be
// LLRS_F32 (a recipe fallback), which keeps the widened values.  With
// staging, the rows go up in chunks of at most 64 MB through its pinned
// buffers, each chunk widened and encoded while the next one is staged.
static int quantize_on_device(llrs_backend *b, uint32_t want, uint32_t src_ty, const uint8_t *src,
                              size_t rows, size_t cols, llrs_tensor **out, LoadStaging *st = nullptr) {
  const size_t n = rows * cols, es = src_ty == LLRS_F32 ? 4 : 2;
  if (want == LLRS_F32 && src_ty == LLRS_F32 && !st)
    return llrs_tensor_upload(b, src, n * 4, LLRS_F32, rows, cols, out);
  llrs_tensor *t = nullptr;
  void *raw = nullptr;
  float *dv = nullptr;
  int rc = tensor_alloc(b, want, rows, cols, &t);
  hipError_t e = hipSuccess;
  if (rc == LLRS_OK) {
    float *vals = want == LLRS_F32 ? (float *)t->dev : nullptr;
    if (!vals) {
      e = hipMalloc(&dv, n * 4 + 4);
      vals = dv;
    }
    if (e == hipSuccess && src_ty != LLRS_F32) e = hipMalloc(&raw, n * 2 + 4);
    // Rows per chunk: whole rows within the staging buffer (all rows without staging).
    const size_t row_src = cols * es;
    const size_t per = st ? std::max<size_t>(1, LoadStaging::kCap / std::max<size_t>(row_src, 1)) : rows;
    if (st && row_src > LoadStaging::kCap) rc = set_error(LLRS_E_UNSUPPORTED, "a %zu-byte row exceeds the load staging", row_src);
    for (size_t r0 = 0, i = 0; r0 < rows && e == hipSuccess && rc == LLRS_OK; r0 += per, i++) {
      const size_t r1 = std::min(rows, r0 + per), off = r0 * row_src, len = (r1 - r0) * row_src;
      uint8_t *dst = src_ty == LLRS_F32 ? (uint8_t *)(vals + r0 * cols) : (uint8_t *)raw + off;
      if (st) {
        const int k = (int)(i & 1);
        e = hipEventSynchronize(st->copied[k]);  // the DMA that last read this buffer is done
        if (e != hipSuccess) break;
        parallel_copy(st->pin[k], src + off, len);
        e = hipMemcpyAsync(dst, st->pin[k], len, hipMemcpyHostToDevice, st->cs);
        if (e == hipSuccess) e = hipEventRecord(st->copied[k], st->cs);
        if (e == hipSuccess) e = hipStreamWaitEvent(b->stream, st->copied[k], 0);
      } else {
        e = hipMemcpyAsync(dst, src + off, len, hipMemcpyHostToDevice, b->stream);
      }
      if (e == hipSuccess && src_ty != LLRS_F32)
        rc = launch_widen(src_ty, dst, (r1 - r0) * cols, vals + r0 * cols, b->stream);
      if (e == hipSuccess && rc == LLRS_OK && want != LLRS_F32)
        rc = launch_encode(want, vals + r0 * cols, r1 - r0, cols, t->dev + r0 * t->row_bytes, t->row_bytes,
                           b->stream);
    }
    if (e == hipSuccess && rc == LLRS_OK) e = hipStreamSynchronize(b->stream);
  }
  if (rc != LLRS_OK || e != hipSuccess) {
    if (st) (void)hipStreamSynchronize(st->cs);
    (void)hipStreamSynchronize(b->stream);
  }
  if (dv) (void)hipFree(dv);
  if (raw) (void)hipFree(raw);
  if (rc == LLRS_OK && e != hipSuccess) rc = set_error(LLRS_E_HIP, "device quantization failed: %s", hipGetErrorString(e));
  if (rc != LLRS_OK) {
    if (t) llrs_tensor_free(t);
    return rc;
  }
  *out = t;
  return LLRS_OK;
}

// load_gguf_matrix + check_matrix + maybe_quantize (src/loader.rs:406-456, 497-507).
static int gguf_matrix(llrs_model *m, const GgufFile &g, const std::string &name, size_t rows,
                       size_t cols, int quantization, llrs_tensor **out, LoadStaging *st) {
  const GgufTensorInfo *t = g.tensor(name);
  if (!t) return set_error(LLRS_E_INVALID, "missing GGUF tensor %s", name.c_str());
  const std::vector<uint64_t> &dims = t->dims;
  if (dims.size() > 2)
    return set_error(LLRS_E_INVALID, "tensor %s has %zu dimensions; Qwen2 loader supports 1D/2D weights",
                     name.c_str(), dims.size());
  if (dims.size() != 2 || dims[1] != rows || dims[0] != cols)
    return set_error(LLRS_E_INVALID, "tensor %s has shape [%llu, %llu], expected [%zu, %zu]",
                     name.c_str(), (unsigned long long)(dims.size() == 2 ? dims[1] : dims[0]),
                     (unsigned long long)(dims.size() == 2 ? dims[0] : 0), rows, cols);
  uint32_t ty = t->type;
  if (quantization != LLRS_QUANT_NONE && (ty == LLRS_F32 || ty == LLRS_F16 || ty == LLRS_BF16))
    return quantize_on_device(m->b, recipe_type(quantization, name, cols), ty, g.data(*t), rows, cols, out, st);
  return llrs_tensor_upload(m->b, g.data(*t), t->nbytes, ty, rows, cols, out);
}

// load_gguf_vector (src/loader.rs:509-517): any type, dequantized bit-exactly
// (value_at) on the device into an f32 vector; missing Q/K/V biases are zeros
// (src/loader.rs:528-531).
static int gguf_vector(llrs_model *m, const GgufFile &g, const std::string &name, size_t len,
                       bool zeros_if_missing, float *dst) {
  const GgufTensorInfo *t = g.tensor(name);
  if (!t) {
    if (!zeros_if_missing) return set_error(LLRS_E_INVALID, "missing GGUF tensor %s", name.c_str());
    LLRS_HIP(hipMemsetAsync(dst, 0, len * 4, m->b->stream));
    LLRS_HIP(hipStreamSynchronize(m->b->stream));
    return LLRS_OK;
  }
  if (t->dims.size() != 1 || t->dims[0] != len)
    return set_error(LLRS_E_INVALID, "tensor %s has the wrong shape, expected [%zu]", name.c_str(), len);
  llrs_tensor *tmp = nullptr;
  LLRS_TRY(llrs_tensor_upload(m->b, g.data(*t), t->nbytes, t->type, 1, len, &tmp));
  int rc = launch_dequant_row(tmp, 0, dst, m->b->stream);
  hipError_t e = hipStreamSynchronize(m->b->stream);
  llrs_tensor_free(tmp);
  LLRS_TRY(rc);
  if (e != hipSuccess) return set_error(LLRS_E_HIP, "vector dequant failed: %s", hipGetErrorString(e));
  return LLRS_OK;
}

static int build_model(llrs_model *m, const MatFn &mat, const VecFn &vec) {
  const llrs_model_config &c = m->cfg;
  size_t H = c.hidden_size, F = c.intermediate_size, KV = c.kv_width;
  auto M = [&](const std::string &name, size_t rows, size_t cols, llrs_tensor **out) -> int {
    LLRS_TRY(mat(name, rows, cols, out));
    m->tensors.push_back(*out);
    m->refs.push_back({name, *out, nullptr, 0});
    return LLRS_OK;
  };
  auto V = [&](const std::string &name, size_t len, bool zeros, float **out) -> int {
    LLRS_TRY(dev_alloc(m->vecs, (void **)out, len * 4));
    LLRS_TRY(vec(name, len, zeros, *out));
    m->refs.push_back({name, nullptr, *out, len});
    return LLRS_OK;
  };
  LLRS_TRY(M("token_embd.weight", c.vocab_size, H, &m->embed));
  LLRS_TRY(V("output_norm.weight", H, false, &m->norm));
  m->layers.resize(c.num_hidden_layers);
  for (size_t i = 0; i < c.num_hidden_layers; i++) {
    DevLayer &L = m->layers[i];
    std::string p = "blk." + std::to_string(i) + ".";
    LLRS_TRY(V(p + "attn_norm.weight", H, false, &L.attn_norm));
    LLRS_TRY(M(p + "attn_q.weight", H, H, &L.q));
    LLRS_TRY(V(p + "attn_q.bias", H, true, &L.bq));
    LLRS_TRY(M(p + "attn_k.weight", KV, H, &L.k));
    LLRS_TRY(V(p + "attn_k.bias", KV, true, &L.bk));
    LLRS_TRY(M(p + "attn_v.weight", KV, H, &L.v));
    LLRS_TRY(V(p + "attn_v.bias", KV, true, &L.bv));
    LLRS_TRY(M(p + "attn_output.weight", H, H, &L.o));
    LLRS_TRY(V(p + "ffn_norm.weight", H, false, &L.ffn_norm));
    LLRS_TRY(M(p + "ffn_gate.weight", F, H, &L.gate));
    LLRS_TRY(M(p + "ffn_up.weight", F, H, &L.up));
    LLRS_TRY(M(p + "ffn_down.weight", H, F, &L.down));
  }
  if (c.tie_word_embeddings) m->lm_head = m->embed;
  else LLRS_TRY(M("output.weight", c.vocab_size, H, &m->lm_head));
  // Bytes one decode step streams from HBM for weights.
  size_t wb = m->lm_head->nbytes + m->embed->row_bytes + H * 4;
  for (auto &L : m->layers)
    wb += L.q->nbytes + L.k->nbytes + L.v->nbytes + L.o->nbytes + L.gate->nbytes + L.up->nbytes +
          L.down->nbytes + (2 * H + H + 2 * KV) * 4;
  m->weight_bytes = wb;
  return LLRS_OK;
}

// A new model holding a reference to b.
static llrs_model *model_new(llrs_backend *b) {
  llrs_model *m = new (std::nothrow) llrs_model();
  if (m) {
    m->b = b;
    backend_retain(b);
  }
  return m;
}

// Drops one reference; the last one frees the weights and releases the
// backend.
static void free_model(llrs_model *m) {
  if (!m || m->owners.fetch_sub(1, std::memory_order_acq_rel) != 1) return;
  llrs_backend *b = m->b;
  (void)hipSetDevice(b->device);
  (void)hipStreamSynchronize(b->stream);
  for (auto *t : m->tensors) llrs_tensor_free(t);
  for (void *p : m->vecs) (void)hipFree(p);
  delete m;
  backend_release(b);
}

static int load_gguf_impl(llrs_backend *b, const char *path, int quantization, llrs_model **out) {
  GgufFile g;
  LLRS_TRY(g.open(path));
  const GgufValue *arch = g.meta("general.architecture");
  if (!arch || arch->kind != GgufValue::STR)
    return set_error(LLRS_E_FORMAT, "missing or non-string GGUF metadata general.architecture");
  if (arch->s != "qwen2")
    return set_error(LLRS_E_UNSUPPORTED, "unsupported GGUF architecture \"%s\"", arch->s.c_str());
  const GgufTensorInfo *te = g.tensor("token_embd.weight");
  if (!te) return set_error(LLRS_E_INVALID, "missing GGUF tensor token_embd.weight");
  if (te->dims.size() != 2) return set_error(LLRS_E_INVALID, "token_embd.weight must be 2D");
  llrs_model_config c{};
  auto u64 = [&](const char *key, size_t &dst) -> int {
    const GgufValue *v = g.meta(key);
    uint64_t x;
    if (!v || !v->as_u64(x))
      return set_error(LLRS_E_FORMAT, "missing or non-integer GGUF metadata %s", key);
    dst = (size_t)x;
    return LLRS_OK;
  };
  LLRS_TRY(u64("qwen2.embedding_length", c.hidden_size));
  LLRS_TRY(u64("qwen2.feed_forward_length", c.intermediate_size));
  LLRS_TRY(u64("qwen2.attention.head_count", c.num_attention_heads));
  LLRS_TRY(u64("qwen2.attention.head_count_kv", c.num_key_value_heads));
  LLRS_TRY(u64("qwen2.block_count", c.num_hidden_layers));
  c.vocab_size = (size_t)te->dims[1];
  const GgufValue *eps = g.meta("qwen2.attention.layer_norm_rms_epsilon");
  if (!eps || !eps->as_f32(c.rms_norm_eps))
    return set_error(LLRS_E_FORMAT,
                     "missing or non-numeric GGUF metadata qwen2.attention.layer_norm_rms_epsilon");
  const GgufValue *th = g.meta("qwen2.rope.freq_base");
  if (!th || !th->as_f32(c.rope_theta)) c.rope_theta = 10000.0f;
  LLRS_TRY(u64("qwen2.context_length", c.max_position_embeddings));
  c.tie_word_embeddings = g.tensor("output.weight") == nullptr;
  LLRS_TRY(validate_config(c));
  if (te->dims[0] != c.hidden_size)
    return set_error(LLRS_E_INVALID, "GGUF embedding width/config mismatch");
  llrs_model *m = model_new(b);
  if (!m) return set_error(LLRS_E_OOM, "out of host memory");
  m->cfg = c;
  LoadStaging stg;
  if (quantization != LLRS_QUANT_NONE) {
    int rc = stg.init(b);
    if (rc != LLRS_OK) {
      free_model(m);
      return rc;
    }
  }
  MatFn mat = [&](const std::string &name, size_t rows, size_t cols, llrs_tensor **t) {
    return gguf_matrix(m, g, name, rows, cols, quantization, t, quantization != LLRS_QUANT_NONE ? &stg : nullptr);
  };
  VecFn vec = [&](const std::string &name, size_t len, bool zeros, float *dst) {
    return gguf_vector(m, g, name, len, zeros, dst);
  };
  int rc = build_model(m, mat, vec);
  if (rc != LLRS_OK) {
    free_model(m);
    return rc;
  }
  *out = m;
  return LLRS_OK;
}

// The Hugging Face tensor name of a GGUF tensor name (the names
// SafetensorsLoader::load reads, src/loader.rs:102-213).
static std::string hf_name(const std::string &g) {
  static const std::pair<const char *, const char *> kTop[] = {
      {"token_embd.weight", "model.embed_tokens.weight"},
      {"output_norm.weight", "model.norm.weight"},
      {"output.weight", "lm_head.weight"}};
  for (const auto &t : kTop)
    if (g == t.first) return t.second;
  static const std::pair<const char *, const char *> kLayer[] = {
      {"attn_norm.weight", "input_layernorm.weight"},
      {"ffn_norm.weight", "post_attention_layernorm.weight"},
      {"attn_q.weight", "self_attn.q_proj.weight"},
      {"attn_q.bias", "self_attn.q_proj.bias"},
      {"attn_k.weight", "self_attn.k_proj.weight"},
      {"attn_k.bias", "self_attn.k_proj.bias"},
      {"attn_v.weight", "self_attn.v_proj.weight"},
      {"attn_v.bias", "self_attn.v_proj.bias"},
      {"attn_output.weight", "self_attn.o_proj.weight"},
      {"ffn_gate.weight", "mlp.gate_proj.weight"},
      {"ffn_up.weight", "mlp.up_proj.weight"},
      {"ffn_down.weight", "mlp.down_proj.weight"}};
  const size_t dot = g.find('.', 4);  // "blk.<i>.<rest>"
  const std::string layer = g.substr(4, dot - 4), rest = g.substr(dot + 1);
  for (const auto &t : kLayer)
    if (rest == t.first) return "model.layers." + layer + "." + t.second;
  return g;
}

static uint32_t st_type(const SafetensorInfo &t) {
  return t.dtype == "F32" ? LLRS_F32 : t.dtype == "F16" ? LLRS_F16 : LLRS_BF16;
}

// load_st_matrix + check_matrix + maybe_quantize (src/loader.rs:406-467).
static int st_matrix(llrs_model *m, SafetensorStore &st, const std::string &name, size_t rows,
                     size_t cols, int quantization, llrs_tensor **out, LoadStaging *stg) {
  const SafetensorsFile *f = nullptr;
  const SafetensorInfo *t = nullptr;
  LLRS_TRY(st.tensor(name, &f, &t));
  if (t->shape.size() != 2 || t->shape[0] != rows || t->shape[1] != cols)
    return set_error(LLRS_E_INVALID, "tensor %s has shape [%llu%s%llu], expected [%zu, %zu]", name.c_str(),
                     (unsigned long long)t->shape[0], t->shape.size() == 2 ? ", " : "",
                     (unsigned long long)(t->shape.size() == 2 ? t->shape[1] : 0), rows, cols);
  const uint32_t ty = st_type(*t);
  if (quantization != LLRS_QUANT_NONE)
    return quantize_on_device(m->b, recipe_type(quantization, name, cols), ty, f->data(*t), rows, cols, out, stg);
  return llrs_tensor_upload(m->b, f->data(*t), t->nbytes, ty, rows, cols, out);
}

// load_st_vector (src/loader.rs:469-477) into an f32 device vector; a missing
// Q/K/V bias is zeros (src/loader.rs:479-495).
static int st_vector(llrs_model *m, SafetensorStore &st, const std::string &name, size_t len,
                     bool zeros_if_missing, float *dst) {
  if (zeros_if_missing && !st.contains(name)) {
    LLRS_HIP(hipMemsetAsync(dst, 0, len * 4, m->b->stream));
    LLRS_HIP(hipStreamSynchronize(m->b->stream));
    return LLRS_OK;
  }
  const SafetensorsFile *f = nullptr;
  const SafetensorInfo *t = nullptr;
  LLRS_TRY(st.tensor(name, &f, &t));
  if (t->shape.size() != 1 || t->shape[0] != len)
    return set_error(LLRS_E_INVALID, "tensor %s has the wrong shape, expected [%zu]", name.c_str(), len);
  const uint32_t ty = st_type(*t);
  if (ty == LLRS_F32) {
    LLRS_HIP(hipMemcpyAsync(dst, f->data(*t), len * 4, hipMemcpyHostToDevice, m->b->stream));
    LLRS_HIP(hipStreamSynchronize(m->b->stream));
    return LLRS_OK;
  }
  void *raw = nullptr;
  LLRS_HIP(hipMalloc(&raw, len * 2 + 4));
  hipError_t e = hipMemcpyAsync(raw, f->data(*t), len * 2, hipMemcpyHostToDevice, m->b->stream);
  int rc = e == hipSuccess ? launch_widen(ty, raw, len, dst, m->b->stream) : LLRS_OK;
  if (e == hipSuccess && rc == LLRS_OK) e = hipStreamSynchronize(m->b->stream);
  (void)hipFree(raw);
  LLRS_TRY(rc);
  if (e != hipSuccess) return set_error(LLRS_E_HIP, "vector upload failed: %s", hipGetErrorString(e));
  return LLRS_OK;
}

static int load_safetensors_impl(llrs_backend *b, const std::string &dir, int quantization,
                                 llrs_model **out) {
  llrs_model_config c{};
  LLRS_TRY(hf_config_read(dir + "/config.json", c));
  SafetensorStore st;
  LLRS_TRY(st.open(dir));
  // The LM head is lm_head.weight when the checkpoint has one, else the
  // embedding matrix (src/loader.rs:203-214), whatever config.json says.
  c.tie_word_embeddings = !st.contains("lm_head.weight");
  LLRS_TRY(validate_config(c));
  llrs_model *m = model_new(b);
  if (!m) return set_error(LLRS_E_OOM, "out of host memory");
  m->cfg = c;
  LoadStaging stg;
  if (quantization != LLRS_QUANT_NONE) {
    int rc = stg.init(b);
    if (rc != LLRS_OK) {
      free_model(m);
      return rc;
    }
  }
  MatFn mat = [&](const std::string &name, size_t rows, size_t cols, llrs_tensor **t) {
    return st_matrix(m, st, hf_name(name), rows, cols, quantization, t, quantization != LLRS_QUANT_NONE ? &stg : nullptr);
  };
  VecFn vec = [&](const std::string &name, size_t len, bool zeros, float *dst) {
    return st_vector(m, st, hf_name(name), len, zeros, dst);
  };
  int rc = build_model(m, mat, vec);
  if (rc != LLRS_OK) {
    free_model(m);
    return rc;
  }
  *out = m;
  return LLRS_OK;
}

static int synth_config_to_model(const llrs_synth_config &s, llrs_model_config &c) {
  c = llrs_model_config{};
  c.hidden_size = s.hidden_size;
  c.intermediate_size = s.intermediate_size;
  c.num_attention_heads = s.num_attention_heads;
  c.num_key_value_heads = s.num_key_value_heads;
  c.num_hidden_layers = s.num_hidden_layers;
  c.vocab_size = s.vocab_size;
  c.max_position_embeddings = s.max_position_embeddings;
  c.rms_norm_eps = s.rms_norm_eps;
  c.rope_theta = s.rope_theta;
  c.tie_word_embeddings = s.tie_word_embeddings;
  if (s.recipe != LLRS_QUANT_NONE && s.recipe != LLRS_QUANT_Q4K && s.recipe != LLRS_QUANT_Q4KM)
    return set_error(LLRS_E_INVALID, "unknown recipe %d", s.recipe);
  return validate_config(c);
}

// ------------------------------------------------------------------ decode step

// Projection groups of the decode step: each is one launch on the tuned path
// (fused RMSNorm prologue / epilogues), or the generic sequence otherwise.
enum Proj { P_QKV = 0, P_O, P_GATE_UP, P_DOWN, P_LM_HEAD, P_COUNT };
// Profiling only: every layer of the step (the persistent kernel, or the
// per-phase launches), embedding and LM head excluded.
constexpr int P_LAYERS = P_COUNT;

static bool fast_ok(const llrs_tensor *t) {
  return t->rows % 4 == 0 && t->rows <= INT32_MAX && fast_gemv_supports(t->type, t->cols);
}

static bool use_fast(llrs_model *m, size_t l, int which) {
  const char *e = getenv("LLRS_GENERIC_GEMV");
  if (e && *e && *e != '0') return false;
  if (which == P_LM_HEAD) return fast_ok(m->lm_head);
  const DevLayer &L = m->layers[l];
  switch (which) {
    case P_QKV:
      return fast_ok(L.q) && fast_ok(L.k) && fast_ok(L.v) && L.q->type == L.k->type &&
             fast_gemv_supports_pair(L.q->type, L.v->type);
    case P_O: return fast_ok(L.o);
    case P_GATE_UP: return fast_ok(L.gate) && fast_ok(L.up) && L.gate->type == L.up->type;
    default: return fast_ok(L.down);
  }
}

static int fast_grid(llrs_model *m, const FastGemvArgs &a, bool dual = false) {
  return fast_gemv_grid(m->b->cu_count, a.rows, a.cols, dual, a.part);
}

static FastSeg seg_of(const llrs_tensor *t, const float *bias, float *out) {
  FastSeg s;
  s.w = t->dev;
  s.type = t->type;
  s.rows = (int)t->rows;
  s.row_bytes = (long)t->row_bytes;
  s.bias = bias;
  s.out = out;
  return s;
}

// The tuned GEMV's arguments for projection group `which` of layer `l` (the
// caller has checked use_fast); shared by the per-phase launches and the
// persistent decode kernel.
static FastGemvArgs projection_args(llrs_model *m, llrs_kv *kv, size_t l, int which) {
  const llrs_model_config &c = m->cfg;
  const int H = (int)c.hidden_size, F = (int)c.intermediate_size;
  FastGemvArgs a{};
  a.eps = c.rms_norm_eps;
  a.cols = H;
  a.x = kv->residual;
  // No balanced split (bal = 0): in the decode step its partial-sum pass cost
  // more than the idle waves it fills.
  if (which == P_LM_HEAD) {
    a.seg[0] = seg_of(m->lm_head, nullptr, kv->logits);
    a.nseg = 1;
    a.rows = (int)c.vocab_size;
    a.norm = m->norm;
    a.epi = kEpiLogits;
    a.amax_key = kv->amax_key;
    a.done = kv->done;
    a.pos = kv->pos;
    a.tok_by_pos = kv->tok_by_pos;
    a.next_token = kv->next_token;
    a.max_pos = (int)kv->max_seq_len;
    return a;
  }
  DevLayer &L = m->layers[l];
  switch (which) {
    case P_QKV:
      a.seg[0] = seg_of(L.q, L.bq, kv->q);
      a.seg[1] = seg_of(L.k, L.bk, kv->k);
      a.seg[2] = seg_of(L.v, L.bv, kv->v);
      a.nseg = 3;
      a.rows = (int)(L.q->rows + L.k->rows + L.v->rows);
      a.norm = L.attn_norm;
      a.epi = kEpiStore;
      break;
    case P_O:
      a.seg[0] = seg_of(L.o, nullptr, kv->residual);
      a.nseg = 1;
      a.rows = H;
      a.x = kv->attn;
      a.epi = kEpiAdd;
      break;
    case P_GATE_UP:
      a.seg[0] = seg_of(L.gate, nullptr, kv->gate);
      a.seg[1] = seg_of(L.up, nullptr, kv->up);
      a.seg[2] = seg_of(L.gate, nullptr, kv->act);
      a.nseg = 1;
      a.rows = F;
      a.norm = L.ffn_norm;
      a.epi = kEpiSwiGlu;
      if (use_fast(m, l, P_DOWN) && F % 64 == 0) {
        // SiLU*up leaves digitised for ffn_down: workgroups own 16-row blocks.
        a.part = 16;
        a.dig_out = kv->act_dig;
      }
      break;
    default:  // P_DOWN
      a.seg[0] = seg_of(L.down, nullptr, kv->residual);
      a.nseg = 1;
      a.rows = H;
      a.cols = F;
      a.x = kv->act;
      a.epi = kEpiAdd;
      if (use_fast(m, l, P_GATE_UP) && F % 64 == 0) a.dig_in = kv->act_dig;
      break;
  }
  return a;
}

// The decode step's launch(es) for projection group `which` of layer `l`; the
// bench's per-kernel timing calls this same function.
static int launch_projection(llrs_model *m, llrs_kv *kv, size_t l, int which, hipStream_t s) {
  const llrs_model_config &c = m->cfg;
  const int H = (int)c.hidden_size, F = (int)c.intermediate_size;
  const float eps = c.rms_norm_eps;
  if (which < 0 || which >= P_COUNT) return set_error(LLRS_E_INVALID, "unknown projection %d", which);
  if (use_fast(m, l, which)) {
    const FastGemvArgs a = projection_args(m, kv, l, which);
    if (which == P_LM_HEAD) {
      // Packed rows (1,536 columns of Q4_K, 896 of Q8_0): eight waves per
      // workgroup; longer rows: four, with the row sums through ds_bpermute.
      const bool packed = fast_gemv_packed(a.seg[0].type, a.cols);
      return launch_gemv_fast(a, fast_grid(m, a), s, packed ? 512 : 256, !packed);
    }
    return launch_gemv_fast(a, fast_grid(m, a, which == P_GATE_UP), s);
  }
  if (which == P_LM_HEAD) {
    LLRS_TRY(launch_rmsnorm(kv->residual, m->norm, kv->hidden, H, eps, s));
    LLRS_TRY(launch_gemv_generic(m->lm_head, kv->hidden, kv->logits, nullptr, false, s));
    return launch_argmax(kv->logits, (int)c.vocab_size, kv->pos, (int)kv->max_seq_len,
                         kv->tok_by_pos, kv->next_token, 1, s);
  }
  DevLayer &L = m->layers[l];
  switch (which) {
    case P_QKV:
      LLRS_TRY(launch_rmsnorm(kv->residual, L.attn_norm, kv->hidden, H, eps, s));
      LLRS_TRY(launch_gemv_generic(L.q, kv->hidden, kv->q, L.bq, false, s));
      LLRS_TRY(launch_gemv_generic(L.k, kv->hidden, kv->k, L.bk, false, s));
      return launch_gemv_generic(L.v, kv->hidden, kv->v, L.bv, false, s);
    case P_O: return launch_gemv_generic(L.o, kv->attn, kv->residual, nullptr, true, s);
    case P_GATE_UP:
      LLRS_TRY(launch_rmsnorm(kv->residual, L.ffn_norm, kv->hidden, H, eps, s));
      LLRS_TRY(launch_gemv_generic(L.gate, kv->hidden, kv->gate, nullptr, false, s));
      LLRS_TRY(launch_gemv_generic(L.up, kv->hidden, kv->up, nullptr, false, s));
      return launch_silu_mul(kv->gate, kv->up, kv->act, F, s);
    default: return launch_gemv_generic(L.down, kv->act, kv->residual, nullptr, true, s);
  }
}

static size_t projection_bytes(llrs_model *m, int which) {
  if (which == P_LM_HEAD) return m->lm_head->nbytes;
  if (which == P_LAYERS) {
    size_t b = 0;
    for (const DevLayer &L : m->layers)
      b += L.q->nbytes + L.k->nbytes + L.v->nbytes + L.o->nbytes + L.gate->nbytes + L.up->nbytes +
           L.down->nbytes;
    return b;
  }
  const DevLayer &L = m->layers[0];
  switch (which) {
    case P_QKV: return L.q->nbytes + L.k->nbytes + L.v->nbytes;
    case P_O: return L.o->nbytes;
    case P_GATE_UP: return L.gate->nbytes + L.up->nbytes;
    default: return L.down->nbytes;
  }
}

// The attention launch of layer l: GQA over the layer's cache at *pos.
static AttnArgs attention_args(llrs_model *m, llrs_kv *kv, size_t l) {
  const llrs_model_config &c = m->cfg;
  const size_t layer_stride = kv->max_seq_len * c.kv_width;
  AttnArgs at{};
  at.q = kv->q;
  at.k = kv->k;
  at.v = kv->v;
  at.rope = kv->rope;
  at.pos = kv->pos;
  at.k_cache = kv->k_cache + l * layer_stride;
  at.v_cache = kv->v_cache + l * layer_stride;
  at.out = kv->attn;
  at.scratch = kv->scores;
  at.epoch = kv->epoch;
  at.err = kv->attn_err;
  at.layer = (int)l;
  at.nlayers = (int)c.num_hidden_layers;
  at.nh = (int)c.num_attention_heads;
  at.nkv = (int)c.num_key_value_heads;
  at.hd = (int)c.head_dim;
  at.max_seq = (int)kv->max_seq_len;
  at.max_chunks = attention_chunks(at.max_seq);
  at.part_stride = attention_part_stride(at.hd);
  at.fold_max = attention_fold_default(at.hd);
  if (const char *e = getenv("LLRS_ATTN_FOLD")) {  // tuning: another fold bound
    const int f = atoi(e);
    if (f > 0) at.fold_max = f;
  }
  at.scale = 1.0f / sqrtf((float)c.head_dim);
  return at;
}

// The step's layers: one persistent launch, or five launches per layer.
static int enqueue_layers(llrs_model *m, llrs_kv *kv, bool long_items) {
  const llrs_model_config &c = m->cfg;
  hipStream_t s = m->b->stream;
  if (kv->p_layers) {
    PersistentArgs p{};
    p.layers = kv->p_layers;
    p.nlayers = (int)c.num_hidden_layers;
    p.attn = kv->p_attn;
    p.act_stride = kv->p_act_stride;
    p.cache_stride = (long)(kv->max_seq_len * c.kv_width);
    p.bar = kv->p_bar;
    p.scalar_poll = kv->p_bar_uc ? 1 : 0;
    p.err = kv->p_err;
    const uint32_t *t = kv->p_types;
    return launch_decode_persistent(p, t[0], t[1], t[2], t[3], t[4], (int)c.head_dim, kv->p_grid,
                                    kv->p_lds, s, long_items);
  }
  for (size_t l = 0; l < c.num_hidden_layers; l++) {
    LLRS_TRY(launch_projection(m, kv, l, P_QKV, s));
    LLRS_TRY(launch_attention(attention_args(m, kv, l), s));
    LLRS_TRY(launch_projection(m, kv, l, P_O, s));
    LLRS_TRY(launch_projection(m, kv, l, P_GATE_UP, s));
    LLRS_TRY(launch_projection(m, kv, l, P_DOWN, s));
  }
  return LLRS_OK;
}

// The embedding of tok_by_pos[*pos] (which also zeroes the persistent
// kernel's barrier counter).
static int enqueue_embed(llrs_model *m, llrs_kv *kv) {
  return launch_embed(m->embed, kv->tok_by_pos, kv->pos, (int)kv->max_seq_len, kv->residual,
                      kv->epoch, m->b->stream, kv->p_bar, kv->p_bar ? kPersistentBarWords : 0);
}

static int enqueue_step(llrs_model *m, llrs_kv *kv, int mode, bool long_items) {
  hipStream_t s = m->b->stream;
  const int max_seq = (int)kv->max_seq_len;
  LLRS_TRY(enqueue_embed(m, kv));
  LLRS_TRY(enqueue_layers(m, kv, long_items));
  if (mode == LLRS_LOGITS_COMPUTE) {
    LLRS_TRY(launch_projection(m, kv, 0, P_LM_HEAD, s));
  } else {
    LLRS_TRY(launch_advance(kv->pos, max_seq, s));
  }
  return LLRS_OK;
}

static bool use_graphs() {
  const char *e = getenv("LLRS_NO_GRAPH");
  return !(e && *e && *e != '0');
}

// One step at position pos (known to the host; the graph reads it from the
// device), replayed from a captured hipGraph (captured on first use).
static int run_step(llrs_model *m, llrs_kv *kv, int mode, size_t pos) {
  const bool lng = persistent_long_items(pos, (int)m->cfg.num_attention_heads);
  if (!use_graphs()) return enqueue_step(m, kv, mode, lng);
  hipStream_t s = m->b->stream;
  const int gi = mode + 2 * (lng ? 1 : 0);
  if (!kv->exec[gi]) {
    LLRS_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(m, kv, mode, lng);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc != LLRS_OK) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    if (e != hipSuccess) return set_error(LLRS_E_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    kv->graph[gi] = g;
    LLRS_HIP(hipGraphInstantiate(&kv->exec[gi], g, nullptr, nullptr, 0));
  }
  LLRS_HIP(hipGraphLaunch(kv->exec[gi], s));
  return LLRS_OK;
}

// Host precompute of every position's RoPE row exactly as prepare_rope
// (src/model.rs:76-84): inv = 1/theta^(2i/hd), angle = pos*inv, glibc sinf/cosf.
static void rope_table(float *dst, size_t max_seq, size_t hd, float theta) {
#pragma clang fp contract(off)
  size_t half = hd / 2;
  std::vector<float> inv(half);
  for (size_t i = 0; i < half; i++) inv[i] = 1.0f / powf(theta, 2.0f * (float)i / (float)hd);
  for (size_t p = 0; p < max_seq; p++)
    for (size_t i = 0; i < half; i++) {
      float a = (float)p * inv[i];
      dst[p * hd + i] = cosf(a);
      dst[p * hd + half + i] = sinf(a);
    }
}

static bool persistent_disabled() {
  const char *e = getenv("LLRS_NO_PERSISTENT");
  return e && *e && *e != '0';
}

// Chooses the persistent decode kernel when every layer runs the tuned GEMV
// with weight types that have an instantiation (one set for every layer, or
// Q4_K q/k/o/gate/up with V and ffn_down types varying by layer), and
// uploads the per-layer arguments it reads.
static int setup_persistent(llrs_model *m, llrs_kv *kv) {
  const llrs_model_config &c = m->cfg;
  if (persistent_disabled() || c.intermediate_size % 64) return LLRS_OK;
  const size_t nl = c.num_hidden_layers;
  uint32_t t[5] = {};
  bool varies = false, mixable = true;
  for (size_t l = 0; l < nl; l++) {
    for (int w = P_QKV; w <= P_DOWN; w++)
      if (!use_fast(m, l, w)) return LLRS_OK;
    const DevLayer &L = m->layers[l];
    const uint32_t tl[5] = {L.q->type, L.v->type, L.o->type, L.gate->type, L.down->type};
    if (l == 0) memcpy(t, tl, sizeof t);
    if (tl[0] != t[0] || tl[2] != t[2] || tl[3] != t[3]) return LLRS_OK;
    varies = varies || tl[1] != t[1] || tl[4] != t[4];
    mixable = mixable && (tl[1] == LLRS_Q8_0 || tl[1] == LLRS_Q4_K || tl[1] == LLRS_Q6_K) &&
              (tl[4] == LLRS_Q4_K || tl[4] == LLRS_Q6_K);
  }
  if (varies || !decode_persistent_supports(t[0], t[1], t[2], t[3], t[4], (int)c.head_dim)) {
    if (!mixable) return LLRS_OK;
    t[1] = t[4] = kTypePerLayer;  // the Q4_K family's per-layer instantiation
    if (!decode_persistent_supports(t[0], t[1], t[2], t[3], t[4], (int)c.head_dim)) return LLRS_OK;
  }
  const int grid = m->b->cu_count;
  // The attention tasks' wait order needs at least 8 G workgroups, and the
  // task partials two LDS buffers.
  if (grid < 8 * (int)(c.num_attention_heads / c.num_key_value_heads)) return LLRS_OK;
  static_assert(2 * kTaskItems * (2 * 128 + 2) * 4 <= kPersistentMinLds, "attention partials fit the LDS");
  // Per-layer activation buffers (each slice 256-byte aligned, so no cache
  // line holds two buffers): q|k|v, attention output, residual after o_proj
  // and after ffn_down, SiLU*up digits.  The last layer's ffn_down writes
  // the shared residual the LM head reads.
  const size_t H = c.hidden_size, KV = c.kv_width, F = c.intermediate_size;
  auto al = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t sz_qkv = al((H + 2 * KV) * 4), sz_h = al(H * 4), sz_dig = al(fast_gemv_digits_size(F));
  const size_t per_layer = sz_qkv + 3 * sz_h + sz_dig;
  uint8_t *act = nullptr;
  LLRS_TRY(dev_alloc(kv->allocs, (void **)&act, nl * per_layer));
  std::vector<PersistentLayer> host(nl);
  size_t lds = 0;
  const float *x_in = kv->residual;
  for (size_t l = 0; l < nl; l++) {
    uint8_t *b = act + l * per_layer;
    float *q = (float *)b, *k = q + H, *v = k + KV;
    float *attn = (float *)(b + sz_qkv), *x_mid = (float *)(b + sz_qkv + sz_h);
    float *x_out = l + 1 == nl ? kv->residual : (float *)(b + sz_qkv + 2 * sz_h);
    uint8_t *dig = b + sz_qkv + 3 * sz_h;
    PersistentLayer &P = host[l];
    P.qkv = projection_args(m, kv, l, P_QKV);
    P.qkv.x = x_in;
    P.qkv.seg[0].out = q;
    P.qkv.seg[1].out = k;
    P.qkv.seg[2].out = v;
    if (l == 0) {
      kv->p_attn = attention_args(m, kv, 0);
      kv->p_attn.q = q;
      kv->p_attn.k = k;
      kv->p_attn.v = v;
      kv->p_attn.out = attn;
    }
    P.o = projection_args(m, kv, l, P_O);
    P.o.x = attn;
    P.o.res_in = x_in;
    P.o.seg[0].out = x_mid;
    P.gate_up = projection_args(m, kv, l, P_GATE_UP);
    P.gate_up.x = x_mid;
    P.gate_up.dig_out = dig;
    P.down = projection_args(m, kv, l, P_DOWN);
    P.down.dig_in = dig;
    P.down.res_in = x_mid;
    P.down.seg[0].out = x_out;
    if (!P.gate_up.dig_out || P.gate_up.part != 16) return LLRS_OK;
    for (const FastGemvArgs *a : {&P.qkv, &P.o, &P.gate_up, &P.down})
      lds = std::max(lds, fast_gemv_lds_bytes(*a, grid, kPersistentThreads));
    x_in = x_out;
  }
  // More than half a CU's LDS per workgroup: exactly one workgroup per CU.
  lds = std::max(lds, kPersistentMinLds);
  if (lds + persistent_static_lds((int)c.head_dim) > kCuLds) return LLRS_OK;
  // The barriers need all `grid` workgroups resident at once: both
  // instantiations must fit one workgroup per CU with this LDS, else the
  // step runs as per-phase launches.
  for (bool lng : {false, true}) {
    int blocks = 0;
    LLRS_TRY(decode_persistent_blocks_per_cu(t[0], t[1], t[2], t[3], t[4], (int)c.head_dim, lds, lng, &blocks));
    if (blocks < 1) return LLRS_OK;
  }
  auto A = [&](void **p, size_t bytes) { return dev_alloc(kv->allocs, p, bytes); };
  LLRS_TRY(A((void **)&kv->p_layers, nl * sizeof(PersistentLayer)));
  // The barrier counters live in uncached memory and are polled by scalar
  // loads, which do not queue behind the CU's weight loads (+2% on the 7B
  // shape); LLRS_SCALAR_POLL=0 keeps them in ordinary memory with vector
  // polls.
  const char *sp = getenv("LLRS_SCALAR_POLL");
  kv->p_bar_uc = !(sp && *sp == '0');
  if (kv->p_bar_uc) {
    LLRS_TRY(uc_acquire(m->b->device, kPersistentBarWords * 4, (void **)&kv->p_bar));
  } else {
    LLRS_TRY(A((void **)&kv->p_bar, kPersistentBarWords * 4));
  }
  LLRS_TRY(A((void **)&kv->p_err, 64));
  hipStream_t s = m->b->stream;
  LLRS_HIP(hipMemcpyAsync(kv->p_layers, host.data(), nl * sizeof(PersistentLayer), hipMemcpyHostToDevice, s));
  LLRS_HIP(hipMemsetAsync(kv->p_bar, 0, kPersistentBarWords * 4, s));
  LLRS_HIP(hipMemsetAsync(kv->p_err, 0, 64, s));
  LLRS_HIP(hipStreamSynchronize(s));
  memcpy(kv->p_types, t, sizeof t);
  kv->p_act_stride = (long)(per_layer / 4);
  kv->p_grid = grid;
  kv->p_lds = lds;
  return LLRS_OK;
}

// Clears the device-side wait flags (outside any graph capture).
static int clear_wait_flags(llrs_kv *kv) {
  hipStream_t s = kv->m->b->stream;
  if (kv->p_err) LLRS_HIP(hipMemsetAsync(kv->p_err, 0, 4, s));
  LLRS_HIP(hipMemsetAsync(kv->attn_err, 0, 4, s));
  LLRS_HIP(hipStreamSynchronize(s));
  return LLRS_OK;
}

// Reports a device-side wait that gave up: a persistent-decode barrier or an
// attention merge (the stream is idle).  The flags are cleared once
// reported: the steps since the last check are untrustworthy (their K/V rows
// too, so the cache should be prefilled again), but later calls run normally.
static int check_persistent(llrs_kv *kv) {
  unsigned err = 0, aerr = 0;
  if (kv->p_err) LLRS_HIP(hipMemcpy(&err, kv->p_err, 4, hipMemcpyDeviceToHost));
  LLRS_HIP(hipMemcpy(&aerr, kv->attn_err, 4, hipMemcpyDeviceToHost));
  if (!err && !aerr) return LLRS_OK;
  LLRS_TRY(clear_wait_flags(kv));
  if (err) return set_error(LLRS_E_HIP, "persistent decode: a device-wide barrier timed out");
  return set_error(LLRS_E_HIP, "decode attention: a merge timed out waiting for partials");
}

// Frees the cache, then drops its reference to the model.
static void free_kv(llrs_kv *kv) {
  if (!kv) return;
  llrs_model *m = kv->m;
  (void)hipSetDevice(m->b->device);
  (void)hipStreamSynchronize(m->b->stream);
  for (int i = 0; i < 4; i++) {
    if (kv->exec[i]) (void)hipGraphExecDestroy(kv->exec[i]);
    if (kv->graph[i]) (void)hipGraphDestroy(kv->graph[i]);
  }
  for (void *p : kv->allocs) (void)hipFree(p);
  if (kv->p_bar_uc) uc_release(kv->p_bar);
  if (kv->pinned) (void)hipHostFree(kv->pinned);
  delete kv;
  free_model(m);
}

static int kv_create_impl(llrs_model *m, size_t max_seq, llrs_kv **out) {
  const llrs_model_config &c = m->cfg;
  if (max_seq == 0) return set_error(LLRS_E_INVALID, "max_seq_len must be positive");
  if (max_seq > c.max_position_embeddings)
    return set_error(LLRS_E_INVALID, "requested context %zu exceeds model limit %zu", max_seq,
                     c.max_position_embeddings);
  if (max_seq > (1u << 24)) return set_error(LLRS_E_INVALID, "context %zu is too large", max_seq);
  llrs_kv *kv = new (std::nothrow) llrs_kv();
  if (!kv) return set_error(LLRS_E_OOM, "out of host memory");
  kv->m = m;
  m->owners.fetch_add(1, std::memory_order_relaxed);  // released by free_kv
  kv->max_seq_len = max_seq;
  size_t L = c.num_hidden_layers, KV = c.kv_width, H = c.hidden_size, F = c.intermediate_size;
  auto A = [&](void **p, size_t bytes) { return dev_alloc(kv->allocs, p, bytes); };
  int rc = LLRS_OK;
  if ((rc = A((void **)&kv->k_cache, L * max_seq * KV * 4)) || (rc = A((void **)&kv->v_cache, L * max_seq * KV * 4)) ||
      (rc = A((void **)&kv->hidden, H * 4)) || (rc = A((void **)&kv->residual, H * 4)) ||
      (rc = A((void **)&kv->q, H * 4)) || (rc = A((void **)&kv->k, KV * 4)) ||
      (rc = A((void **)&kv->v, KV * 4)) || (rc = A((void **)&kv->attn, H * 4)) ||
      (rc = A((void **)&kv->gate, F * 4)) || (rc = A((void **)&kv->up, F * 4)) ||
      (rc = A((void **)&kv->act, F * 4)) || (rc = A((void **)&kv->logits, c.vocab_size * 4)) ||
      (rc = A((void **)&kv->scores, attention_scratch_words((int)c.num_attention_heads,
                                                            (int)c.head_dim, (int)max_seq) * 8)) ||
      (rc = A((void **)&kv->epoch, 64)) || (rc = A((void **)&kv->attn_err, 64)) ||
      (rc = A((void **)&kv->rope, max_seq * c.head_dim * 4)) || (rc = A((void **)&kv->pos, 64)) ||
      (rc = A((void **)&kv->tok_by_pos, (max_seq + 1) * 4)) || (rc = A((void **)&kv->next_token, 64)) ||
      (rc = A((void **)&kv->amax_key, 64)) || (rc = A((void **)&kv->done, 64)) ||
      (rc = A((void **)&kv->act_dig, fast_gemv_digits_size(F)))) {
    free_kv(kv);
    return rc;
  }
  hipError_t e = hipHostMalloc((void **)&kv->pinned, (max_seq + 2) * 4, hipHostMallocDefault);
  if (e != hipSuccess) {
    kv->pinned = nullptr;
    free_kv(kv);
    return set_error(LLRS_E_OOM, "hipHostMalloc failed: %s", hipGetErrorString(e));
  }
  std::vector<float> rope(max_seq * c.head_dim);
  rope_table(rope.data(), max_seq, c.head_dim, c.rope_theta);
  hipStream_t s = m->b->stream;
  e = hipMemcpyAsync(kv->rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice, s);
  // Zero-fill the state (the reference's vec![0.0; ...]); fill kernels via memset
  // outside any graph capture.
  if (e == hipSuccess) e = hipMemsetAsync(kv->k_cache, 0, L * max_seq * KV * 4, s);
  if (e == hipSuccess) e = hipMemsetAsync(kv->v_cache, 0, L * max_seq * KV * 4, s);
  if (e == hipSuccess) e = hipMemsetAsync(kv->logits, 0, c.vocab_size * 4, s);
  if (e == hipSuccess) e = hipMemsetAsync(kv->tok_by_pos, 0, (max_seq + 1) * 4, s);
  if (e == hipSuccess) e = hipMemsetAsync(kv->pos, 0, 64, s);
  if (e == hipSuccess) e = hipMemsetAsync(kv->amax_key, 0, 64, s);
  if (e == hipSuccess) e = hipMemsetAsync(kv->done, 0, 64, s);
  if (e == hipSuccess) e = hipMemsetAsync(kv->act_dig, 0, fast_gemv_digits_size(F), s);
  // Tag 0 is never a step's (the embedding advances the epoch first).
  if (e == hipSuccess)
    e = hipMemsetAsync(kv->scores, 0,
                       attention_scratch_words((int)c.num_attention_heads, (int)c.head_dim, (int)max_seq) * 8, s);
  if (e == hipSuccess) e = hipMemsetAsync(kv->epoch, 0, 64, s);
  if (e == hipSuccess) e = hipMemsetAsync(kv->attn_err, 0, 64, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    free_kv(kv);
    return set_error(LLRS_E_HIP, "KV cache init failed: %s", hipGetErrorString(e));
  }
  if ((rc = setup_persistent(m, kv)) != LLRS_OK) {
    free_kv(kv);
    return rc;
  }
  *out = kv;
  return LLRS_OK;
}

// Stages tok_by_pos[pos .. pos+n) = tokens and *pos = pos on the device.
static int stage_tokens(llrs_kv *kv, const uint32_t *tokens, size_t n, size_t pos) {
  hipStream_t s = kv->m->b->stream;
  LLRS_HIP(hipStreamSynchronize(s));  // the pinned staging buffer is free again
  memcpy(kv->pinned, tokens, n * 4);
  kv->pinned[n] = (uint32_t)pos;
  if (n) LLRS_HIP(hipMemcpyAsync(kv->tok_by_pos + pos, kv->pinned, n * 4, hipMemcpyHostToDevice, s));
  LLRS_HIP(hipMemcpyAsync(kv->pos, kv->pinned + n, 4, hipMemcpyHostToDevice, s));
  return LLRS_OK;
}

// Rows of one prefill chunk: bounds the prefill buffers (7B: ~114 MB).
constexpr size_t kPrefillRows = 512;

static bool prefill_tokenwise() {
  const char *e = getenv("LLRS_PREFILL_TOKENWISE");
  return e && *e && *e != '0';
}

static int prefill_buffers(llrs_kv *kv) {
  if (kv->pf_cap) return LLRS_OK;
  const llrs_model_config &c = kv->m->cfg;
  const size_t T = kv->max_seq_len < kPrefillRows ? kv->max_seq_len : kPrefillRows;
  const size_t H = c.hidden_size, F = c.intermediate_size, KV = c.kv_width;
  auto A = [&](void **p, size_t bytes) { return dev_alloc(kv->allocs, p, bytes); };
  LLRS_TRY(A((void **)&kv->pf_x, T * H * 4));
  LLRS_TRY(A((void **)&kv->pf_q, T * H * 4));
  LLRS_TRY(A((void **)&kv->pf_k, T * KV * 4));
  LLRS_TRY(A((void **)&kv->pf_v, T * KV * 4));
  LLRS_TRY(A((void **)&kv->pf_g, T * F * 4));
  LLRS_TRY(A((void **)&kv->pf_u, T * F * 4));
  LLRS_TRY(A((void **)&kv->pf_h, T * (H > F ? H : F) * 2));
  LLRS_TRY(A((void **)&kv->pf_hl, T * (H > F ? H : F) * 2));
  // Room for a Q4_K product's reads past the last sum (k/32 + 56 columns).
  kv->pf_ldxs = (int)(((H > F ? H : F) / 32 + 56 + 7) / 8 * 8);
  LLRS_TRY(A((void **)&kv->pf_xs, T * kv->pf_ldxs * 2));
  LLRS_TRY(A((void **)&kv->pf_xsl, T * kv->pf_ldxs * 2));
  LLRS_TRY(A((void **)&kv->pf_xs2, T * kv->pf_ldxs * 2));
  LLRS_TRY(A((void **)&kv->pf_xsl2, T * kv->pf_ldxs * 2));
  LLRS_HIP(hipMemset(kv->pf_xs, 0, T * kv->pf_ldxs * 2));
  LLRS_HIP(hipMemset(kv->pf_xsl, 0, T * kv->pf_ldxs * 2));
  LLRS_HIP(hipMemset(kv->pf_xs2, 0, T * kv->pf_ldxs * 2));
  LLRS_HIP(hipMemset(kv->pf_xsl2, 0, T * kv->pf_ldxs * 2));
  {
    const size_t np = (kv->max_seq_len + 15) / 16 * 16, n = np * KV * 2;
    kv->pf_kvf.positions = (int)np;
    kv->pf_kvf.kvw = (int)KV;
    LLRS_TRY(A((void **)&kv->pf_kvf.kh, n));
    LLRS_TRY(A((void **)&kv->pf_kvf.kl, n));
    LLRS_TRY(A((void **)&kv->pf_kvf.vh, n));
    LLRS_TRY(A((void **)&kv->pf_kvf.vl, n));
  }
  kv->pf_part_cap = prefill_split_scratch_floats();
  LLRS_TRY(A((void **)&kv->pf_part, kv->pf_part_cap * 4));
  kv->pf_cap = T;
  return LLRS_OK;
}

// Whether the Q4_K integer-code product will read activation sums of `ws`'s input.
static bool needs_xsum(std::initializer_list<const llrs_tensor *> ws) {
  if (!prefill_codes_enabled()) return false;
  for (const llrs_tensor *w : ws)
    if (w->type == LLRS_Q4_K) return true;
  return false;
}

// The activation sums of a/a_lo (k columns) that Q4_K products of this input read.
static int prefill_xsum(llrs_kv *kv, const f16 *a, const f16 *a_lo, int k, int T, hipStream_t s) {
  return launch_xsum_f16(a, a_lo, k, k, T, kv->pf_xs, kv->pf_xsl, kv->pf_ldxs, s);
}

// `xsum`: prefill_xsum has run on this input (Q4_K weights then take the integer-code product).
static int prefill_gemm(llrs_kv *kv, const llrs_tensor *w, const f16 *a, const f16 *a_lo, int lda,
                        float *c, int ldc, const float *bias, int T, bool accumulate, bool xsum,
                        hipStream_t s, bool xs2 = false) {
  PrefillGemmArgs g{};
  if (xsum && w->type == LLRS_Q4_K) {
    g.xs = xs2 ? kv->pf_xs2 : kv->pf_xs;
    g.xs_lo = xs2 ? kv->pf_xsl2 : kv->pf_xsl;
    g.ldxs = kv->pf_ldxs;
  }
  g.part = kv->pf_part;
  g.part_cap = kv->pf_part_cap;
  g.a = a;
  g.a_lo = a_lo;
  g.lda = lda;
  g.w = w->dev;
  g.type = w->type;
  g.row_bytes = (long)w->row_bytes;
  g.n = (int)w->rows;
  g.k = (int)w->cols;
  g.c = c;
  g.ldc = ldc;
  g.bias = bias;
  g.t = T;
  g.accumulate = accumulate ? 1 : 0;
  return launch_prefill_gemm(g, s);
}

// Whether gate and up run as one dual product with SwiGLU in its epilogue:
// both Q4_K on their codes, the FFN width a multiple of 64 (unless
// LLRS_PREFILL_DUAL=0, read per call, for comparisons).
static bool use_dual_gate_up(const DevLayer &L, int F) {
  const char *e = getenv("LLRS_PREFILL_DUAL");
  return !(e && strcmp(e, "0") == 0) && L.gate->type == LLRS_Q4_K && L.up->type == LLRS_Q4_K &&
         L.gate->row_bytes == L.up->row_bytes && F % 64 == 0 && prefill_codes_enabled();
}

// silu(gate) * up as f16 pairs into h/hl [T][F] (and, for a Q4_K ffn_down,
// its 32-column sums into pf_xs2) from the dual product over pf_h.
static int prefill_gate_up_dual(llrs_kv *kv, const DevLayer &L, int H, int F, int T, f16 *h, f16 *hl,
                                bool down_xs, hipStream_t s) {
  PrefillGemmArgs g{};
  g.part = kv->pf_part;
  g.part_cap = kv->pf_part_cap;
  g.a = kv->pf_h;
  g.a_lo = kv->pf_hl;
  g.lda = H;
  g.xs = kv->pf_xs;
  g.xs_lo = kv->pf_xsl;
  g.ldxs = kv->pf_ldxs;
  g.w = L.gate->dev;
  g.w2 = L.up->dev;
  g.type = LLRS_Q4_K;
  g.row_bytes = (long)L.gate->row_bytes;
  g.dual_rows = F;
  g.n = 2 * F;
  g.k = H;
  g.t = T;
  g.h = h;
  g.hl = hl;
  g.ldh = F;
  if (down_xs) {
    g.xso = kv->pf_xs2;
    g.xso_lo = kv->pf_xsl2;
    g.ldxso = kv->pf_ldxs;
  }
  return launch_prefill_gemm(g, s);
}

// Q, K (and V when it is Q4_K too) of one input as one segmented Q4_K product
// over pf_h (one launch and one split-K reduction instead of two or three):
// when they all run on their codes and every boundary is a multiple of 128
// rows (unless LLRS_PREFILL_QKV=0, read per call, for comparisons).  Returns
// whether V was included; sets *done when the product ran.
static int prefill_qkv_segmented(llrs_kv *kv, const DevLayer &L, int H, int KV, int T, bool &done,
                                 bool &with_v, hipStream_t s) {
  done = with_v = false;
  const char *e = getenv("LLRS_PREFILL_QKV");
  if ((e && strcmp(e, "0") == 0) || !prefill_codes_enabled() || L.q->type != LLRS_Q4_K ||
      L.k->type != LLRS_Q4_K || L.k->row_bytes != L.q->row_bytes || H % 128)
    return LLRS_OK;
  with_v = L.v->type == LLRS_Q4_K && L.v->row_bytes == L.q->row_bytes && KV % 128 == 0;
  PrefillGemmArgs g{};
  g.part = kv->pf_part;
  g.part_cap = kv->pf_part_cap;
  g.a = kv->pf_h;
  g.a_lo = kv->pf_hl;
  g.lda = H;
  g.xs = kv->pf_xs;
  g.xs_lo = kv->pf_xsl;
  g.ldxs = kv->pf_ldxs;
  g.w = L.q->dev;
  g.type = LLRS_Q4_K;
  g.row_bytes = (long)L.q->row_bytes;
  g.k = H;
  g.t = T;
  g.nseg = with_v ? 3 : 2;
  const llrs_tensor *w[3] = {L.q, L.k, L.v};
  float *c[3] = {kv->pf_q, kv->pf_k, kv->pf_v};
  const float *b[3] = {L.bq, L.bk, L.bv};
  const int rows[3] = {H, KV, KV}, ldc[3] = {H, KV, KV};
  g.seg_base[0] = 0;
  for (int i = 0; i < g.nseg; i++) {
    g.seg_w[i] = w[i]->dev;
    g.seg_c[i] = c[i];
    g.seg_ldc[i] = ldc[i];
    g.seg_bias[i] = b[i];
    g.seg_base[i + 1] = g.seg_base[i] + rows[i];
  }
  g.n = g.seg_base[g.nseg];
  g.c = kv->pf_q;  // unused with segments
  g.ldc = H;
  LLRS_TRY(launch_prefill_gemm(g, s));
  done = true;
  return LLRS_OK;
}

// CausalModel::prefill (src/architecture.rs:60-77) with the prompt's rows
// batched through each layer: MFMA dequant-GEMMs for the matrices, causal
// attention over the cache, then the decode step's fused LM head on the last
// row.  Tokens are staged in tok_by_pos[start, start + n); ends with *pos =
// start + n and the greedy token of the last logits at tok_by_pos[start + n],
// exactly as the token-by-token loop leaves them.
static int prefill_batched(llrs_model *m, llrs_kv *kv, size_t start, size_t n) {
  const llrs_model_config &c = m->cfg;
  hipStream_t s = m->b->stream;
  LLRS_TRY(prefill_buffers(kv));
  const int H = (int)c.hidden_size, F = (int)c.intermediate_size, KV = (int)c.kv_width;
  const int nh = (int)c.num_attention_heads, nkv = (int)c.num_key_value_heads, hd = (int)c.head_dim;
  const float eps = c.rms_norm_eps, scale = 1.0f / sqrtf((float)hd);
  const size_t layer_stride = kv->max_seq_len * c.kv_width;
  size_t last_rows = 0;
  for (size_t c0 = 0; c0 < n; c0 += kv->pf_cap) {
    const int T = (int)(n - c0 < kv->pf_cap ? n - c0 : kv->pf_cap);
    const int st = (int)(start + c0);
    LLRS_TRY(launch_embed_rows(m->embed, kv->tok_by_pos + st, T, kv->pf_x, s));
    for (size_t l = 0; l < c.num_hidden_layers; l++) {
      const DevLayer &L = m->layers[l];
      float *kc = kv->k_cache + l * layer_stride, *vc = kv->v_cache + l * layer_stride;
      bool xs = needs_xsum({L.q, L.k, L.v});
      LLRS_TRY(launch_rmsnorm_rows_f16(kv->pf_x, L.attn_norm, kv->pf_h, kv->pf_hl, T, H, eps, s,
                                       xs ? kv->pf_xs : nullptr, kv->pf_xsl, kv->pf_ldxs));
      bool qk_done = false, with_v = false;
      if (xs) LLRS_TRY(prefill_qkv_segmented(kv, L, H, KV, T, qk_done, with_v, s));
      if (!qk_done) {
        LLRS_TRY(prefill_gemm(kv, L.q, kv->pf_h, kv->pf_hl, H, kv->pf_q, H, L.bq, T, false, xs, s));
        LLRS_TRY(prefill_gemm(kv, L.k, kv->pf_h, kv->pf_hl, H, kv->pf_k, KV, L.bk, T, false, xs, s));
      }
      if (!with_v)
        LLRS_TRY(prefill_gemm(kv, L.v, kv->pf_h, kv->pf_hl, H, kv->pf_v, KV, L.bv, T, false, xs, s));
      LLRS_TRY(launch_rope_append(kv->pf_q, kv->pf_k, kv->pf_v, kv->rope, T, st, nh, nkv, hd, kc, vc, s));
      LLRS_TRY(launch_attention_rows(kv->pf_q, kc, vc, T, st, nh, nkv, hd, scale, kv->pf_h, kv->pf_hl, s,
                                     &kv->pf_kvf));
      xs = needs_xsum({L.o});
      if (xs) LLRS_TRY(prefill_xsum(kv, kv->pf_h, kv->pf_hl, H, T, s));
      LLRS_TRY(prefill_gemm(kv, L.o, kv->pf_h, kv->pf_hl, H, kv->pf_x, H, nullptr, T, true, xs, s));
      xs = needs_xsum({L.gate, L.up});
      LLRS_TRY(launch_rmsnorm_rows_f16(kv->pf_x, L.ffn_norm, kv->pf_h, kv->pf_hl, T, H, eps, s,
                                       xs ? kv->pf_xs : nullptr, kv->pf_xsl, kv->pf_ldxs));
      if (xs && use_dual_gate_up(L, F)) {
        // SwiGLU in the product's epilogue: its f16 pairs go to the gate/up
        // scratch (pf_h is this product's input), the sums to pf_xs2.
        f16 *h = reinterpret_cast<f16 *>(kv->pf_g), *hl = reinterpret_cast<f16 *>(kv->pf_u);
        xs = needs_xsum({L.down});
        LLRS_TRY(prefill_gate_up_dual(kv, L, H, F, T, h, hl, xs, s));
        LLRS_TRY(prefill_gemm(kv, L.down, h, hl, F, kv->pf_x, H, nullptr, T, true, xs, s, true));
      } else {
        LLRS_TRY(prefill_gemm(kv, L.gate, kv->pf_h, kv->pf_hl, H, kv->pf_g, F, nullptr, T, false, xs, s));
        LLRS_TRY(prefill_gemm(kv, L.up, kv->pf_h, kv->pf_hl, H, kv->pf_u, F, nullptr, T, false, xs, s));
        xs = needs_xsum({L.down});
        LLRS_TRY(launch_swiglu_f16(kv->pf_g, kv->pf_u, kv->pf_h, kv->pf_hl, (size_t)T * F, F, s,
                                   xs ? kv->pf_xs : nullptr, kv->pf_xsl, kv->pf_ldxs));
        LLRS_TRY(prefill_gemm(kv, L.down, kv->pf_h, kv->pf_hl, F, kv->pf_x, H, nullptr, T, true, xs, s));
      }
    }
    last_rows = (size_t)T;
  }
  LLRS_HIP(hipMemcpyAsync(kv->residual, kv->pf_x + (last_rows - 1) * H, (size_t)H * 4,
                          hipMemcpyDeviceToDevice, s));
  LLRS_TRY(launch_set_pos(kv->pos, (int)(start + n - 1), s));
  return launch_projection(m, kv, 0, P_LM_HEAD, s);
}

// The repeat window's length limit of llrs_sample.
constexpr size_t kMaxRecent = 65536;

// validate_sampling (src/engine.rs:327-338).
static int validate_sampling(const llrs_sampling *opts) {
  if (!std::isfinite(opts->temperature) || opts->temperature < 0.0f)
    return set_error(LLRS_E_INVALID, "temperature must be finite and non-negative");
  if (!std::isfinite(opts->top_p) || !(0.0f < opts->top_p && opts->top_p <= 1.0f))
    return set_error(LLRS_E_INVALID, "top_p must be in (0, 1]");
  if (!std::isfinite(opts->repetition_penalty) || opts->repetition_penalty <= 0.0f)
    return set_error(LLRS_E_INVALID, "repetition_penalty must be finite and positive");
  return LLRS_OK;
}

// Arguments of llrs_sample: the options, the window and the draw.
static int validate_sample(llrs_kv *kv, const llrs_sampling *opts, const uint32_t *recent,
                           size_t n_recent, float uniform, uint32_t *out_token) {
  if (!kv || !opts || !out_token || (n_recent && !recent))
    return set_error(LLRS_E_INVALID, "kv/opts/recent/out is NULL");
  LLRS_TRY(validate_sampling(opts));
  if (!std::isfinite(uniform) || uniform < 0.0f || uniform >= 1.0f)
    return set_error(LLRS_E_INVALID, "the uniform draw must be in [0, 1)");
  if (n_recent > kMaxRecent) return set_error(LLRS_E_INVALID, "repeat window %zu > %zu", n_recent, kMaxRecent);
  return LLRS_OK;
}

// sample_current_logits over the cache's logits with scratch w (the device is current).
static int sample_with(llrs_kv *kv, const llrs_sampling *opts, const uint32_t *recent, size_t n_recent,
                       float uniform, SampleScratch &w, uint32_t *out_token) {
  llrs_model *m = kv->m;
  hipStream_t s = m->b->stream;
  const int V = (int)m->cfg.vocab_size;
  if (n_recent) LLRS_HIP(hipMemcpyAsync(w.recent, recent, n_recent * 4, hipMemcpyHostToDevice, s));
  const SampleParams p{opts->temperature, (int)std::min<uint32_t>(opts->top_k, (uint32_t)V), opts->top_p,
                       opts->repetition_penalty};
  LLRS_TRY(launch_sample(kv->logits, V, p, (int)n_recent, uniform, w, s));
  LLRS_HIP(hipMemcpyAsync(kv->pinned, w.token, 4, hipMemcpyDeviceToHost, s));
  LLRS_HIP(hipStreamSynchronize(s));
  *out_token = kv->pinned[0];
  return LLRS_OK;
}

}  // namespace llrs

using namespace llrs;

extern "C" {

int llrs_model_load_gguf(llrs_backend *b, const char *path, int quantization, llrs_model **out) {
  clear_error();
  if (!b || !path || !out) return set_error(LLRS_E_INVALID, "backend/path/out is NULL");
  *out = nullptr;
  if (quantization < LLRS_QUANT_NONE || quantization > LLRS_QUANT_Q4KM)
    return set_error(LLRS_E_INVALID, "unknown quantization %d", quantization);
  LLRS_HIP(hipSetDevice(b->device));
  return load_gguf_impl(b, path, quantization, out);
}

int llrs_model_load_safetensors(llrs_backend *b, const char *model_dir, int quantization,
                                llrs_model **out) {
  clear_error();
  if (!b || !model_dir || !out) return set_error(LLRS_E_INVALID, "backend/model_dir/out is NULL");
  *out = nullptr;
  if (quantization < LLRS_QUANT_NONE || quantization > LLRS_QUANT_Q4KM)
    return set_error(LLRS_E_INVALID, "unknown quantization %d", quantization);
  LLRS_HIP(hipSetDevice(b->device));
  return load_safetensors_impl(b, model_dir, quantization, out);
}

int llrs_model_load(llrs_backend *b, const char *path, int quantization, llrs_model **out) {
  clear_error();
  if (!b || !path || !out) return set_error(LLRS_E_INVALID, "backend/path/out is NULL");
  *out = nullptr;
  int format = 0;
  std::string resolved;
  LLRS_TRY(detect_model_format(path, format, resolved));
  return format == LLRS_FORMAT_GGUF ? llrs_model_load_gguf(b, resolved.c_str(), quantization, out)
                                    : llrs_model_load_safetensors(b, resolved.c_str(), quantization, out);
}

// Releases the caller's handle; caches made from the model keep it alive
// until they are freed.
void llrs_model_free(llrs_model *m) { free_model(m); }

int llrs_model_config_get(const llrs_model *m, llrs_model_config *out) {
  clear_error();
  if (!m || !out) return set_error(LLRS_E_INVALID, "model/out is NULL");
  *out = m->cfg;
  return LLRS_OK;
}

size_t llrs_model_weight_bytes(const llrs_model *m) { return m ? m->weight_bytes : 0; }

int llrs_synth_write_gguf(const llrs_synth_config *cfg, const char *path) {
  clear_error();
  if (!cfg || !path) return set_error(LLRS_E_INVALID, "cfg/path is NULL");
  llrs_model_config c;
  LLRS_TRY(synth_config_to_model(*cfg, c));
  auto specs = synth_specs(*cfg);
  std::vector<GgufOutTensor> tensors(specs.size());
  for (size_t i = 0; i < specs.size(); i++) LLRS_TRY(synth_tensor(*cfg, i, specs[i], tensors[i]));
  GgufWriter w;
  w.add_str("general.architecture", "qwen2");
  w.add_u32("general.alignment", 32);
  w.add_u32("qwen2.embedding_length", (uint32_t)c.hidden_size);
  w.add_u32("qwen2.feed_forward_length", (uint32_t)c.intermediate_size);
  w.add_u32("qwen2.attention.head_count", (uint32_t)c.num_attention_heads);
  w.add_u32("qwen2.attention.head_count_kv", (uint32_t)c.num_key_value_heads);
  w.add_u32("qwen2.block_count", (uint32_t)c.num_hidden_layers);
  w.add_u32("qwen2.context_length", (uint32_t)c.max_position_embeddings);
  w.add_f32("qwen2.attention.layer_norm_rms_epsilon", c.rms_norm_eps);
  w.add_f32("qwen2.rope.freq_base", c.rope_theta);
  return w.write(path, tensors);
}

int llrs_model_synthetic(llrs_backend *b, const llrs_synth_config *cfg, llrs_model **out) {
  clear_error();
  if (!b || !cfg || !out) return set_error(LLRS_E_INVALID, "backend/cfg/out is NULL");
  *out = nullptr;
  LLRS_HIP(hipSetDevice(b->device));
  llrs_model_config c;
  LLRS_TRY(synth_config_to_model(*cfg, c));
  auto specs = synth_specs(*cfg);
  llrs_model *m = model_new(b);
  if (!m) return set_error(LLRS_E_OOM, "out of host memory");
  m->cfg = c;
  // Generated and encoded on the GPU with the host generator's functions, so
  // the bytes equal those llrs_synth_write_gguf writes for the same config.
  auto find = [&](const std::string &name) -> long {
    for (size_t i = 0; i < specs.size(); i++)
      if (specs[i].name == name) return (long)i;
    return -1;
  };
  MatFn mat = [&](const std::string &name, size_t rows, size_t cols, llrs_tensor **t) -> int {
    long i = find(name);
    if (i < 0) return set_error(LLRS_E_INVALID, "missing tensor %s", name.c_str());
    uint32_t ty = synth_type(*cfg, specs[i]);
    LLRS_TRY(tensor_alloc(b, ty, rows, cols, t));
    int rc = launch_synth_encode(ty, enc::tensor_key(cfg->seed, (uint64_t)i), rows, cols,
                                 cfg->weight_std, false, (*t)->dev, (*t)->row_bytes, b->stream);
    if (rc != LLRS_OK) {
      llrs_tensor_free(*t);
      *t = nullptr;
    }
    return rc;
  };
  VecFn vec = [&](const std::string &name, size_t len, bool, float *dst) -> int {
    long i = find(name);
    if (i < 0) return set_error(LLRS_E_INVALID, "missing tensor %s", name.c_str());
    return launch_synth_encode(LLRS_F32, enc::tensor_key(cfg->seed, (uint64_t)i), 1, len,
                               cfg->weight_std, specs[i].kind == SynthSpec::GAIN,
                               (uint8_t *)dst, len * 4, b->stream);
  };
  int rc = build_model(m, mat, vec);
  if (rc == LLRS_OK) {
    hipError_t e = hipStreamSynchronize(b->stream);
    if (e != hipSuccess) rc = set_error(LLRS_E_HIP, "synthetic generation failed: %s", hipGetErrorString(e));
  }
  if (rc != LLRS_OK) {
    free_model(m);
    return rc;
  }
  *out = m;
  return LLRS_OK;
}

int llrs_model_export_gguf(const llrs_model *m, const char *path) {
  clear_error();
  if (!m || !path) return set_error(LLRS_E_INVALID, "model/path is NULL");
  LLRS_HIP(hipSetDevice(m->b->device));
  const llrs_model_config &c = m->cfg;
  GgufWriter w;
  w.add_str("general.architecture", "qwen2");
  w.add_u32("general.alignment", 32);
  w.add_u32("qwen2.embedding_length", (uint32_t)c.hidden_size);
  w.add_u32("qwen2.feed_forward_length", (uint32_t)c.intermediate_size);
  w.add_u32("qwen2.attention.head_count", (uint32_t)c.num_attention_heads);
  w.add_u32("qwen2.attention.head_count_kv", (uint32_t)c.num_key_value_heads);
  w.add_u32("qwen2.block_count", (uint32_t)c.num_hidden_layers);
  w.add_u32("qwen2.context_length", (uint32_t)c.max_position_embeddings);
  w.add_f32("qwen2.attention.layer_norm_rms_epsilon", c.rms_norm_eps);
  w.add_f32("qwen2.rope.freq_base", c.rope_theta);
  std::vector<GgufOutTensor> infos;
  std::vector<size_t> sizes;
  for (const auto &r : m->refs) {
    GgufOutTensor t;
    t.name = r.name;
    if (r.mat) {
      t.dims = {r.mat->cols, r.mat->rows};
      t.type = r.mat->type;
      sizes.push_back(r.mat->nbytes);
    } else {
      t.dims = {r.len};
      t.type = LLRS_F32;
      sizes.push_back(r.len * 4);
    }
    infos.push_back(t);
  }
  return w.write_streamed(path, infos, sizes, [&](size_t i, std::vector<uint8_t> &buf) -> int {
    const TensorRef &r = m->refs[i];
    buf.resize(sizes[i]);
    const void *src = r.mat ? (const void *)r.mat->dev : (const void *)r.vec;
    LLRS_HIP(hipMemcpyAsync(buf.data(), src, sizes[i], hipMemcpyDeviceToHost, m->b->stream));
    LLRS_HIP(hipStreamSynchronize(m->b->stream));
    return LLRS_OK;
  });
}

int llrs_kv_create(llrs_model *m, size_t max_seq_len, llrs_kv **out) {
  clear_error();
  if (!m || !out) return set_error(LLRS_E_INVALID, "model/out is NULL");
  *out = nullptr;
  LLRS_HIP(hipSetDevice(m->b->device));
  return kv_create_impl(m, max_seq_len, out);
}

void llrs_kv_free(llrs_kv *kv) { free_kv(kv); }

int llrs_kv_reset(llrs_kv *kv) {
  clear_error();
  if (!kv) return set_error(LLRS_E_INVALID, "kv is NULL");
  // KVCache::reset (src/cache.rs:55-57) keeps the rows (positions are written
  // before they are read); only the device's wait flags start over.
  LLRS_HIP(hipSetDevice(kv->m->b->device));
  return clear_wait_flags(kv);
}

int llrs_kv_debug_set_wait_flag(llrs_kv *kv, int which) {
  clear_error();
  if (!kv) return set_error(LLRS_E_INVALID, "kv is NULL");
  if (which != 0 && which != 1) return set_error(LLRS_E_INVALID, "unknown wait flag %d", which);
  if (which == 0 && !kv->p_err) return set_error(LLRS_E_INVALID, "the cache has no persistent decode");
  LLRS_HIP(hipSetDevice(kv->m->b->device));
  const unsigned one = 1;
  LLRS_HIP(hipMemcpy(which == 0 ? kv->p_err : kv->attn_err, &one, 4, hipMemcpyHostToDevice));
  return LLRS_OK;
}

int llrs_kv_decode_path(const llrs_kv *kv) { return kv && kv->p_layers ? 1 : 0; }

int llrs_forward_token(llrs_model *m, llrs_kv *kv, uint32_t token, size_t pos, int logits_mode) {
  clear_error();
  if (!m || !kv || kv->m != m) return set_error(LLRS_E_INVALID, "model/kv mismatch");
  if (token >= m->cfg.vocab_size)
    return set_error(LLRS_E_INVALID, "token id %u is outside vocabulary", token);
  if (pos >= kv->max_seq_len)
    return set_error(LLRS_E_INVALID, "position %zu exceeds configured context %zu", pos,
                     kv->max_seq_len);
  if (logits_mode != LLRS_LOGITS_SKIP && logits_mode != LLRS_LOGITS_COMPUTE)
    return set_error(LLRS_E_INVALID, "unknown logits mode %d", logits_mode);
  LLRS_HIP(hipSetDevice(m->b->device));
  LLRS_TRY(stage_tokens(kv, &token, 1, pos));
  LLRS_TRY(run_step(m, kv, logits_mode, pos));
  LLRS_HIP(hipStreamSynchronize(m->b->stream));
  return check_persistent(kv);
}

int llrs_prefill(llrs_model *m, llrs_kv *kv, const uint32_t *tokens, size_t n, size_t start_pos) {
  clear_error();
  if (!m || !kv || kv->m != m) return set_error(LLRS_E_INVALID, "model/kv mismatch");
  if (n == 0) return set_error(LLRS_E_INVALID, "prefill requires at least one token");
  if (!tokens) return set_error(LLRS_E_INVALID, "tokens is NULL");
  for (size_t i = 0; i < n; i++) {
    if (tokens[i] >= m->cfg.vocab_size)
      return set_error(LLRS_E_INVALID, "token id %u is outside vocabulary", tokens[i]);
    if (start_pos + i >= kv->max_seq_len)
      return set_error(LLRS_E_INVALID, "position %zu exceeds configured context %zu",
                       start_pos + i, kv->max_seq_len);
  }
  LLRS_HIP(hipSetDevice(m->b->device));
  LLRS_TRY(stage_tokens(kv, tokens, n, start_pos));
  if (n >= 2 && !prefill_tokenwise()) {
    LLRS_TRY(prefill_batched(m, kv, start_pos, n));
  } else {
    for (size_t i = 0; i < n; i++)
      LLRS_TRY(run_step(m, kv, i + 1 == n ? LLRS_LOGITS_COMPUTE : LLRS_LOGITS_SKIP, start_pos + i));
  }
  LLRS_HIP(hipStreamSynchronize(m->b->stream));
  return check_persistent(kv);
}

int llrs_decode_greedy(llrs_model *m, llrs_kv *kv, size_t start_pos, size_t n_steps,
                       uint32_t *out_tokens) {
  clear_error();
  if (!m || !kv || kv->m != m) return set_error(LLRS_E_INVALID, "model/kv mismatch");
  if (n_steps == 0) return LLRS_OK;
  if (!out_tokens) return set_error(LLRS_E_INVALID, "out_tokens is NULL");
  if (start_pos + n_steps > kv->max_seq_len)
    return set_error(LLRS_E_INVALID, "benchmark token counts exceed context");
  LLRS_HIP(hipSetDevice(m->b->device));
  hipStream_t s = m->b->stream;
  LLRS_TRY(stage_tokens(kv, nullptr, 0, start_pos));
  // token = argmax(current logits) for position start_pos; nothing advances.
  LLRS_TRY(launch_argmax(kv->logits, (int)m->cfg.vocab_size, kv->pos, (int)kv->max_seq_len,
                         kv->tok_by_pos, kv->next_token, 0, s));
  // The device's wait flags are checked every kCheckEvery steps, so a
  // failed step stops the loop within that many steps.
  constexpr size_t kCheckEvery = 64;
  for (size_t i = 0; i < n_steps; i++) {
    LLRS_TRY(run_step(m, kv, LLRS_LOGITS_COMPUTE, start_pos + i));
    if ((i + 1) % kCheckEvery == 0 && i + 1 < n_steps) {
      LLRS_HIP(hipStreamSynchronize(s));
      LLRS_TRY(check_persistent(kv));
    }
  }
  LLRS_HIP(hipMemcpyAsync(kv->pinned, kv->tok_by_pos + start_pos, n_steps * 4,
                          hipMemcpyDeviceToHost, s));
  LLRS_HIP(hipStreamSynchronize(s));
  memcpy(out_tokens, kv->pinned, n_steps * 4);
  return check_persistent(kv);
}

int llrs_argmax(llrs_kv *kv, uint32_t *out_token) {
  clear_error();
  if (!kv || !out_token) return set_error(LLRS_E_INVALID, "kv/out is NULL");
  llrs_model *m = kv->m;
  LLRS_HIP(hipSetDevice(m->b->device));
  hipStream_t s = m->b->stream;
  // Evaluate into the spare slot after the context so no state changes.
  LLRS_HIP(hipStreamSynchronize(s));
  uint32_t saved = 0;
  LLRS_HIP(hipMemcpy(&saved, kv->pos, 4, hipMemcpyDeviceToHost));
  LLRS_TRY(stage_tokens(kv, nullptr, 0, kv->max_seq_len));
  LLRS_TRY(launch_argmax(kv->logits, (int)m->cfg.vocab_size, kv->pos, (int)kv->max_seq_len,
                         kv->tok_by_pos, kv->next_token, 0, s));
  LLRS_HIP(hipMemcpyAsync(kv->pinned, kv->next_token, 4, hipMemcpyDeviceToHost, s));
  LLRS_HIP(hipStreamSynchronize(s));
  *out_token = kv->pinned[0];
  LLRS_TRY(stage_tokens(kv, nullptr, 0, saved));
  LLRS_HIP(hipStreamSynchronize(s));
  return LLRS_OK;
}

int llrs_sample(llrs_kv *kv, const llrs_sampling *opts, const uint32_t *recent, size_t n_recent,
                float uniform, uint32_t *out_token) {
  clear_error();
  LLRS_TRY(validate_sample(kv, opts, recent, n_recent, uniform, out_token));
  llrs_model *m = kv->m;
  LLRS_HIP(hipSetDevice(m->b->device));
  const int V = (int)m->cfg.vocab_size;
  SampleScratch &w = kv->sample;
  if (!w.n) {
    auto A = [&](void **p, size_t bytes) { return dev_alloc(kv->allocs, p, bytes); };
    w.tmp_bytes = sample_sort_bytes(V);
    LLRS_TRY(A((void **)&w.keys, (size_t)V * 4));
    LLRS_TRY(A((void **)&w.keys_sorted, (size_t)V * 4));
    LLRS_TRY(A((void **)&w.idx, (size_t)V * 4));
    LLRS_TRY(A((void **)&w.idx_sorted, (size_t)V * 4));
    LLRS_TRY(A((void **)&w.recent, kMaxRecent * 4));
    LLRS_TRY(A((void **)&w.token, 64));
    LLRS_TRY(A(&w.tmp, w.tmp_bytes ? w.tmp_bytes : 1));
    w.max_recent = (int)kMaxRecent;
    w.n = V;
  }
  return sample_with(kv, opts, recent, n_recent, uniform, w, out_token);
}

int llrs_sample_noalloc(llrs_kv *kv, const llrs_sampling *opts, const uint32_t *recent,
                        size_t n_recent, float uniform, uint32_t *out_token) {
  clear_error();
  LLRS_TRY(validate_sample(kv, opts, recent, n_recent, uniform, out_token));
  if (kv->m->cfg.vocab_size > (size_t)kNoAllocMaxVocab)
    return set_error(LLRS_E_INVALID, "llrs_sample_noalloc: vocabulary %zu exceeds its limit of %d tokens",
                     kv->m->cfg.vocab_size, kNoAllocMaxVocab);
  if (n_recent > (size_t)kNoAllocMaxRecent)
    return set_error(LLRS_E_INVALID, "llrs_sample_noalloc: repeat window %zu exceeds its limit of %d tokens",
                     n_recent, kNoAllocMaxRecent);
  LLRS_HIP(hipSetDevice(kv->m->b->device));
  SampleScratch w;
  LLRS_TRY(sample_noalloc_scratch(w));
  return sample_with(kv, opts, recent, n_recent, uniform, w, out_token);
}

int llrs_generate(llrs_model *m, llrs_kv *kv, const uint32_t *prompt, size_t n_prompt,
                  const llrs_sampling *opts, size_t repeat_last_n, const uint32_t *eos_ids,
                  size_t n_eos, size_t max_new_tokens, const float *uniforms, uint32_t *out_tokens,
                  llrs_generation *result) {
  clear_error();
  if (!m || !kv || kv->m != m) return set_error(LLRS_E_INVALID, "model/kv mismatch");
  if (!opts || !result || (n_eos && !eos_ids) || (max_new_tokens && !out_tokens))
    return set_error(LLRS_E_INVALID, "opts/result/eos_ids/out_tokens is NULL");
  *result = llrs_generation{};
  if (n_prompt == 0 || !prompt) return set_error(LLRS_E_INVALID, "the prompt is empty");
  if (n_prompt >= kv->max_seq_len)
    return set_error(LLRS_E_INVALID, "prompt has %zu tokens, but context is %zu", n_prompt,
                     kv->max_seq_len);
  // validate_sampling (src/engine.rs:327-338) before anything runs, and the
  // window and draws this loop needs.
  LLRS_TRY(validate_sampling(opts));
  if (repeat_last_n > kMaxRecent)
    return set_error(LLRS_E_INVALID, "repeat window %zu > %zu", repeat_last_n, kMaxRecent);
  if (opts->temperature > 0.0f && max_new_tokens && !uniforms)
    return set_error(LLRS_E_INVALID, "sampling with temperature > 0 needs one uniform draw per token");
  // reset(), then the last repeat_last_n prompt tokens seed the window (src/engine.rs:136-143).
  LLRS_TRY(llrs_kv_reset(kv));
  std::vector<uint32_t> recent;
  auto remember = [&](uint32_t t) {  // InferenceEngine::remember (src/engine.rs:243-251)
    if (!repeat_last_n) return;
    recent.push_back(t);
    if (recent.size() > repeat_last_n) recent.erase(recent.begin());
  };
  for (size_t i = n_prompt > repeat_last_n ? n_prompt - repeat_last_n : 0; i < n_prompt; i++)
    remember(prompt[i]);
  using clock = std::chrono::steady_clock;
  const auto t0 = clock::now();
  LLRS_TRY(llrs_prefill(m, kv, prompt, n_prompt, 0));
  const auto t1 = clock::now();
  const size_t count = std::min(max_new_tokens, kv->max_seq_len - n_prompt);
  size_t gen = 0;
  for (size_t i = 0; i < count; i++) {
    uint32_t tok = 0;
    LLRS_TRY(llrs_sample(kv, opts, recent.data(), recent.size(), uniforms ? uniforms[i] : 0.0f, &tok));
    out_tokens[gen++] = tok;
    remember(tok);
    if (std::find(eos_ids, eos_ids + n_eos, tok) != eos_ids + n_eos) {
      result->stopped_on_eos = 1;
      break;
    }
    LLRS_TRY(llrs_forward_token(m, kv, tok, n_prompt + gen - 1, LLRS_LOGITS_COMPUTE));
  }
  const auto t2 = clock::now();
  result->prompt_tokens = n_prompt;
  result->generated_tokens = gen;
  result->prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
  result->decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
  return LLRS_OK;
}

int llrs_read_logits(llrs_kv *kv, float *out, size_t n) {
  clear_error();
  if (!kv || !out) return set_error(LLRS_E_INVALID, "kv/out is NULL");
  if (n != kv->m->cfg.vocab_size)
    return set_error(LLRS_E_INVALID, "logits length %zu != vocab %zu", n, kv->m->cfg.vocab_size);
  LLRS_HIP(hipSetDevice(kv->m->b->device));
  LLRS_HIP(hipMemcpyAsync(out, kv->logits, n * 4, hipMemcpyDeviceToHost, kv->m->b->stream));
  LLRS_HIP(hipStreamSynchronize(kv->m->b->stream));
  return LLRS_OK;
}

int llrs_read_kv(llrs_kv *kv, size_t layer, int which, float *out, size_t n) {
  clear_error();
  if (!kv || !out) return set_error(LLRS_E_INVALID, "kv/out is NULL");
  const llrs_model_config &c = kv->m->cfg;
  if (layer >= c.num_hidden_layers) return set_error(LLRS_E_INVALID, "KV layer out of bounds");
  size_t per = kv->max_seq_len * c.kv_width;
  if (n > per) return set_error(LLRS_E_INVALID, "read of %zu floats exceeds the layer (%zu)", n, per);
  const float *src = (which ? kv->v_cache : kv->k_cache) + layer * per;
  LLRS_HIP(hipSetDevice(kv->m->b->device));
  LLRS_HIP(hipMemcpyAsync(out, src, n * 4, hipMemcpyDeviceToHost, kv->m->b->stream));
  LLRS_HIP(hipStreamSynchronize(kv->m->b->stream));
  return LLRS_OK;
}

int llrs_read_tokens(llrs_kv *kv, size_t start, size_t n, uint32_t *out) {
  clear_error();
  if (!kv || (n && !out)) return set_error(LLRS_E_INVALID, "kv/out is NULL");
  if (start > kv->max_seq_len + 1 || n > kv->max_seq_len + 1 - start)
    return set_error(LLRS_E_INVALID, "token range [%zu, %zu) exceeds the context", start, start + n);
  if (!n) return LLRS_OK;
  LLRS_HIP(hipSetDevice(kv->m->b->device));
  LLRS_HIP(hipMemcpyAsync(out, kv->tok_by_pos + start, n * 4, hipMemcpyDeviceToHost, kv->m->b->stream));
  LLRS_HIP(hipStreamSynchronize(kv->m->b->stream));
  return LLRS_OK;
}

int llrs_profile_projection(llrs_model *m, llrs_kv *kv, int which, int iters, double *avg_us,
                            size_t *bytes_per_launch) {
  clear_error();
  if (!m || !kv || kv->m != m || !avg_us) return set_error(LLRS_E_INVALID, "bad arguments");
  if (which < 0 || which > P_LAYERS) return set_error(LLRS_E_INVALID, "unknown projection %d", which);
  if (iters < 1) return set_error(LLRS_E_INVALID, "iters must be positive");
  LLRS_HIP(hipSetDevice(m->b->device));
  hipStream_t s = m->b->stream;
  // The LM-head launch advances the device position; keep the caller's.
  int saved_pos = 0;
  LLRS_HIP(hipStreamSynchronize(s));
  LLRS_HIP(hipMemcpy(&saved_pos, kv->pos, 4, hipMemcpyDeviceToHost));
  struct Restore {
    llrs_kv *kv;
    int pos;
    ~Restore() {
      (void)hipStreamSynchronize(kv->m->b->stream);
      (void)hipMemcpy(kv->pos, &pos, 4, hipMemcpyHostToDevice);
    }
  } restore{kv, saved_pos};
  if (which == P_LAYERS) {
    // Each round: the embedding (outside the timed span), then the layers
    // between two events.  Rounds recompute the same position, so they are
    // idempotent.
    std::vector<hipEvent_t> ev(2 * (size_t)iters + 2, nullptr);
    int rc = LLRS_OK;
    hipError_t e = hipSuccess;
    for (auto &x : ev)
      if (e == hipSuccess) e = hipEventCreate(&x);
    for (int it = -1; it < iters && rc == LLRS_OK && e == hipSuccess; it++) {  // round -1 warms
      rc = enqueue_embed(m, kv);
      if (rc == LLRS_OK) e = hipEventRecord(ev[2 * (it + 1)], s);
      if (rc == LLRS_OK && e == hipSuccess) rc = enqueue_layers(m, kv, persistent_long_items((size_t)saved_pos, (int)m->cfg.num_attention_heads));
      if (rc == LLRS_OK && e == hipSuccess) e = hipEventRecord(ev[2 * (it + 1) + 1], s);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    double total = 0;
    for (int it = 0; it < iters && e == hipSuccess; it++) {
      float ms = 0.f;
      e = hipEventElapsedTime(&ms, ev[2 * (it + 1)], ev[2 * (it + 1) + 1]);
      total += ms;
    }
    for (auto &x : ev)
      if (x) (void)hipEventDestroy(x);
    LLRS_TRY(rc);
    if (e != hipSuccess) return set_error(LLRS_E_HIP, "event timing failed: %s", hipGetErrorString(e));
    LLRS_TRY(check_persistent(kv));
    *avg_us = 1000.0 * total / iters;
    if (bytes_per_launch) *bytes_per_launch = projection_bytes(m, which);
    return LLRS_OK;
  }
  size_t layers = which == P_LM_HEAD ? 1 : m->cfg.num_hidden_layers;
  hipEvent_t e0, e1;
  LLRS_HIP(hipEventCreate(&e0));
  LLRS_HIP(hipEventCreate(&e1));
  int rc = LLRS_OK;
  for (size_t l = 0; l < layers && rc == LLRS_OK; l++) rc = launch_projection(m, kv, l, which, s);  // warm
  hipError_t e = hipEventRecord(e0, s);
  for (int it = 0; it < iters && rc == LLRS_OK && e == hipSuccess; it++)
    for (size_t l = 0; l < layers && rc == LLRS_OK; l++) rc = launch_projection(m, kv, l, which, s);
  if (e == hipSuccess) e = hipEventRecord(e1, s);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  LLRS_TRY(rc);
  if (e != hipSuccess) return set_error(LLRS_E_HIP, "event timing failed: %s", hipGetErrorString(e));
  *avg_us = 1000.0 * (double)ms / (double)(iters * layers);
  if (bytes_per_launch) *bytes_per_launch = projection_bytes(m, which);
  return LLRS_OK;
}

}  // extern "C"
