/*
 * CPU ORACLE -- test infrastructure only (see oracle.h).
 *
 * Restates the reference's model path in plain C:
 *   GGUF reader      src/gguf.rs:77-258, 339-369 (v2/v3, metadata types 0-12,
 *                    tensor table, alignment, eager range validation)
 *   GGUF loader      src/loader.rs:233-399, 497-534 (qwen2.* metadata -> config,
 *                    tensor-name map, missing Q/K/V bias -> zeros, tied head)
 *   config checks    src/config.rs:48-89
 *   KV cache/buffers src/cache.rs:13-101
 *   forward_impl     src/model.rs:135-271 (RMSNorm 65-73, RoPE 76-95,
 *                    softmax 298-313)
 *   prefill          src/architecture.rs:60-77
 *   argmax           src/engine.rs:233-241
 *   decode loop      src/engine.rs:205-216
 *
 * Pinned by: tests/test_oracle_model.py -- a tiny Qwen2 built from the same
 * dequantized weights in Hugging Face transformers' Qwen2ForCausalLM (an
 * independent implementation of the architecture; float64), plus closed forms
 * (pos 0: RoPE is the identity and attention returns the V row; the softmax
 * uniform fallback; constant-vector RMSNorm) and the reference's minimal GGUF
 * v3 file (src/gguf.rs:382-418).
 */
#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "oracle.h"

static __thread char g_err[512];
const char *oq_last_error(void) { return g_err; }
static int fail(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return -1;
}

/* ---------------------------------- GGUF ---------------------------------- */

typedef struct {
  char *key;
  int kind; /* 0 u64, 1 i64, 2 f64, 3 bool, 4 string, 5 array */
  uint64_t u;
  int64_t i;
  double f;
  char *s;
} gg_meta;

typedef struct {
  char *name;
  uint32_t ndim;
  uint64_t dims[4];
  uint32_t type;
  uint64_t offset;
} gg_tensor;

typedef struct {
  uint8_t *map;
  size_t size;
  uint32_t version;
  gg_meta *meta;
  size_t n_meta;
  gg_tensor *tensors;
  size_t n_tensors;
  size_t data_offset;
} gguf;

typedef struct {
  const uint8_t *d;
  size_t n, pos;
  int err;
} rdr;

static const uint8_t *take(rdr *r, size_t len) {
  if (r->err || r->pos > r->n || len > r->n - r->pos) {
    if (!r->err) fail("truncated GGUF file at byte %zu", r->pos);
    r->err = 1;
    return NULL;
  }
  const uint8_t *p = r->d + r->pos;
  r->pos += len;
  return p;
}
static uint64_t rd_le(rdr *r, int n) {
  const uint8_t *p = take(r, (size_t)n);
  uint64_t v = 0;
  if (!p) return 0;
  for (int i = n - 1; i >= 0; i--) v = (v << 8) | p[i];
  return v;
}
static char *rd_string(rdr *r) {
  uint64_t len = rd_le(r, 8);
  if (r->err) return NULL;
  if (len > (1u << 30)) {
    fail("unreasonable GGUF string length %llu", (unsigned long long)len);
    r->err = 1;
    return NULL;
  }
  const uint8_t *p = take(r, (size_t)len);
  if (!p) return NULL;
  char *s = (char *)malloc((size_t)len + 1);
  memcpy(s, p, (size_t)len);
  s[len] = 0;
  return s;
}

/* metadata_value (src/gguf.rs:339-369). */
static int rd_meta_value(rdr *r, uint32_t ty, gg_meta *m) {
  switch (ty) {
    case 0: m->kind = 0; m->u = rd_le(r, 1); break;
    case 1: m->kind = 1; m->i = (int8_t)rd_le(r, 1); break;
    case 2: m->kind = 0; m->u = rd_le(r, 2); break;
    case 3: m->kind = 1; m->i = (int16_t)rd_le(r, 2); break;
    case 4: m->kind = 0; m->u = rd_le(r, 4); break;
    case 5: m->kind = 1; m->i = (int32_t)rd_le(r, 4); break;
    case 6: {
      uint32_t b = (uint32_t)rd_le(r, 4);
      float f;
      memcpy(&f, &b, 4);
      m->kind = 2;
      m->f = f;
      break;
    }
    case 7: m->kind = 3; m->u = rd_le(r, 1) != 0; break;
    case 8: m->kind = 4; m->s = rd_string(r); break;
    case 9: {
      uint32_t et = (uint32_t)rd_le(r, 4);
      if (r->err) return -1;
      if (et == 9) return fail("nested GGUF arrays are not supported by the format");
      uint64_t len = rd_le(r, 8);
      if (r->err) return -1;
      if (len > 100000000ull) return fail("unreasonable GGUF array length %llu", (unsigned long long)len);
      for (uint64_t k = 0; k < len; k++) {
        gg_meta tmp = {0};
        if (rd_meta_value(r, et, &tmp)) return -1;
        free(tmp.s);
      }
      m->kind = 5;
      m->u = len;
      break;
    }
    case 10: m->kind = 0; m->u = rd_le(r, 8); break;
    case 11: m->kind = 1; m->i = (int64_t)rd_le(r, 8); break;
    case 12: {
      uint64_t b = rd_le(r, 8);
      memcpy(&m->f, &b, 8);
      m->kind = 2;
      break;
    }
    default: return fail("unknown GGUF metadata type %u", ty);
  }
  return r->err ? -1 : 0;
}

static void gguf_close(gguf *g) {
  if (!g) return;
  for (size_t i = 0; i < g->n_meta; i++) { free(g->meta[i].key); free(g->meta[i].s); }
  for (size_t i = 0; i < g->n_tensors; i++) free(g->tensors[i].name);
  free(g->meta);
  free(g->tensors);
  if (g->map) munmap(g->map, g->size);
  free(g);
}

static const gg_meta *meta_get(const gguf *g, const char *key) {
  for (size_t i = 0; i < g->n_meta; i++)
    if (!strcmp(g->meta[i].key, key)) return &g->meta[i];
  return NULL;
}
static const gg_tensor *tensor_get(const gguf *g, const char *name) {
  for (size_t i = 0; i < g->n_tensors; i++)
    if (!strcmp(g->tensors[i].name, name)) return &g->tensors[i];
  return NULL;
}

/* tensor_range (src/gguf.rs:217-250). */
static int tensor_range(const gguf *g, const gg_tensor *t, size_t *start, size_t *len) {
  int bs = oq_block_size(t->type);
  if (!bs) return fail("tensor %s: unsupported GGML tensor type %u", t->name, t->type);
  unsigned __int128 el = 1;
  for (uint32_t i = 0; i < t->ndim; i++) {
    el *= t->dims[i];
    if (el > (unsigned __int128)SIZE_MAX) return fail("tensor %s element count overflow", t->name);
  }
  size_t elements = (size_t)el;
  if (elements % (size_t)bs) return fail("tensor %s element count is incompatible", t->name);
  if (t->dims[0] % (uint64_t)bs) return fail("tensor %s row width is incompatible", t->name);
  size_t l = elements / (size_t)bs * (size_t)oq_type_size(t->type);
  if (t->offset > SIZE_MAX - g->data_offset) return fail("tensor %s offset overflow", t->name);
  size_t s = g->data_offset + (size_t)t->offset;
  if (s > g->size || l > g->size - s) return fail("tensor %s is outside the GGUF file", t->name);
  *start = s;
  *len = l;
  return 0;
}

/* GgufFile::open (src/gguf.rs:78-169). */
static gguf *gguf_open(const char *path) {
  int fd = open(path, O_RDONLY);
  if (fd < 0) { fail("failed to open %s", path); return NULL; }
  struct stat st;
  fstat(fd, &st);
  gguf *g = (gguf *)calloc(1, sizeof *g);
  g->size = (size_t)st.st_size;
  g->map = g->size ? (uint8_t *)mmap(NULL, g->size, PROT_READ, MAP_PRIVATE, fd, 0) : NULL;
  close(fd);
  if (g->size && g->map == MAP_FAILED) { g->map = NULL; gguf_close(g); fail("mmap failed"); return NULL; }
  rdr r = {g->map, g->size, 0, 0};
  const uint8_t *magic = take(&r, 4);
  if (!magic || memcmp(magic, "GGUF", 4)) { fail("%s is not a GGUF file", path); gguf_close(g); return NULL; }
  g->version = (uint32_t)rd_le(&r, 4);
  if (r.err) { gguf_close(g); return NULL; }
  if (g->version < 2 || g->version > 3) {
    fail("unsupported GGUF version %u; versions 2 and 3 are supported", g->version);
    gguf_close(g);
    return NULL;
  }
  uint64_t nt = rd_le(&r, 8), nm = rd_le(&r, 8);
  if (r.err) { gguf_close(g); return NULL; }
  if (nt > 1000000 || nm > 1000000) { fail("unreasonable GGUF header counts"); gguf_close(g); return NULL; }
  g->meta = (gg_meta *)calloc(nm ? nm : 1, sizeof(gg_meta));
  for (uint64_t i = 0; i < nm; i++) {
    char *key = rd_string(&r);
    uint32_t ty = (uint32_t)rd_le(&r, 4);
    if (r.err) { free(key); gguf_close(g); return NULL; }
    gg_meta m = {0};
    m.key = key;
    if (rd_meta_value(&r, ty, &m)) { free(key); free(m.s); gguf_close(g); return NULL; }
    if (meta_get(g, key)) { fail("duplicate GGUF metadata key %s", key); free(key); free(m.s); gguf_close(g); return NULL; }
    g->meta[g->n_meta++] = m;
  }
  g->tensors = (gg_tensor *)calloc(nt ? nt : 1, sizeof(gg_tensor));
  for (uint64_t i = 0; i < nt; i++) {
    gg_tensor t = {0};
    t.name = rd_string(&r);
    t.ndim = (uint32_t)rd_le(&r, 4);
    if (r.err) { free(t.name); gguf_close(g); return NULL; }
    if (t.ndim < 1 || t.ndim > 4) {
      fail("tensor %s has invalid dimension count %u", t.name, t.ndim);
      free(t.name); gguf_close(g); return NULL;
    }
    for (uint32_t k = 0; k < t.ndim; k++) t.dims[k] = rd_le(&r, 8);
    t.type = (uint32_t)rd_le(&r, 4);
    t.offset = rd_le(&r, 8);
    if (r.err) { free(t.name); gguf_close(g); return NULL; }
    if (tensor_get(g, t.name)) { fail("duplicate GGUF tensor %s", t.name); free(t.name); gguf_close(g); return NULL; }
    g->tensors[g->n_tensors++] = t;
  }
  const gg_meta *al = meta_get(g, "general.alignment");
  uint64_t alignment = 32;
  if (al && al->kind == 0) alignment = al->u;
  else if (al && al->kind == 1 && al->i >= 0) alignment = (uint64_t)al->i;
  if (alignment == 0 || (alignment & (alignment - 1)) || alignment > (1u << 20)) {
    fail("invalid GGUF alignment %llu", (unsigned long long)alignment);
    gguf_close(g);
    return NULL;
  }
  g->data_offset = (r.pos + (size_t)alignment - 1) & ~((size_t)alignment - 1);
  if (g->data_offset > g->size) { fail("GGUF tensor data offset is outside the file"); gguf_close(g); return NULL; }
  for (size_t i = 0; i < g->n_tensors; i++) {
    size_t s, l;
    if (tensor_range(g, &g->tensors[i], &s, &l)) { gguf_close(g); return NULL; }
  }
  return g;
}

/* --------------------------------- model ---------------------------------- */

typedef struct {
  const uint8_t *data;
  uint32_t type;
  size_t rows, cols;
} oq_mat;

typedef struct {
  float *attn_norm, *ffn_norm;
  oq_mat q, k, v, o, gate, up, down;
  float *bq, *bk, *bv;
} oq_layer;

struct oq_model {
  gguf *g;
  oq_config cfg;
  oq_mat embed, lm_head;
  float *norm;
  oq_layer *layers;
  int kernel, threads;
};

struct oq_state {
  size_t max_seq_len, n_layers, kv_width, vocab;
  float **k_cache, **v_cache;
  float *hidden, *residual, *q, *k, *v, *attention, *projection, *gate, *up, *down, *scores,
      *rope_cos, *rope_sin, *logits;
};

static uint64_t meta_u64(const gguf *g, const char *key, int *err) {
  const gg_meta *m = meta_get(g, key);
  if (m && m->kind == 0) return m->u;
  if (m && m->kind == 1 && m->i >= 0) return (uint64_t)m->i;
  *err = fail("missing or non-integer GGUF metadata %s", key);
  return 0;
}
static int meta_f32(const gguf *g, const char *key, float *out) {
  const gg_meta *m = meta_get(g, key);
  if (!m) return -1;
  if (m->kind == 2) *out = (float)m->f;
  else if (m->kind == 0) *out = (float)m->u;
  else if (m->kind == 1) *out = (float)m->i;
  else return -1;
  return 0;
}

/* load_gguf_matrix + check_matrix (src/loader.rs:449-456, 497-507). */
static int load_matrix(const gguf *g, const char *name, size_t rows, size_t cols, oq_mat *out) {
  const gg_tensor *t = tensor_get(g, name);
  if (!t) return fail("missing GGUF tensor %s", name);
  if (t->ndim > 2) return fail("tensor %s has %u dimensions", name, t->ndim);
  size_t s, l;
  if (tensor_range(g, t, &s, &l)) return -1;
  size_t r = t->ndim == 1 ? 1 : (size_t)t->dims[1], c = (size_t)t->dims[0];
  if (t->ndim != 2 || r != rows || c != cols)
    return fail("tensor %s has shape [%zu, %zu], expected [%zu, %zu]", name, r, c, rows, cols);
  out->data = g->map + s;
  out->type = t->type;
  out->rows = rows;
  out->cols = cols;
  return 0;
}

/* load_gguf_vector (src/loader.rs:509-517): any supported type, dequantized to f32. */
static float *load_vector(const gguf *g, const char *name, size_t len) {
  const gg_tensor *t = tensor_get(g, name);
  if (!t) { fail("missing GGUF tensor %s", name); return NULL; }
  size_t s, l;
  if (tensor_range(g, t, &s, &l)) return NULL;
  if (t->ndim != 1 || t->dims[0] != len) { fail("tensor %s has the wrong shape, expected [%zu]", name, len); return NULL; }
  float *v = (float *)malloc(len * sizeof(float));
  oq_dequant_row(g->map + s, t->type, len, v);
  return v;
}

static float *load_bias(const gguf *g, const char *name, size_t rows, int *err) {
  if (!tensor_get(g, name)) return (float *)calloc(rows, sizeof(float)); /* zeros if absent */
  float *b = load_vector(g, name, rows);
  if (!b) *err = -1;
  return b;
}

void oq_model_free(oq_model *m) {
  if (!m) return;
  if (m->layers)
    for (size_t i = 0; i < m->cfg.num_hidden_layers; i++) {
      oq_layer *L = &m->layers[i];
      free(L->attn_norm); free(L->ffn_norm); free(L->bq); free(L->bk); free(L->bv);
    }
  free(m->layers);
  free(m->norm);
  gguf_close(m->g);
  free(m);
}

oq_model *oq_model_load_gguf(const char *path, int kernel, int threads) {
  gguf *g = gguf_open(path);
  if (!g) return NULL;
  oq_model *m = (oq_model *)calloc(1, sizeof *m);
  m->g = g;
  m->kernel = kernel;
  m->threads = threads;
  const gg_meta *arch = meta_get(g, "general.architecture");
  if (!arch || arch->kind != 4) { fail("missing or non-string GGUF metadata general.architecture"); oq_model_free(m); return NULL; }
  if (strcmp(arch->s, "qwen2")) { fail("unsupported GGUF architecture \"%s\"", arch->s); oq_model_free(m); return NULL; }
  const gg_tensor *te = tensor_get(g, "token_embd.weight");
  if (!te) { fail("missing GGUF tensor token_embd.weight"); oq_model_free(m); return NULL; }
  if (te->ndim != 2) { fail("token_embd.weight must be 2D"); oq_model_free(m); return NULL; }
  oq_config *c = &m->cfg;
  int err = 0;
  c->hidden_size = (size_t)meta_u64(g, "qwen2.embedding_length", &err);
  c->intermediate_size = (size_t)meta_u64(g, "qwen2.feed_forward_length", &err);
  c->num_attention_heads = (size_t)meta_u64(g, "qwen2.attention.head_count", &err);
  c->num_key_value_heads = (size_t)meta_u64(g, "qwen2.attention.head_count_kv", &err);
  c->num_hidden_layers = (size_t)meta_u64(g, "qwen2.block_count", &err);
  c->vocab_size = (size_t)te->dims[1];
  if (err) { oq_model_free(m); return NULL; }
  if (meta_f32(g, "qwen2.attention.layer_norm_rms_epsilon", &c->rms_norm_eps)) {
    fail("missing or non-numeric GGUF metadata qwen2.attention.layer_norm_rms_epsilon");
    oq_model_free(m);
    return NULL;
  }
  if (meta_f32(g, "qwen2.rope.freq_base", &c->rope_theta)) c->rope_theta = 10000.0f;
  c->max_position_embeddings = (size_t)meta_u64(g, "qwen2.context_length", &err);
  if (err) { oq_model_free(m); return NULL; }
  c->tie_word_embeddings = tensor_get(g, "output.weight") == NULL;
  /* LlamaConfig::validate (src/config.rs:57-89); head_dim = hidden / heads. */
  if (!c->hidden_size || !c->intermediate_size || !c->num_attention_heads || !c->num_key_value_heads ||
      !c->num_hidden_layers || !c->vocab_size) { fail("invalid Qwen2 config: dimensions must be non-zero"); oq_model_free(m); return NULL; }
  if (c->hidden_size % c->num_attention_heads) { fail("hidden_size must be divisible by num_attention_heads"); oq_model_free(m); return NULL; }
  if (c->num_attention_heads % c->num_key_value_heads) { fail("num_attention_heads must be divisible by num_key_value_heads"); oq_model_free(m); return NULL; }
  c->head_dim = c->hidden_size / c->num_attention_heads;
  c->kv_width = c->num_key_value_heads * c->head_dim;
  if (c->head_dim % 2) { fail("Qwen2 RoPE requires an even head_dim"); oq_model_free(m); return NULL; }
  if (!isfinite(c->rms_norm_eps) || c->rms_norm_eps <= 0) { fail("rms_norm_eps must be finite and positive"); oq_model_free(m); return NULL; }
  if (!isfinite(c->rope_theta) || c->rope_theta <= 0) { fail("rope_theta must be finite and positive"); oq_model_free(m); return NULL; }
  if (te->dims[0] != c->hidden_size) { fail("GGUF embedding width/config mismatch"); oq_model_free(m); return NULL; }

  size_t H = c->hidden_size, F = c->intermediate_size, KV = c->kv_width;
  if (load_matrix(g, "token_embd.weight", c->vocab_size, H, &m->embed)) { oq_model_free(m); return NULL; }
  if (!(m->norm = load_vector(g, "output_norm.weight", H))) { oq_model_free(m); return NULL; }
  m->layers = (oq_layer *)calloc(c->num_hidden_layers, sizeof(oq_layer));
  char name[128];
  for (size_t i = 0; i < c->num_hidden_layers; i++) {
    oq_layer *L = &m->layers[i];
#define NM(s) (snprintf(name, sizeof name, "blk.%zu." s, i), name)
    if (!(L->attn_norm = load_vector(g, NM("attn_norm.weight"), H)) ||
        load_matrix(g, NM("attn_q.weight"), H, H, &L->q) ||
        !(L->bq = load_bias(g, NM("attn_q.bias"), H, &err)) ||
        load_matrix(g, NM("attn_k.weight"), KV, H, &L->k) ||
        !(L->bk = load_bias(g, NM("attn_k.bias"), KV, &err)) ||
        load_matrix(g, NM("attn_v.weight"), KV, H, &L->v) ||
        !(L->bv = load_bias(g, NM("attn_v.bias"), KV, &err)) ||
        load_matrix(g, NM("attn_output.weight"), H, H, &L->o) ||
        !(L->ffn_norm = load_vector(g, NM("ffn_norm.weight"), H)) ||
        load_matrix(g, NM("ffn_gate.weight"), F, H, &L->gate) ||
        load_matrix(g, NM("ffn_up.weight"), F, H, &L->up) ||
        load_matrix(g, NM("ffn_down.weight"), H, F, &L->down) || err) {
      oq_model_free(m);
      return NULL;
    }
#undef NM
  }
  if (c->tie_word_embeddings) m->lm_head = m->embed;
  else if (load_matrix(g, "output.weight", c->vocab_size, H, &m->lm_head)) { oq_model_free(m); return NULL; }
  return m;
}

void oq_model_config(const oq_model *m, oq_config *out) { *out = m->cfg; }

int oq_gguf_read_f32(const char *path, const char *name, uint32_t *version, size_t *rows,
                     size_t *cols, float *out, size_t capacity) {
  gguf *g = gguf_open(path);
  if (!g) return -1;
  const gg_tensor *t = tensor_get(g, name);
  if (!t) { fail("missing GGUF tensor %s", name); gguf_close(g); return -1; }
  if (t->ndim > 2) { fail("tensor %s has %u dimensions", name, t->ndim); gguf_close(g); return -1; }
  size_t s, l;
  if (tensor_range(g, t, &s, &l)) { gguf_close(g); return -1; }
  size_t r = t->ndim == 2 ? (size_t)t->dims[1] : 1, c = (size_t)t->dims[0];
  if (version) *version = g->version;
  if (rows) *rows = r;
  if (cols) *cols = c;
  if (out) {
    if (capacity < r * c) { fail("capacity too small"); gguf_close(g); return -1; }
    size_t rb = oq_row_bytes(t->type, c);
    for (size_t i = 0; i < r; i++) oq_dequant_row(g->map + s + i * rb, t->type, c, out + i * c);
  }
  gguf_close(g);
  return 0;
}

oq_state *oq_state_new(const oq_model *m, size_t max_seq_len) {
  const oq_config *c = &m->cfg;
  if (max_seq_len == 0) { fail("max_seq_len must be positive"); return NULL; }
  if (max_seq_len > c->max_position_embeddings) {
    fail("requested context %zu exceeds model limit %zu", max_seq_len, c->max_position_embeddings);
    return NULL;
  }
  oq_state *s = (oq_state *)calloc(1, sizeof *s);
  s->max_seq_len = max_seq_len;
  s->n_layers = c->num_hidden_layers;
  s->kv_width = c->kv_width;
  s->vocab = c->vocab_size;
  s->k_cache = (float **)calloc(c->num_hidden_layers, sizeof(float *));
  s->v_cache = (float **)calloc(c->num_hidden_layers, sizeof(float *));
  for (size_t i = 0; i < c->num_hidden_layers; i++) {
    s->k_cache[i] = (float *)calloc(max_seq_len * c->kv_width, sizeof(float));
    s->v_cache[i] = (float *)calloc(max_seq_len * c->kv_width, sizeof(float));
  }
  size_t H = c->hidden_size, KV = c->kv_width, F = c->intermediate_size;
  s->hidden = (float *)calloc(H, 4);
  s->residual = (float *)calloc(H, 4);
  s->q = (float *)calloc(H, 4);
  s->k = (float *)calloc(KV, 4);
  s->v = (float *)calloc(KV, 4);
  s->attention = (float *)calloc(H, 4);
  s->projection = (float *)calloc(H, 4);
  s->gate = (float *)calloc(F, 4);
  s->up = (float *)calloc(F, 4);
  s->down = (float *)calloc(H, 4);
  s->scores = (float *)calloc(max_seq_len, 4);
  s->rope_cos = (float *)calloc(c->head_dim / 2, 4);
  s->rope_sin = (float *)calloc(c->head_dim / 2, 4);
  s->logits = (float *)calloc(c->vocab_size, 4);
  return s;
}

void oq_state_free(oq_state *s) {
  if (!s) return;
  for (size_t i = 0; i < s->n_layers; i++) { free(s->k_cache[i]); free(s->v_cache[i]); }
  free(s->hidden); free(s->residual); free(s->q); free(s->k); free(s->v); free(s->attention);
  free(s->projection); free(s->gate); free(s->up); free(s->down); free(s->scores);
  free(s->rope_cos); free(s->rope_sin); free(s->logits);
  free(s->k_cache); free(s->v_cache);
  free(s);
}

static void rmsnorm(float *h, const float *w, size_t n, float eps) {
  float sum = -0.0f;
  for (size_t i = 0; i < n; i++) sum += h[i] * h[i];
  float mean_sq = sum / (float)n;
  float inv_rms = 1.0f / sqrtf(mean_sq + eps);
  for (size_t i = 0; i < n; i++) h[i] *= inv_rms * w[i];
}

static void prepare_rope(size_t pos, size_t hd, float theta, float *cs, float *sn) {
  for (size_t i = 0; i < hd / 2; i++) {
    float inv_freq = 1.0f / powf(theta, 2.0f * (float)i / (float)hd);
    float angle = (float)pos * inv_freq;
    sn[i] = sinf(angle);
    cs[i] = cosf(angle);
  }
}

static void apply_rope(float *x, size_t len, const float *cs, const float *sn) {
  size_t half = len / 2;
  for (size_t i = 0; i < half; i++) {
    float re = x[i], im = x[i + half];
    x[i] = re * cs[i] - im * sn[i];
    x[i + half] = re * sn[i] + im * cs[i];
  }
}

static void softmax(float *v, size_t n) {
  float mx = -INFINITY;
  for (size_t i = 0; i < n; i++) mx = fmaxf(mx, v[i]);
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    v[i] = expf(v[i] - mx);
    sum += v[i];
  }
  if (isfinite(sum) && sum > 0.0f) {
    for (size_t i = 0; i < n; i++) v[i] /= sum;
  } else {
    float u = 1.0f / (float)n;
    for (size_t i = 0; i < n; i++) v[i] = u;
  }
}

static int linear(const oq_model *m, const oq_mat *w, const float *bias, const float *x, float *y) {
  if (oq_matvec(w->data, w->type, w->rows, w->cols, x, y, m->kernel, m->threads, 128 * 1024))
    return fail("matvec failed");
  if (bias)
    for (size_t i = 0; i < w->rows; i++) y[i] += bias[i];
  return 0;
}

int oq_forward_token(const oq_model *m, oq_state *s, uint32_t token, size_t pos, int logits_mode) {
  const oq_config *c = &m->cfg;
  if ((size_t)token >= c->vocab_size) return fail("token id %u is outside vocabulary", token);
  if (pos >= s->max_seq_len) return fail("position %zu exceeds configured context %zu", pos, s->max_seq_len);
  size_t H = c->hidden_size, hd = c->head_dim, nh = c->num_attention_heads, nkv = c->num_key_value_heads;
  size_t KV = c->kv_width, groups = nh / nkv, F = c->intermediate_size;
  float scale = 1.0f / sqrtf((float)hd);
  prepare_rope(pos, hd, c->rope_theta, s->rope_cos, s->rope_sin);
  oq_dequant_row(m->embed.data + (size_t)token * oq_row_bytes(m->embed.type, H), m->embed.type, H, s->residual);
  for (size_t li = 0; li < c->num_hidden_layers; li++) {
    const oq_layer *L = &m->layers[li];
    memcpy(s->hidden, s->residual, H * 4);
    rmsnorm(s->hidden, L->attn_norm, H, c->rms_norm_eps);
    if (linear(m, &L->q, L->bq, s->hidden, s->q) || linear(m, &L->k, L->bk, s->hidden, s->k) ||
        linear(m, &L->v, L->bv, s->hidden, s->v))
      return -1;
    for (size_t h = 0; h < nh; h++) apply_rope(s->q + h * hd, hd, s->rope_cos, s->rope_sin);
    for (size_t h = 0; h < nkv; h++) apply_rope(s->k + h * hd, hd, s->rope_cos, s->rope_sin);
    memcpy(s->k_cache[li] + pos * KV, s->k, KV * 4);
    memcpy(s->v_cache[li] + pos * KV, s->v, KV * 4);
    memset(s->attention, 0, H * 4);
    for (size_t h = 0; h < nh; h++) {
      size_t kvh = h / groups;
      const float *qh = s->q + h * hd;
      for (size_t p = 0; p <= pos; p++) {
        const float *key = s->k_cache[li] + p * KV + kvh * hd;
        float dot = -0.0f;
        for (size_t d = 0; d < hd; d++) dot += qh[d] * key[d];
        s->scores[p] = dot * scale;
      }
      softmax(s->scores, pos + 1);
      float *out = s->attention + h * hd;
      for (size_t p = 0; p <= pos; p++) {
        float w = s->scores[p];
        const float *val = s->v_cache[li] + p * KV + kvh * hd;
        for (size_t d = 0; d < hd; d++) out[d] += w * val[d];
      }
    }
    if (linear(m, &L->o, NULL, s->attention, s->projection)) return -1;
    for (size_t i = 0; i < H; i++) s->residual[i] += s->projection[i];
    memcpy(s->hidden, s->residual, H * 4);
    rmsnorm(s->hidden, L->ffn_norm, H, c->rms_norm_eps);
    if (linear(m, &L->gate, NULL, s->hidden, s->gate) || linear(m, &L->up, NULL, s->hidden, s->up)) return -1;
    for (size_t i = 0; i < F; i++) {
      float g = s->gate[i];
      s->gate[i] = (g / (1.0f + expf(-g))) * s->up[i];
    }
    if (linear(m, &L->down, NULL, s->gate, s->down)) return -1;
    for (size_t i = 0; i < H; i++) s->residual[i] += s->down[i];
  }
  if (logits_mode) {
    memcpy(s->hidden, s->residual, H * 4);
    rmsnorm(s->hidden, m->norm, H, c->rms_norm_eps);
    if (linear(m, &m->lm_head, NULL, s->hidden, s->logits)) return -1;
  }
  return 0;
}

int oq_prefill(const oq_model *m, oq_state *s, const uint32_t *tokens, size_t n, size_t start_pos) {
  if (n == 0) return fail("prefill requires at least one token");
  for (size_t i = 0; i < n; i++)
    if (oq_forward_token(m, s, tokens[i], start_pos + i, i + 1 == n)) return -1;
  return 0;
}

/* f32::total_cmp key: flip the magnitude bits of negatives, compare as i32. */
static inline int32_t total_key(float f) {
  int32_t b;
  memcpy(&b, &f, 4);
  return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

uint32_t oq_argmax(const float *logits, size_t n) {
  if (n == 0) return 0;
  size_t best = 0;
  int32_t bk = total_key(logits[0]);
  for (size_t i = 1; i < n; i++) {
    int32_t k = total_key(logits[i]);
    if (k >= bk) { bk = k; best = i; } /* Iterator::max_by keeps the last maximum */
  }
  return (uint32_t)best;
}

/* ---- sampling: sample_current_logits (src/engine.rs:253-325) ---- */

typedef struct { uint32_t token; float value; } oq_cand;

/* Descending in total_cmp order (src/engine.rs:285); equal values keep the
 * lower token first (the reference's unstable sort leaves them unordered). */
static int cand_cmp(const void *a, const void *b) {
  const oq_cand *x = (const oq_cand *)a, *y = (const oq_cand *)b;
  int32_t kx = total_key(x->value), ky = total_key(y->value);
  if (kx != ky) return kx > ky ? -1 : 1;
  return x->token < y->token ? -1 : (x->token > y->token);
}

uint32_t oq_sample(const float *logits, size_t n, float temperature, size_t top_k, float top_p,
                   float repetition_penalty, const uint32_t *recent, size_t n_recent, float uniform) {
  if (n == 0) return 0;
  unsigned char *seen = calloc(n, 1);
  oq_cand *c = malloc(n * sizeof *c);
  if (!seen || !c) {
    free(seen);
    free(c);
    return 0;
  }
  for (size_t i = 0; i < n_recent; i++)
    if (recent[i] < n) seen[recent[i]] = 1;
  for (size_t t = 0; t < n; t++) { /* src/engine.rs:262-278 */
    float v = logits[t];
    if (repetition_penalty != 1.0f && seen[t]) v = v > 0.0f ? v / repetition_penalty : v * repetition_penalty;
    if (temperature > 0.0f) v /= temperature;
    if (!isfinite(v)) v = -INFINITY;
    c[t].token = (uint32_t)t;
    c[t].value = v;
  }
  qsort(c, n, sizeof *c, cand_cmp);
  uint32_t out = c[0].token;
  if (temperature > 0.0f) {
    size_t m = (top_k > 0 && top_k < n) ? top_k : n;
    float max = c[0].value, sum = 0.0f;
    for (size_t i = 0; i < m; i++) {
      c[i].value = expf(c[i].value - max);
      sum += c[i].value;
    }
    if (isfinite(sum) && sum > 0.0f) {
      for (size_t i = 0; i < m; i++) c[i].value /= sum;
      float cumulative = 0.0f;
      size_t cutoff = m;
      for (size_t i = 0; i < m; i++) {
        cumulative += c[i].value;
        if (cumulative >= top_p) {
          cutoff = i + 1;
          break;
        }
      }
      float kept_sum = 0.0f;
      for (size_t i = 0; i < cutoff; i++) kept_sum += c[i].value;
      float random = uniform * kept_sum;
      out = c[cutoff - 1].token;
      for (size_t i = 0; i < cutoff; i++) {
        random -= c[i].value;
        if (random <= 0.0f) {
          out = c[i].token;
          break;
        }
      }
    }
  }
  free(seen);
  free(c);
  return out;
}

int oq_decode_greedy(const oq_model *m, oq_state *s, size_t start_pos, size_t n_steps, uint32_t *out) {
  for (size_t i = 0; i < n_steps; i++) {
    uint32_t tok = oq_argmax(s->logits, m->cfg.vocab_size);
    out[i] = tok;
    if (oq_forward_token(m, s, tok, start_pos + i, 1)) return -1;
  }
  return 0;
}

const float *oq_state_logits(const oq_state *s) { return s->logits; }
const float *oq_state_residual(const oq_state *s) { return s->residual; }
const float *oq_state_k_cache(const oq_state *s, size_t layer) { return s->k_cache[layer]; }
const float *oq_state_v_cache(const oq_state *s, size_t layer) { return s->v_cache[layer]; }

int oq_state_load(oq_state *s, int what, size_t layer, const float *src, size_t n) {
  if (what == 2) {
    if (n != s->vocab) return fail("logits length %zu != vocab %zu", n, s->vocab);
    memcpy(s->logits, src, n * sizeof(float));
    return 0;
  }
  if (what != 0 && what != 1) return fail("unknown state part %d", what);
  if (layer >= s->n_layers) return fail("layer %zu out of bounds", layer);
  size_t kvw = s->kv_width;
  if (n > s->max_seq_len * kvw) return fail("%zu floats exceed the layer's cache", n);
  memcpy(what ? s->v_cache[layer] : s->k_cache[layer], src, n * sizeof(float));
  return 0;
}
