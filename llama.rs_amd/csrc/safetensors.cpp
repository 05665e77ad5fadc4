// Hugging Face checkpoint directories (see safetensors.h).
#include "safetensors.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <sstream>

#include "common.h"
#include "json.h"

namespace fs = std::filesystem;

namespace llrs {

namespace {

constexpr uint64_t kMaxHeader = 100000000;  // the safetensors crate's MAX_HEADER_SIZE

// Element sizes of the safetensors 0.4 dtypes.
int dtype_size(const std::string &d) {
  static const std::pair<const char *, int> kSizes[] = {
      {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"F8_E5M2", 1}, {"F8_E4M3", 1},
      {"I16", 2},  {"U16", 2}, {"F16", 2}, {"BF16", 2},    {"I32", 4},
      {"U32", 4},  {"F32", 4}, {"F64", 8}, {"I64", 8},     {"U64", 8}};
  for (const auto &s : kSizes)
    if (d == s.first) return s.second;
  return 0;
}

bool valid_utf8(const uint8_t *s, size_t n) {
  size_t i = 0;
  while (i < n) {
    const uint8_t c = s[i];
    int k;
    uint32_t cp;
    if (c < 0x80) {
      i++;
      continue;
    } else if ((c & 0xe0) == 0xc0) {
      k = 1;
      cp = c & 0x1f;
    } else if ((c & 0xf0) == 0xe0) {
      k = 2;
      cp = c & 0x0f;
    } else if ((c & 0xf8) == 0xf0) {
      k = 3;
      cp = c & 0x07;
    } else {
      return false;
    }
    for (int j = 1; j <= k; j++) {
      if (i + j >= n || (s[i + j] & 0xc0) != 0x80) return false;
      cp = (cp << 6) | (s[i + j] & 0x3f);
    }
    if ((k == 1 && cp < 0x80) || (k == 2 && cp < 0x800) || (k == 3 && cp < 0x10000) ||
        cp > 0x10ffff || (cp >= 0xd800 && cp < 0xe000))
      return false;
    i += (size_t)k + 1;
  }
  return true;
}

bool read_text(const std::string &path, std::string &out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream ss;
  ss << f.rdbuf();
  out = ss.str();
  return !f.bad();
}

bool has_ext(const fs::path &p, const char *ext) { return p.extension() == std::string(".") + ext; }

}  // namespace

SafetensorsFile::~SafetensorsFile() {
  if (map_) munmap(map_, size_);
}

int SafetensorsFile::open(const std::string &p) {
  path = p;
  int fd = ::open(p.c_str(), O_RDONLY);
  if (fd < 0) return set_error(LLRS_E_IO, "failed to open %s", p.c_str());
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return set_error(LLRS_E_IO, "failed to stat %s", p.c_str());
  }
  size_ = (size_t)st.st_size;
  if (size_) {
    void *m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      ::close(fd);
      return set_error(LLRS_E_IO, "failed to mmap %s", p.c_str());
    }
    map_ = (uint8_t *)m;
  }
  ::close(fd);
  return LLRS_OK;
}

int SafetensorsFile::parse() {
  if (parsed_) return LLRS_OK;
  const char *f = path.c_str();
  if (size_ < 8) return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: header too small", f);
  uint64_t n = 0;
  for (int i = 7; i >= 0; i--) n = (n << 8) | map_[i];
  if (n > kMaxHeader) return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: header too large", f);
  if (n > size_ - 8)
    return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: header length exceeds the file", f);
  const uint8_t *h = map_ + 8;
  if (!valid_utf8(h, (size_t)n))
    return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: header is not UTF-8", f);
  JsonValue doc;
  std::string err;
  if (!json_parse((const char *)h, (size_t)n, doc, err))
    return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: header JSON: %s", f, err.c_str());
  if (doc.kind != JsonValue::OBJECT)
    return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: the header is not a JSON object", f);
  std::map<std::string, SafetensorInfo> out;
  for (const auto &m : doc.members) {
    const std::string &name = m.first;
    const JsonValue &v = m.second;
    if (name == "__metadata__") {
      bool ok = v.kind == JsonValue::NUL || v.kind == JsonValue::OBJECT;
      for (const auto &kv : v.members) ok = ok && kv.second.kind == JsonValue::STRING;
      if (!ok)
        return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: __metadata__ must map strings to strings", f);
      continue;
    }
    const JsonValue *dt = v.get("dtype"), *sh = v.get("shape"), *off = v.get("data_offsets");
    if (v.kind != JsonValue::OBJECT || !dt || !sh || !off || dt->kind != JsonValue::STRING ||
        sh->kind != JsonValue::ARRAY || off->kind != JsonValue::ARRAY || off->items.size() != 2)
      return set_error(LLRS_E_FORMAT,
                       "invalid safetensors file %s: tensor %s needs dtype, shape and two data_offsets", f,
                       name.c_str());
    SafetensorInfo t;
    t.dtype = dt->text;
    if (!dtype_size(t.dtype))
      return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: tensor %s has unknown dtype %s", f,
                       name.c_str(), t.dtype.c_str());
    for (const auto &d : sh->items) {
      uint64_t x;
      if (!d.as_u64(x))
        return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: tensor %s has a bad shape", f, name.c_str());
      t.shape.push_back(x);
    }
    uint64_t s, e;
    if (!off->items[0].as_u64(s) || !off->items[1].as_u64(e))
      return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: tensor %s has bad data_offsets", f, name.c_str());
    t.start = (size_t)s;  // relative for now
    t.nbytes = (size_t)e;
    out[name] = t;  // a repeated name: the last entry counts
  }
  // Metadata::validate: in offset order the ranges tile [0, end) exactly
  // and each holds elements x dtype size bytes.
  std::vector<std::pair<std::string, SafetensorInfo *>> order;
  for (auto &kv : out) order.push_back({kv.first, &kv.second});
  std::stable_sort(order.begin(), order.end(), [](const auto &a, const auto &b) {
    return a.second->start != b.second->start ? a.second->start < b.second->start
                                              : a.second->nbytes < b.second->nbytes;
  });
  uint64_t pos = 0;
  for (auto &o : order) {
    SafetensorInfo &t = *o.second;
    const uint64_t s = t.start, e = t.nbytes;
    if (s != pos || e < s)
      return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: tensor %s has invalid offsets", f,
                       o.first.c_str());
    pos = e;
    uint64_t elems = 1;
    for (uint64_t d : t.shape) {
      if (d && elems > UINT64_MAX / d)
        return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: tensor %s size overflows", f, o.first.c_str());
      elems *= d;
    }
    const uint64_t es = (uint64_t)dtype_size(t.dtype);
    if (elems > UINT64_MAX / es)
      return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: tensor %s size overflows", f, o.first.c_str());
    if (e - s != elems * es)
      return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: tensor %s holds %llu bytes, its shape needs %llu",
                       f, o.first.c_str(), (unsigned long long)(e - s), (unsigned long long)(elems * es));
    t.start = (size_t)(8 + n + s);
    t.nbytes = (size_t)(e - s);
  }
  if (pos != size_ - 8 - n)
    return set_error(LLRS_E_FORMAT, "invalid safetensors file %s: the data section holds %llu bytes, the tensors %llu",
                     f, (unsigned long long)(size_ - 8 - n), (unsigned long long)pos);
  tensors.swap(out);
  parsed_ = true;
  return LLRS_OK;
}

const SafetensorInfo *SafetensorsFile::tensor(const std::string &name) const {
  auto it = tensors.find(name);
  return it == tensors.end() ? nullptr : &it->second;
}

int SafetensorStore::open(const std::string &dir) {
  const fs::path d(dir);
  const fs::path index = d / "model.safetensors.index.json";
  std::error_code ec;
  std::vector<std::string> paths;
  indexed_ = fs::exists(index, ec);
  if (indexed_) {
    std::string text, err;
    if (!read_text(index.string(), text))
      return set_error(LLRS_E_IO, "failed to read %s", index.string().c_str());
    JsonValue doc;
    if (!json_parse(text.data(), text.size(), doc, err))
      return set_error(LLRS_E_FORMAT, "%s: %s", index.string().c_str(), err.c_str());
    const JsonValue *wm = doc.get("weight_map");
    if (!wm || wm->kind != JsonValue::OBJECT)
      return set_error(LLRS_E_FORMAT, "%s has no weight_map object", index.string().c_str());
    for (const auto &m : wm->members) {
      if (m.second.kind != JsonValue::STRING)
        return set_error(LLRS_E_FORMAT, "%s: weight_map values must be file names", index.string().c_str());
      const std::string p = (d / m.second.text).string();
      where_[m.first] = p;
      paths.push_back(p);
    }
    std::sort(paths.begin(), paths.end());
    paths.erase(std::unique(paths.begin(), paths.end()), paths.end());
  } else {
    for (fs::directory_iterator it(d, ec), end; !ec && it != end; it.increment(ec))
      if (has_ext(it->path(), "safetensors")) paths.push_back(it->path().string());
    if (ec) return set_error(LLRS_E_IO, "failed to list %s", dir.c_str());
    std::sort(paths.begin(), paths.end());
    if (paths.empty()) return set_error(LLRS_E_INVALID, "no .safetensors files in %s", dir.c_str());
  }
  for (const std::string &p : paths) {
    auto f = std::make_unique<SafetensorsFile>();
    LLRS_TRY(f->open(p));
    if (!indexed_) {
      LLRS_TRY(f->parse());
      for (const auto &t : f->tensors)
        if (!where_.emplace(t.first, p).second)
          return set_error(LLRS_E_INVALID, "duplicate safetensors tensor %s", t.first.c_str());
    }
    files_[p] = std::move(f);
  }
  return LLRS_OK;
}

int SafetensorStore::tensor(const std::string &name, const SafetensorsFile **file,
                            const SafetensorInfo **info) {
  auto w = where_.find(name);
  if (w == where_.end()) return set_error(LLRS_E_INVALID, "missing safetensors tensor %s", name.c_str());
  SafetensorsFile &f = *files_.at(w->second);
  LLRS_TRY(f.parse());
  const SafetensorInfo *t = f.tensor(name);
  if (!t)
    return set_error(LLRS_E_INVALID, "safetensors tensor %s is not in %s", name.c_str(), f.path.c_str());
  if (t->dtype != "F32" && t->dtype != "F16" && t->dtype != "BF16")
    return set_error(LLRS_E_UNSUPPORTED, "unsupported safetensors dtype %s; use F32/F16/BF16", t->dtype.c_str());
  if (t->shape.empty() || t->shape.size() > 2)
    return set_error(LLRS_E_INVALID, "invalid safetensors tensor %s: only 1D and 2D tensors are supported",
                     name.c_str());
  *file = &f;
  *info = t;
  return LLRS_OK;
}

int hf_config_read(const std::string &config_path, llrs_model_config &c) {
  std::string text, err;
  if (!read_text(config_path, text)) return set_error(LLRS_E_IO, "failed to read %s", config_path.c_str());
  JsonValue doc;
  if (!json_parse(text.data(), text.size(), doc, err))
    return set_error(LLRS_E_FORMAT, "%s: %s", config_path.c_str(), err.c_str());
  if (doc.kind != JsonValue::OBJECT) return set_error(LLRS_E_FORMAT, "%s is not a JSON object", config_path.c_str());
  const JsonValue *mt = doc.get("model_type");
  if (!mt || mt->kind != JsonValue::STRING) return set_error(LLRS_E_INVALID, "config.json is missing model_type");
  if (mt->text != "qwen2")
    return set_error(LLRS_E_UNSUPPORTED, "unsupported Hugging Face model_type \"%s\"", mt->text.c_str());
  c = llrs_model_config{};
  auto usize = [&](const char *key, size_t &dst, bool required, size_t dflt) -> int {
    const JsonValue *v = doc.get(key);
    if (!v) {
      if (required) return set_error(LLRS_E_FORMAT, "config.json: missing field `%s`", key);
      dst = dflt;
      return LLRS_OK;
    }
    uint64_t x;
    if (!v->as_u64(x)) return set_error(LLRS_E_FORMAT, "config.json: `%s` must be a non-negative integer", key);
    dst = (size_t)x;
    return LLRS_OK;
  };
  auto f32 = [&](const char *key, float &dst, float dflt) -> int {
    const JsonValue *v = doc.get(key);
    double x;
    if (!v) {
      dst = dflt;
      return LLRS_OK;
    }
    if (!v->as_f64(x)) return set_error(LLRS_E_FORMAT, "config.json: `%s` must be a number", key);
    dst = (float)x;
    return LLRS_OK;
  };
  LLRS_TRY(usize("hidden_size", c.hidden_size, true, 0));
  LLRS_TRY(usize("intermediate_size", c.intermediate_size, true, 0));
  LLRS_TRY(usize("num_attention_heads", c.num_attention_heads, true, 0));
  LLRS_TRY(usize("num_key_value_heads", c.num_key_value_heads, true, 0));
  LLRS_TRY(usize("num_hidden_layers", c.num_hidden_layers, true, 0));
  LLRS_TRY(usize("vocab_size", c.vocab_size, true, 0));
  LLRS_TRY(f32("rms_norm_eps", c.rms_norm_eps, 1e-6f));
  LLRS_TRY(f32("rope_theta", c.rope_theta, 10000.0f));
  LLRS_TRY(usize("max_position_embeddings", c.max_position_embeddings, false, 32768));
  const JsonValue *hd = doc.get("head_dim");
  const bool has_hd = hd && hd->kind != JsonValue::NUL;
  if (has_hd) LLRS_TRY(usize("head_dim", c.head_dim, true, 0));
  const JsonValue *tie = doc.get("tie_word_embeddings");
  if (tie && tie->kind != JsonValue::BOOL)
    return set_error(LLRS_E_FORMAT, "config.json: `tie_word_embeddings` must be a boolean");
  c.tie_word_embeddings = tie && tie->b;
  // LlamaConfig::validate (src/config.rs:57-89).
  if (!c.hidden_size || !c.intermediate_size || !c.num_attention_heads || !c.num_key_value_heads ||
      !c.num_hidden_layers || !c.vocab_size)
    return set_error(LLRS_E_INVALID, "invalid Qwen2 config: dimensions must be non-zero");
  if (c.hidden_size % c.num_attention_heads && !has_hd)
    return set_error(LLRS_E_INVALID, "hidden_size must be divisible by num_attention_heads");
  if (c.num_attention_heads % c.num_key_value_heads)
    return set_error(LLRS_E_INVALID, "num_attention_heads must be divisible by num_key_value_heads");
  if (!has_hd) c.head_dim = c.hidden_size / c.num_attention_heads;
  if (c.head_dim == 0 || c.num_attention_heads > SIZE_MAX / c.head_dim ||
      c.num_attention_heads * c.head_dim != c.hidden_size)
    return set_error(LLRS_E_INVALID, "num_attention_heads * head_dim must equal hidden_size");
  if (c.head_dim % 2) return set_error(LLRS_E_INVALID, "Qwen2 RoPE requires an even head_dim");
  if (!std::isfinite(c.rms_norm_eps) || c.rms_norm_eps <= 0)
    return set_error(LLRS_E_INVALID, "rms_norm_eps must be finite and positive");
  if (!std::isfinite(c.rope_theta) || c.rope_theta <= 0)
    return set_error(LLRS_E_INVALID, "rope_theta must be finite and positive");
  c.kv_width = c.num_key_value_heads * c.head_dim;
  return LLRS_OK;
}

int detect_model_format(const std::string &path, int &format, std::string &resolved) {
  const fs::path p(path);
  std::error_code ec;
  const bool is_file = fs::is_regular_file(p, ec);
  if (is_file && has_ext(p, "gguf")) {
    format = LLRS_FORMAT_GGUF;
    resolved = path;
    return LLRS_OK;
  }
  if (is_file && has_ext(p, "safetensors")) {
    format = LLRS_FORMAT_SAFETENSORS;
    resolved = p.has_parent_path() ? p.parent_path().string() : std::string(".");
    return LLRS_OK;
  }
  if (fs::is_directory(p, ec)) {
    if (fs::exists(p / "model.safetensors", ec) || fs::exists(p / "model.safetensors.index.json", ec)) {
      format = LLRS_FORMAT_SAFETENSORS;
      resolved = path;
      return LLRS_OK;
    }
    std::vector<std::string> ggufs;
    for (fs::directory_iterator it(p, ec), end; !ec && it != end; it.increment(ec))
      if (has_ext(it->path(), "gguf")) ggufs.push_back(it->path().string());
    std::sort(ggufs.begin(), ggufs.end());
    if (ggufs.size() == 1) {
      format = LLRS_FORMAT_GGUF;
      resolved = ggufs[0];
      return LLRS_OK;
    }
    if (ggufs.size() > 1)
      return set_error(LLRS_E_INVALID, "%s contains multiple GGUF files; pass the desired file explicitly",
                       path.c_str());
  }
  return set_error(LLRS_E_INVALID, "cannot detect model format at %s", path.c_str());
}

}  // namespace llrs

extern "C" int llrs_model_format(const char *path, int *format, char *resolved, size_t capacity) {
  using namespace llrs;
  clear_error();
  if (!path || !format) return set_error(LLRS_E_INVALID, "path and format must not be NULL");
  std::string r;
  LLRS_TRY(detect_model_format(path, *format, r));
  if (resolved) {
    if (r.size() + 1 > capacity)
      return set_error(LLRS_E_INVALID, "resolved path needs %zu bytes, capacity %zu", r.size() + 1, capacity);
    memcpy(resolved, r.c_str(), r.size() + 1);
  }
  return LLRS_OK;
}

extern "C" int llrs_hf_config_read(const char *config_json_path, llrs_model_config *out) {
  using namespace llrs;
  clear_error();
  if (!config_json_path || !out) return set_error(LLRS_E_INVALID, "arguments must not be NULL");
  return hf_config_read(config_json_path, *out);
}

extern "C" int llrs_safetensors_read_tensor(const char *model_dir, const char *name, uint32_t *ggml_type,
                                            size_t *shape, size_t *ndim, void *out, size_t out_capacity,
                                            size_t *nbytes) {
  using namespace llrs;
  clear_error();
  if (!model_dir || !name) return set_error(LLRS_E_INVALID, "model_dir and name must not be NULL");
  SafetensorStore st;
  LLRS_TRY(st.open(model_dir));
  const SafetensorsFile *f = nullptr;
  const SafetensorInfo *t = nullptr;
  LLRS_TRY(st.tensor(name, &f, &t));
  if (ggml_type) *ggml_type = t->dtype == "F32" ? LLRS_F32 : t->dtype == "F16" ? LLRS_F16 : LLRS_BF16;
  if (ndim) *ndim = t->shape.size();
  if (shape)
    for (size_t i = 0; i < t->shape.size(); i++) shape[i] = (size_t)t->shape[i];
  if (nbytes) *nbytes = t->nbytes;
  if (!out) return LLRS_OK;
  if (out_capacity < t->nbytes)
    return set_error(LLRS_E_INVALID, "output capacity %zu < %zu", out_capacity, t->nbytes);
  memcpy(out, f->data(*t), t->nbytes);
  return LLRS_OK;
}
