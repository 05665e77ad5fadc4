// GGUF v2/v3 reader and v3 writer.
//
// The reader enforces the reference's checks (src/gguf.rs:78-250, 339-369):
// magic, version 2..3, header counts <= 1e6, metadata types 0-12 (arrays are
// walked and skipped, nested arrays rejected), string length <= 2^30, array
// length <= 1e8, 1..4 dimensions, duplicate keys/tensors, power-of-two
// alignment <= 2^20 (default 32), and every tensor range validated eagerly.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>

#include "common.h"

namespace llrs {

bool GgufValue::as_u64(uint64_t &out) const {
  if (kind == U64) { out = u; return true; }
  if (kind == I64 && i >= 0) { out = (uint64_t)i; return true; }
  return false;
}
bool GgufValue::as_f32(float &out) const {
  if (kind == F64) { out = (float)f; return true; }
  if (kind == U64) { out = (float)u; return true; }
  if (kind == I64) { out = (float)i; return true; }
  return false;
}

namespace {
struct Reader {
  const uint8_t *d;
  size_t n, pos = 0;
  bool err = false;
  const uint8_t *take(size_t len) {
    if (err || pos > n || len > n - pos) {
      if (!err) set_error(LLRS_E_FORMAT, "truncated GGUF file at byte %zu", pos);
      err = true;
      return nullptr;
    }
    const uint8_t *p = d + pos;
    pos += len;
    return p;
  }
  uint64_t le(int bytes) {
    const uint8_t *p = take((size_t)bytes);
    uint64_t v = 0;
    if (p)
      for (int k = bytes - 1; k >= 0; k--) v = (v << 8) | p[k];
    return v;
  }
  bool str(std::string &out) {
    uint64_t len = le(8);
    if (err) return false;
    if (len > (1ull << 30)) {
      set_error(LLRS_E_FORMAT, "unreasonable GGUF string length %llu", (unsigned long long)len);
      err = true;
      return false;
    }
    const uint8_t *p = take((size_t)len);
    if (!p) return false;
    out.assign((const char *)p, (size_t)len);
    return true;
  }
  bool value(uint32_t ty, GgufValue &v) {
    switch (ty) {
      case 0: v.kind = GgufValue::U64; v.u = le(1); break;
      case 1: v.kind = GgufValue::I64; v.i = (int8_t)le(1); break;
      case 2: v.kind = GgufValue::U64; v.u = le(2); break;
      case 3: v.kind = GgufValue::I64; v.i = (int16_t)le(2); break;
      case 4: v.kind = GgufValue::U64; v.u = le(4); break;
      case 5: v.kind = GgufValue::I64; v.i = (int32_t)le(4); break;
      case 6: {
        uint32_t b = (uint32_t)le(4);
        float f;
        memcpy(&f, &b, 4);
        v.kind = GgufValue::F64;
        v.f = f;
        break;
      }
      case 7: v.kind = GgufValue::BOOL; v.u = le(1) != 0; break;
      case 8: v.kind = GgufValue::STR; if (!str(v.s)) return false; break;
      case 9: {
        uint32_t et = (uint32_t)le(4);
        if (err) return false;
        if (et == 9) {
          set_error(LLRS_E_FORMAT, "nested GGUF arrays are not supported by the format");
          return false;
        }
        uint64_t len = le(8);
        if (err) return false;
        if (len > 100000000ull) {
          set_error(LLRS_E_FORMAT, "unreasonable GGUF array length %llu", (unsigned long long)len);
          return false;
        }
        for (uint64_t k = 0; k < len; k++) {
          GgufValue tmp;
          if (!value(et, tmp)) return false;
        }
        v.kind = GgufValue::ARRAY;
        v.array_type = et;
        v.array_len = len;
        break;
      }
      case 10: v.kind = GgufValue::U64; v.u = le(8); break;
      case 11: v.kind = GgufValue::I64; v.i = (int64_t)le(8); break;
      case 12: {
        uint64_t b = le(8);
        memcpy(&v.f, &b, 8);
        v.kind = GgufValue::F64;
        break;
      }
      default: set_error(LLRS_E_FORMAT, "unknown GGUF metadata type %u", ty); return false;
    }
    return !err;
  }
};
}  // namespace

GgufFile::~GgufFile() {
  if (map_) munmap(map_, size_);
}

int GgufFile::open(const std::string &path) {
  int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) return set_error(LLRS_E_IO, "failed to open %s", path.c_str());
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return set_error(LLRS_E_IO, "failed to stat %s", path.c_str());
  }
  size_ = (size_t)st.st_size;
  if (size_) {
    void *p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      ::close(fd);
      return set_error(LLRS_E_IO, "failed to mmap %s", path.c_str());
    }
    map_ = (uint8_t *)p;
  }
  ::close(fd);
  Reader r{map_, size_};
  const uint8_t *magic = r.take(4);
  if (!magic || memcmp(magic, "GGUF", 4) != 0)
    return set_error(LLRS_E_FORMAT, "%s is not a GGUF file", path.c_str());
  version = (uint32_t)r.le(4);
  if (r.err) return LLRS_E_FORMAT;
  if (version < 2 || version > 3)
    return set_error(LLRS_E_FORMAT, "unsupported GGUF version %u; versions 2 and 3 are supported",
                     version);
  uint64_t nt = r.le(8), nm = r.le(8);
  if (r.err) return LLRS_E_FORMAT;
  if (nt > 1000000 || nm > 1000000) return set_error(LLRS_E_FORMAT, "unreasonable GGUF header counts");
  for (uint64_t k = 0; k < nm; k++) {
    std::string key;
    if (!r.str(key)) return LLRS_E_FORMAT;
    uint32_t ty = (uint32_t)r.le(4);
    if (r.err) return LLRS_E_FORMAT;
    GgufValue v;
    if (!r.value(ty, v)) return LLRS_E_FORMAT;
    if (!metadata.emplace(key, v).second)
      return set_error(LLRS_E_FORMAT, "duplicate GGUF metadata key %s", key.c_str());
  }
  for (uint64_t k = 0; k < nt; k++) {
    GgufTensorInfo t;
    if (!r.str(t.name)) return LLRS_E_FORMAT;
    uint32_t nd = (uint32_t)r.le(4);
    if (r.err) return LLRS_E_FORMAT;
    if (nd < 1 || nd > 4)
      return set_error(LLRS_E_FORMAT, "tensor %s has invalid dimension count %u", t.name.c_str(), nd);
    for (uint32_t i = 0; i < nd; i++) t.dims.push_back(r.le(8));
    t.type = (uint32_t)r.le(4);
    t.offset = r.le(8);
    if (r.err) return LLRS_E_FORMAT;
    std::string name = t.name;
    if (!tensors.emplace(name, t).second)
      return set_error(LLRS_E_FORMAT, "duplicate GGUF tensor %s", name.c_str());
  }
  uint64_t alignment = 32;
  if (const GgufValue *al = meta("general.alignment")) {
    uint64_t a;
    if (al->as_u64(a)) alignment = a;
  }
  if (alignment == 0 || (alignment & (alignment - 1)) || alignment > (1u << 20))
    return set_error(LLRS_E_FORMAT, "invalid GGUF alignment %llu", (unsigned long long)alignment);
  data_offset_ = (r.pos + (size_t)alignment - 1) & ~((size_t)alignment - 1);
  if (data_offset_ > size_) return set_error(LLRS_E_FORMAT, "GGUF tensor data offset is outside the file");
  // tensor_range for every tensor (src/gguf.rs:164-167, 217-250).
  for (auto &kv : tensors) {
    GgufTensorInfo &t = kv.second;
    int bs = block_size(t.type);
    if (!bs)
      return set_error(LLRS_E_UNSUPPORTED, "tensor %s: unsupported GGML tensor type %u",
                       t.name.c_str(), t.type);
    unsigned __int128 el = 1;
    for (uint64_t d : t.dims) {
      el *= d;
      if (el > (unsigned __int128)SIZE_MAX)
        return set_error(LLRS_E_FORMAT, "tensor %s element count overflow", t.name.c_str());
    }
    size_t elements = (size_t)el;
    if (elements % (size_t)bs)
      return set_error(LLRS_E_FORMAT, "tensor %s element count is incompatible with %s",
                       t.name.c_str(), type_name(t.type));
    if (t.dims[0] % (uint64_t)bs)
      return set_error(LLRS_E_FORMAT, "tensor %s row width %llu is incompatible with %s",
                       t.name.c_str(), (unsigned long long)t.dims[0], type_name(t.type));
    size_t len = elements / (size_t)bs * (size_t)type_size(t.type);
    if (t.offset > SIZE_MAX - data_offset_)
      return set_error(LLRS_E_FORMAT, "tensor %s offset overflow", t.name.c_str());
    size_t start = data_offset_ + (size_t)t.offset;
    if (start > size_ || len > size_ - start)
      return set_error(LLRS_E_FORMAT, "tensor %s is outside the GGUF file", t.name.c_str());
    t.start = start;
    t.nbytes = len;
  }
  return LLRS_OK;
}

const GgufValue *GgufFile::meta(const std::string &key) const {
  auto it = metadata.find(key);
  return it == metadata.end() ? nullptr : &it->second;
}
const GgufTensorInfo *GgufFile::tensor(const std::string &name) const {
  auto it = tensors.find(name);
  return it == tensors.end() ? nullptr : &it->second;
}

static void put_le(std::vector<uint8_t> &o, uint64_t v, int n) {
  for (int k = 0; k < n; k++) o.push_back((uint8_t)(v >> (8 * k)));
}
static void put_str(std::vector<uint8_t> &o, const std::string &s) {
  put_le(o, s.size(), 8);
  o.insert(o.end(), s.begin(), s.end());
}

void GgufWriter::add_u32(const std::string &k, uint32_t v) {
  put_str(meta_, k);
  put_le(meta_, 4, 4);
  put_le(meta_, v, 4);
  n_meta_++;
}
void GgufWriter::add_f32(const std::string &k, float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  put_str(meta_, k);
  put_le(meta_, 6, 4);
  put_le(meta_, b, 4);
  n_meta_++;
}
void GgufWriter::add_str(const std::string &k, const std::string &v) {
  put_str(meta_, k);
  put_le(meta_, 8, 4);
  put_str(meta_, v);
  n_meta_++;
}

int GgufWriter::write(const std::string &path, const std::vector<GgufOutTensor> &tensors) const {
  std::vector<size_t> sizes;
  for (const auto &t : tensors) sizes.push_back(t.bytes.size());
  return write_streamed(path, tensors, sizes, [&](size_t i, std::vector<uint8_t> &buf) {
    buf = tensors[i].bytes;
    return (int)LLRS_OK;
  });
}

int GgufWriter::write_streamed(const std::string &path, const std::vector<GgufOutTensor> &tensors,
                               const std::vector<size_t> &nbytes,
                               const std::function<int(size_t, std::vector<uint8_t> &)> &fetch) const {
  const size_t align = 32;
  std::vector<uint8_t> head;
  head.insert(head.end(), {'G', 'G', 'U', 'F'});
  put_le(head, 3, 4);
  put_le(head, tensors.size(), 8);
  put_le(head, n_meta_, 8);
  head.insert(head.end(), meta_.begin(), meta_.end());
  uint64_t off = 0;
  for (size_t i = 0; i < tensors.size(); i++) {
    const auto &t = tensors[i];
    put_str(head, t.name);
    put_le(head, t.dims.size(), 4);
    for (uint64_t d : t.dims) put_le(head, d, 8);
    put_le(head, t.type, 4);
    put_le(head, off, 8);
    off += (nbytes[i] + align - 1) / align * align;
  }
  while (head.size() % align) head.push_back(0);
  FILE *f = fopen(path.c_str(), "wb");
  if (!f) return set_error(LLRS_E_IO, "failed to create %s", path.c_str());
  bool ok = fwrite(head.data(), 1, head.size(), f) == head.size();
  static const uint8_t zeros[32] = {0};
  std::vector<uint8_t> buf;
  int rc = LLRS_OK;
  for (size_t i = 0; i < tensors.size() && ok; i++) {
    rc = fetch(i, buf);
    if (rc != LLRS_OK || buf.size() != nbytes[i]) {
      ok = false;
      break;
    }
    ok = fwrite(buf.data(), 1, buf.size(), f) == buf.size();
    size_t pad = (align - buf.size() % align) % align;
    if (ok && pad) ok = fwrite(zeros, 1, pad, f) == pad;
  }
  if (fclose(f) != 0) ok = false;
  if (rc != LLRS_OK) return rc;
  if (!ok) return set_error(LLRS_E_IO, "failed to write %s", path.c_str());
  return LLRS_OK;
}

}  // namespace llrs

extern "C" int llrs_gguf_read_tensor(const char *path, const char *name, uint32_t *version,
                                     uint32_t *ggml_type, size_t *rows, size_t *cols, void *out,
                                     size_t out_capacity, size_t *nbytes) {
  using namespace llrs;
  clear_error();
  if (!path || !name) return set_error(LLRS_E_INVALID, "path/name is NULL");
  GgufFile g;
  LLRS_TRY(g.open(path));
  const GgufTensorInfo *t = g.tensor(name);
  if (!t) return set_error(LLRS_E_INVALID, "missing GGUF tensor %s", name);
  if (t->dims.size() > 2)
    return set_error(LLRS_E_INVALID, "tensor %s has %zu dimensions; Qwen2 loader supports 1D/2D weights",
                     name, t->dims.size());
  if (version) *version = g.version;
  if (ggml_type) *ggml_type = t->type;
  if (rows) *rows = t->dims.size() == 2 ? (size_t)t->dims[1] : 1;
  if (cols) *cols = (size_t)t->dims[0];
  if (nbytes) *nbytes = t->nbytes;
  if (!out) return LLRS_OK;
  if (out_capacity < t->nbytes)
    return set_error(LLRS_E_INVALID, "output capacity %zu < %zu", out_capacity, t->nbytes);
  memcpy(out, g.data(*t), t->nbytes);
  return LLRS_OK;
}
