// GGUF v2/v3 reader and v3 writer (the format of src/gguf.rs).
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <string>
#include <vector>

namespace llrs {

struct GgufValue {
  enum Kind { U64, I64, F64, BOOL, STR, ARRAY } kind = U64;
  uint64_t u = 0;
  int64_t i = 0;
  double f = 0;
  std::string s;
  uint32_t array_type = 0;
  uint64_t array_len = 0;
  bool as_u64(uint64_t &out) const;
  bool as_f32(float &out) const;
};

struct GgufTensorInfo {
  std::string name;
  std::vector<uint64_t> dims;  // GGML order: dims[0] is the contiguous row width
  uint32_t type = 0;
  uint64_t offset = 0;
  size_t start = 0, nbytes = 0;  // absolute file range, validated at open
};

class GgufFile {
 public:
  ~GgufFile();
  // GgufFile::open (src/gguf.rs:78-169); returns an LLRS_E_* code and sets the error text.
  int open(const std::string &path);
  const GgufValue *meta(const std::string &key) const;
  const GgufTensorInfo *tensor(const std::string &name) const;
  const uint8_t *data(const GgufTensorInfo &t) const { return map_ + t.start; }
  uint32_t version = 0;
  std::map<std::string, GgufValue> metadata;
  std::map<std::string, GgufTensorInfo> tensors;

 private:
  uint8_t *map_ = nullptr;
  size_t size_ = 0;
  size_t data_offset_ = 0;
};

// A tensor to be written: GGML dims order, native bytes.
struct GgufOutTensor {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  std::vector<uint8_t> bytes;
};

class GgufWriter {
 public:
  void add_u32(const std::string &k, uint32_t v);
  void add_f32(const std::string &k, float v);
  void add_str(const std::string &k, const std::string &v);
  // Writes header, metadata, tensor table and 32-byte aligned data.
  int write(const std::string &path, const std::vector<GgufOutTensor> &tensors) const;
  // Streaming form: `tensors` carry name/dims/type only; `nbytes[i]` is the
  // size of tensor i and fetch(i, buf) fills its bytes just before writing.
  int write_streamed(const std::string &path, const std::vector<GgufOutTensor> &tensors,
                     const std::vector<size_t> &nbytes,
                     const std::function<int(size_t, std::vector<uint8_t> &)> &fetch) const;

 private:
  std::vector<uint8_t> meta_;
  uint64_t n_meta_ = 0;
};

}  // namespace llrs
