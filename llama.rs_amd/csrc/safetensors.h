// Hugging Face checkpoint directories: the .safetensors format (the
// `safetensors` crate 0.4 that src/loader.rs:9 uses), the shard store
// (SafetensorStore, src/loader.rs:536-623), config.json (LlamaConfig,
// src/config.rs:17-90) and ModelLoader::load's format detection
// (src/loader.rs:44-77).  Host code only.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "llrs.h"

namespace llrs {

struct SafetensorInfo {
  std::string dtype;            // the header's dtype string ("F16", "BF16", "F32", ...)
  std::vector<uint64_t> shape;  // row-major, outermost first
  size_t start = 0, nbytes = 0; // absolute file range, validated at parse
};

// One .safetensors file, memory-mapped.  parse() restates
// SafeTensors::deserialize: an 8-byte little-endian header length (at most
// 100,000,000), a UTF-8 JSON object (whitespace around it allowed) whose members map
// tensor names to {dtype, shape, data_offsets} (plus an optional
// "__metadata__" map of strings), offsets that tile the data section
// exactly in offset order, and byte sizes equal to elements x dtype size.
class SafetensorsFile {
 public:
  ~SafetensorsFile();
  int open(const std::string &path);  // mmap only
  int parse();                        // validates; idempotent
  const SafetensorInfo *tensor(const std::string &name) const;
  const uint8_t *data(const SafetensorInfo &t) const { return map_ + t.start; }
  std::string path;
  std::map<std::string, SafetensorInfo> tensors;

 private:
  uint8_t *map_ = nullptr;
  size_t size_ = 0;
  bool parsed_ = false;
};

// The tensors of a checkpoint directory: the shards model.safetensors.index.json
// names (its weight_map), or else every *.safetensors file in the directory,
// where a name may appear only once.
class SafetensorStore {
 public:
  int open(const std::string &dir);
  bool contains(const std::string &name) const { return where_.count(name) != 0; }
  // The tensor's file and entry; errors name the tensor.
  int tensor(const std::string &name, const SafetensorsFile **file, const SafetensorInfo **info);

 private:
  std::map<std::string, std::unique_ptr<SafetensorsFile>> files_;
  std::map<std::string, std::string> where_;  // tensor name -> shard path
  bool indexed_ = false;
};

// Reads config.json: model_type must be "qwen2"; the LlamaConfig fields with
// their defaults (rms_norm_eps 1e-6, rope_theta 10000,
// max_position_embeddings 32768, head_dim hidden_size / heads,
// tie_word_embeddings false) and LlamaConfig::validate's checks.
int hf_config_read(const std::string &config_path, llrs_model_config &out);

// ModelLoader::load's choice for `path`: LLRS_FORMAT_GGUF with the file to
// open, or LLRS_FORMAT_SAFETENSORS with the checkpoint directory.
int detect_model_format(const std::string &path, int &format, std::string &resolved);

}  // namespace llrs
