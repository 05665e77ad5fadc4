// The engine's end-of-sequence discovery (find_eos_tokens,
// src/engine.rs:340-387): host-only, no GPU.
//
// model_dir(path) is the path itself when it is a directory, else its parent
// (src/engine.rs:340-346).  generation_config.json there, when it exists,
// contributes "eos_token_id" (a number, or an array whose numeric entries
// count; values that are not non-negative integers fitting 32 bits are
// skipped, as serde_json's as_u64 + u32::try_from skip them).  Then the ids of
// "<|im_end|>" and "<|endoftext|>" in tokenizer.json, looked up as the
// tokenizers crate's Tokenizer::token_to_id does: the added tokens first,
// then the model's vocabulary (an object of token -> id for BPE, WordPiece
// and WordLevel models, an array of [token, score] pairs indexed by id for
// Unigram).  The result is sorted and deduplicated.  The reference loads
// tokenizer.json before this (InferenceEngine::from_path, src/engine.rs:61-63),
// so a missing or malformed one is an error here too.
#include <sys/stat.h>

#include <algorithm>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "common.h"
#include "json.h"

namespace llrs {

namespace {

bool is_dir(const std::string &p) {
  struct stat st;
  return stat(p.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
}
bool exists(const std::string &p) {
  struct stat st;
  return stat(p.c_str(), &st) == 0;
}

std::string model_dir(const std::string &path) {
  if (is_dir(path)) return path;
  const size_t slash = path.find_last_of('/');
  if (slash == std::string::npos) return ".";
  return slash == 0 ? "/" : path.substr(0, slash);
}

int read_json(const std::string &file, const char *what, JsonValue &out) {
  std::ifstream in(file, std::ios::binary);
  if (!in) return set_error(LLRS_E_IO, "failed to %s %s", what, file.c_str());
  std::stringstream ss;
  ss << in.rdbuf();
  const std::string text = ss.str();
  std::string err;
  if (!json_parse(text.data(), text.size(), out, err))
    return set_error(LLRS_E_FORMAT, "failed to parse %s: %s", file.c_str(), err.c_str());
  return LLRS_OK;
}

void push_id(const JsonValue &v, std::vector<uint32_t> &ids) {
  uint64_t u = 0;
  if (v.kind == JsonValue::NUMBER && v.as_u64(u) && u <= 0xffffffffull) ids.push_back((uint32_t)u);
}

// Tokenizer::token_to_id: added tokens, then the model's vocabulary.
bool token_to_id(const JsonValue &tok, const std::string &token, uint32_t &id) {
  if (const JsonValue *added = tok.get("added_tokens"); added && added->kind == JsonValue::ARRAY) {
    for (const JsonValue &a : added->items) {
      const JsonValue *c = a.get("content"), *i = a.get("id");
      uint64_t u = 0;
      if (c && c->kind == JsonValue::STRING && c->text == token && i && i->as_u64(u) &&
          u <= 0xffffffffull) {
        id = (uint32_t)u;
        return true;
      }
    }
  }
  const JsonValue *model = tok.get("model");
  const JsonValue *vocab = model ? model->get("vocab") : nullptr;
  if (!vocab) return false;
  if (vocab->kind == JsonValue::OBJECT) {
    if (const JsonValue *v = vocab->get(token)) {
      uint64_t u = 0;
      if (v->as_u64(u) && u <= 0xffffffffull) {
        id = (uint32_t)u;
        return true;
      }
    }
    return false;
  }
  if (vocab->kind == JsonValue::ARRAY) {  // Unigram: [token, score] pairs, id = index
    for (size_t i = 0; i < vocab->items.size(); i++) {
      const JsonValue &e = vocab->items[i];
      if (e.kind == JsonValue::ARRAY && !e.items.empty() && e.items[0].kind == JsonValue::STRING &&
          e.items[0].text == token) {
        id = (uint32_t)i;
        return true;
      }
    }
  }
  return false;
}

}  // namespace

}  // namespace llrs

using namespace llrs;

extern "C" int llrs_find_eos_tokens(const char *model_path, uint32_t *out, size_t capacity,
                                    size_t *n_out) {
  clear_error();
  if (!model_path || !n_out || (capacity && !out))
    return set_error(LLRS_E_INVALID, "model_path/out/n_out is NULL");
  *n_out = 0;
  const std::string dir = model_dir(model_path);
  std::vector<uint32_t> ids;
  const std::string gen = dir + "/generation_config.json";
  if (exists(gen)) {
    JsonValue g;
    LLRS_TRY(read_json(gen, "read", g));
    if (const JsonValue *eos = g.get("eos_token_id")) {
      if (eos->kind == JsonValue::NUMBER) push_id(*eos, ids);
      if (eos->kind == JsonValue::ARRAY)
        for (const JsonValue &v : eos->items) push_id(v, ids);
    }
  }
  JsonValue tok;
  LLRS_TRY(read_json(dir + "/tokenizer.json", "load", tok));
  for (const char *t : {"<|im_end|>", "<|endoftext|>"}) {
    uint32_t id = 0;
    if (token_to_id(tok, t, id)) ids.push_back(id);
  }
  std::sort(ids.begin(), ids.end());
  ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
  *n_out = ids.size();
  if (capacity < ids.size() && out)
    return set_error(LLRS_E_INVALID, "%zu EOS ids do not fit a buffer of %zu", ids.size(), capacity);
  if (out) std::copy(ids.begin(), ids.end(), out);
  return LLRS_OK;
}
