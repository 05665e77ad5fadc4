// A small JSON (RFC 8259) reader for the three JSON documents a Hugging Face
// checkpoint directory holds: config.json, model.safetensors.index.json and
// each .safetensors header.  Numbers keep their text so that integer fields
// can be read exactly (as serde_json reads a usize: a non-negative integer
// with no fraction or exponent).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace llrs {

struct JsonValue {
  enum Kind { NUL, BOOL, NUMBER, STRING, ARRAY, OBJECT } kind = NUL;
  bool b = false;
  std::string text;  // STRING: the decoded string; NUMBER: the number's lexeme
  std::vector<JsonValue> items;                             // ARRAY
  std::vector<std::pair<std::string, JsonValue>> members;  // OBJECT, in document order

  // OBJECT member by key (the last one if the key repeats, as serde_json's
  // map deserialisation keeps), or nullptr.
  const JsonValue *get(const std::string &key) const;
  // NUMBER written as a non-negative integer that fits 64 bits.
  bool as_u64(uint64_t &out) const;
  // Any NUMBER, rounded to the nearest double.
  bool as_f64(double &out) const;
};

// Parses a whole document (surrounding whitespace allowed).  Returns false
// and fills `error` ("... at byte N") on malformed input or nesting deeper
// than 128 levels.
bool json_parse(const char *data, size_t n, JsonValue &out, std::string &error);

}  // namespace llrs
