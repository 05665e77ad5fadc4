// Synthetic Qwen2 model generation (seeded random-init + load-time recipes).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "common.h"
#include "gguf.h"

namespace llrs {

struct SynthSpec {
  std::string name;
  uint64_t rows, cols;
  enum Kind { MATRIX, GAIN, BIAS } kind;
};

// The model's tensors in generation order (the index keys each RNG stream).
std::vector<SynthSpec> synth_specs(const llrs_synth_config &c);
// GGML type that the recipe assigns to a matrix (after fallbacks).
uint32_t recipe_type(int recipe, const std::string &name, uint64_t cols);
// Generates tensor `index` (values, then quantization) into `out`.
int synth_tensor(const llrs_synth_config &c, size_t index, const SynthSpec &spec,
                 GgufOutTensor &out);
void synth_normals(uint64_t seed, uint64_t tensor, uint64_t row, float *out, size_t n);

}  // namespace llrs
