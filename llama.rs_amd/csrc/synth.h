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

// The model's tensors in generation order (the index keys each tensor's RNG).
std::vector<SynthSpec> synth_specs(const llrs_synth_config &c);
// GGML type that maybe_quantize assigns to a matrix (after fallbacks).
uint32_t recipe_type(int recipe, const std::string &name, uint64_t cols);
// The type a synthetic tensor is stored in (F32 for gains and biases).
uint32_t synth_type(const llrs_synth_config &c, const SynthSpec &spec);
// Generates tensor `index` on the host (values, then quantization) into `out`.
int synth_tensor(const llrs_synth_config &c, size_t index, const SynthSpec &spec,
                 GgufOutTensor &out);

}  // namespace llrs
