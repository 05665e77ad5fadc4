// Host-side GGML quantizers (restated from src/quant.rs:187-259, 650-967).
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "common.h"

namespace llrs {

uint16_t f32_to_f16_bits(float f);
float f16_bits_to_f32_host(uint16_t h);

// Quantizes `rows` rows of `cols` values with the reference's entry point for
// `requested` (LLRS_Q4_K / Q6_K / Q5_0 / Q8_0), applying its fallbacks; the
// native block bytes go to `out` and the type actually produced is returned.
uint32_t quantize_rows(uint32_t requested, const float *values, size_t rows, size_t cols,
                       std::vector<uint8_t> &out);

}  // namespace llrs
