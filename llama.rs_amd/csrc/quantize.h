// Quantizers (host) and synthetic-weight / encode kernels (device).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "common.h"

namespace llrs {

uint16_t f32_to_f16_bits(float f);
float f16_bits_to_f32_host(uint16_t h);

// The type the reference's quantize_* entry point for `requested` produces
// at row width `cols`, after its fallbacks (src/quant.rs:190-259).
uint32_t final_quant_type(uint32_t requested, size_t cols);
// Encodes one row of `cols` values as type `ty` (a final type) into out.
void encode_row(uint32_t ty, const float *v, size_t cols, uint8_t *out);
// Quantizes `rows` rows with the entry point for `requested`; returns the type produced.
uint32_t quantize_rows(uint32_t requested, const float *values, size_t rows, size_t cols,
                       std::vector<uint8_t> &out);

// GPU: generates and encodes a synthetic tensor (type ty, final) directly in HBM.
int launch_synth_encode(uint32_t ty, uint64_t key, size_t rows, size_t cols, float sd, bool gain,
                        uint8_t *out, size_t rbytes, hipStream_t s);
// GPU: encodes device f32 rows as ty (Q4_K, Q6_K, Q5_0 or Q8_0).
int launch_encode(uint32_t ty, const float *vals, size_t rows, size_t cols, uint8_t *out,
                  size_t rbytes, hipStream_t s);

// GPU: n F16 or BF16 values (device) widened to f32.
int launch_widen(uint32_t ty, const void *src, size_t n, float *dst, hipStream_t s);

}  // namespace llrs
