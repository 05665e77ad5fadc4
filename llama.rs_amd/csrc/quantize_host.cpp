// Load-time quantization on the host (QuantTensor::quantize_*,
// src/quant.rs:187-259): the shared encoders of quant_encode.h run on the CPU.
// Host-only code (no HIP calls), compiled with -ffp-contract=off so that its
// f32 arithmetic matches the GPU build of the same encoders bit for bit.
#include <cstring>
#include <vector>

#include "common.h"
#include "quant_encode.h"
#include "quantize.h"

namespace llrs {

uint16_t f32_to_f16_bits(float f) { return enc::f32_to_f16(f); }
float f16_bits_to_f32_host(uint16_t h) { return enc::f16_to_f32(h); }

uint32_t final_quant_type(uint32_t requested, size_t cols) {
  uint32_t ty = requested;
  if (ty == LLRS_Q4_K && cols % 256) ty = LLRS_Q5_0;  // quantize_q4k -> quantize_q5_0
  if (ty == LLRS_Q6_K && cols % 256) ty = LLRS_Q8_0;  // quantize_q6k -> quantize_q8_0
  if ((ty == LLRS_Q5_0 || ty == LLRS_Q8_0) && cols % 32) ty = LLRS_F32;
  return ty;
}

void encode_row(uint32_t ty, const float *v, size_t cols, uint8_t *out) {
  switch (ty) {
    case LLRS_Q4_K: for (size_t c = 0; c < cols; c += 256) enc::block_q4k(v + c, out + c / 256 * 144); break;
    case LLRS_Q6_K: for (size_t c = 0; c < cols; c += 256) enc::block_q6k(v + c, out + c / 256 * 210); break;
    case LLRS_Q5_0: for (size_t c = 0; c < cols; c += 32) enc::block_q5_0(v + c, out + c / 32 * 22); break;
    case LLRS_Q8_0: for (size_t c = 0; c < cols; c += 32) enc::block_q8_0(v + c, out + c / 32 * 34); break;
    default: memcpy(out, v, cols * 4); break;
  }
}

uint32_t quantize_rows(uint32_t requested, const float *values, size_t rows, size_t cols,
                       std::vector<uint8_t> &out) {
  uint32_t ty = final_quant_type(requested, cols);
  size_t rb = ty == LLRS_F32 ? cols * 4 : row_bytes(ty, cols);
  out.assign(rb * rows, 0);
  for (size_t r = 0; r < rows; r++) encode_row(ty, values + r * cols, cols, out.data() + r * rb);
  return ty;
}

}  // namespace llrs

extern "C" int llrs_quantize(uint32_t ggml_type, const float *values, size_t rows, size_t cols,
                             void *out, size_t out_capacity, size_t *out_nbytes,
                             uint32_t *out_type) {
  using namespace llrs;
  clear_error();
  if (ggml_type != LLRS_Q4_K && ggml_type != LLRS_Q5_0 && ggml_type != LLRS_Q8_0 &&
      ggml_type != LLRS_Q6_K)
    return set_error(LLRS_E_UNSUPPORTED, "llrs_quantize supports Q4_K, Q5_0, Q8_0 and Q6_K");
  if (!values && rows * cols) return set_error(LLRS_E_INVALID, "values is NULL");
  uint32_t ty = final_quant_type(ggml_type, cols);
  size_t need = ty == LLRS_F32 ? rows * cols * 4 : row_bytes(ty, cols) * rows;
  if (out_nbytes) *out_nbytes = need;
  if (out_type) *out_type = ty;
  if (!out) return LLRS_OK;
  if (out_capacity < need)
    return set_error(LLRS_E_INVALID, "output capacity %zu < %zu", out_capacity, need);
  std::vector<uint8_t> buf;
  quantize_rows(ggml_type, values, rows, cols, buf);
  memcpy(out, buf.data(), need);
  return LLRS_OK;
}
