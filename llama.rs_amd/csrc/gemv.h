// Launchers for the dequant-GEMV and dequantization kernels.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace llrs {

// y = W x (+ bias) (or y += W x when accumulate): every GGML type, any shape.
int launch_gemv_generic(const llrs_tensor *w, const float *x, float *y, const float *bias,
                        bool accumulate, hipStream_t s);
// out[c] = value_at(row, c) for c < cols, bit-exact.
int launch_dequant_row(const llrs_tensor *w, size_t row, float *out_dev, hipStream_t s);

}  // namespace llrs
