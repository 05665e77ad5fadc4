// Shared host-side definitions of the llrs HIP backend (C++ side of include/llrs.h).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/llrs.h"

namespace llrs {

// GGML block geometry, QuantType::block_size / type_size (src/quant.rs:46-67).
inline int block_size(uint32_t t) {
  switch (t) {
    case LLRS_F32: case LLRS_F16: case LLRS_BF16: return 1;
    case LLRS_Q4_0: case LLRS_Q4_1: case LLRS_Q5_0: case LLRS_Q5_1: case LLRS_Q8_0: return 32;
    case LLRS_Q4_K: case LLRS_Q5_K: case LLRS_Q6_K: return 256;
    default: return 0;
  }
}
inline int type_size(uint32_t t) {
  switch (t) {
    case LLRS_F32: return 4;
    case LLRS_F16: case LLRS_BF16: return 2;
    case LLRS_Q4_0: return 18;
    case LLRS_Q4_1: return 20;
    case LLRS_Q5_0: return 22;
    case LLRS_Q5_1: return 24;
    case LLRS_Q8_0: return 34;
    case LLRS_Q4_K: return 144;
    case LLRS_Q5_K: return 176;
    case LLRS_Q6_K: return 210;
    default: return 0;
  }
}
inline const char *type_name(uint32_t t) {
  switch (t) {
    case LLRS_F32: return "F32";
    case LLRS_F16: return "F16";
    case LLRS_BF16: return "BF16";
    case LLRS_Q4_0: return "Q4_0";
    case LLRS_Q4_1: return "Q4_1";
    case LLRS_Q5_0: return "Q5_0";
    case LLRS_Q5_1: return "Q5_1";
    case LLRS_Q8_0: return "Q8_0";
    case LLRS_Q4_K: return "Q4_K";
    case LLRS_Q5_K: return "Q5_K";
    case LLRS_Q6_K: return "Q6_K";
    default: return "?";
  }
}
inline size_t row_bytes(uint32_t t, size_t cols) {
  int bs = block_size(t);
  return bs ? cols / (size_t)bs * (size_t)type_size(t) : 0;
}

// Thread-local error text behind llrs_last_error().
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define LLRS_HIP(call)                                                                 \
  do {                                                                                 \
    hipError_t e_ = (call);                                                            \
    if (e_ != hipSuccess)                                                              \
      return ::llrs::set_error(e_ == hipErrorOutOfMemory ? LLRS_E_OOM : LLRS_E_HIP,    \
                               "%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), \
                               __FILE__, __LINE__);                                    \
  } while (0)

#define LLRS_TRY(call)          \
  do {                          \
    int r_ = (call);            \
    if (r_ != LLRS_OK) return r_; \
  } while (0)

// Tensor memory keeps this many zero bytes after the last row so that
// vectorised loads that round a row span outward never leave the allocation.
constexpr size_t kTensorTailPad = 256;

// Allocates an uninitialised device tensor of native layout (tail pad zeroed).
// The tensor holds a counted reference to its backend.
int tensor_alloc(llrs_backend *b, uint32_t ty, size_t rows, size_t cols, llrs_tensor **out);

// Counted ownership of a backend, as the reference's Arc<dyn KernelBackend>
// held by every model (src/model.rs:117, src/loader.rs:99, 242): the
// creator's handle, every tensor and every model hold one reference each,
// and the device state is released with the last of them, so destroying the
// backend handle while a model or cache still uses it only drops the handle.
void backend_retain(llrs_backend *b);
void backend_release(llrs_backend *b);

}  // namespace llrs

struct llrs_backend;
struct llrs_tensor;

struct llrs_backend {
  int device = 0;
  hipStream_t stream = nullptr;
  int cu_count = 0;
  int xcd_count = 8;
  std::string name;
  // Scratch device buffers for the host-pointer matvec entry point.
  float *x_dev = nullptr, *y_dev = nullptr;
  size_t x_cap = 0, y_cap = 0;
  std::atomic<int> refs{1};  // the creator's handle + one per tensor and model
};

struct llrs_tensor {
  llrs_backend *b = nullptr;
  uint32_t type = 0;
  size_t rows = 0, cols = 0, row_bytes = 0, nbytes = 0;
  uint8_t *dev = nullptr;  // native GGUF block bytes, rows contiguous, + kTensorTailPad
};
