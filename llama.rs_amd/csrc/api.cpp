// C ABI: backend, tensors, matvec (include/llrs.h).
//
// HipBackend is the MI355X counterpart of CpuBackend (src/backend.rs:97-163):
// it owns one HIP device and one stream instead of a rayon pool.  Tensors are
// uploaded once in their native GGUF block layout (src/quant.rs:86-157).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <new>

#include "common.h"
#include "decode.h"
#include "gemv.h"

namespace llrs {


static int ensure_scratch(llrs_backend *b, size_t nx, size_t ny) {
  if (nx > b->x_cap) {
    if (b->x_dev) LLRS_HIP(hipFree(b->x_dev));
    b->x_dev = nullptr;
    b->x_cap = 0;
    LLRS_HIP(hipMalloc(&b->x_dev, nx * sizeof(float)));
    b->x_cap = nx;
  }
  if (ny > b->y_cap) {
    if (b->y_dev) LLRS_HIP(hipFree(b->y_dev));
    b->y_dev = nullptr;
    b->y_cap = 0;
    LLRS_HIP(hipMalloc(&b->y_dev, ny * sizeof(float)));
    b->y_cap = ny;
  }
  return LLRS_OK;
}

// y = W x on the device: the tuned kernel for the types and widths it covers,
// the generic kernel otherwise (or when LLRS_GENERIC_GEMV is set).
static int launch_matvec(llrs_backend *b, const llrs_tensor *w, const float *x, float *y) {
  const char *e = getenv("LLRS_GENERIC_GEMV");
  bool generic = e && *e && *e != '0';
  if (generic || !fast_gemv_supports(w->type, w->cols) || w->rows > (size_t)INT32_MAX)
    return launch_gemv_generic(w, x, y, nullptr, false, b->stream);
  FastGemvArgs a{};
  a.seg[0].w = w->dev;
  a.seg[0].type = w->type;
  a.seg[0].rows = (int)w->rows;
  a.seg[0].row_bytes = (long)w->row_bytes;
  a.seg[0].out = y;
  a.nseg = 1;
  a.rows = (int)w->rows;
  a.cols = (int)w->cols;
  a.x = x;
  a.epi = kEpiStore;
  {  // the balanced split (LLRS_BAL=0 turns it off)
    const char *eb = getenv("LLRS_BAL");
    a.bal = !(eb && *eb == '0');
  }
  // One 512-thread workgroup per CU (two waves per SIMD, one digitised x per
  // CU): measured faster than 256-thread blocks at one to three per CU on
  // every tuned type at 18944 x 3584 and 3584 x 18944.
  const int grid = std::min(b->cu_count, fast_gemv_grid(b->cu_count, a.rows, a.cols, false, 0));
  return launch_gemv_fast(a, grid, b->stream, 512);
}

// validate_matvec (src/quant.rs:303-318).
static int validate_matvec(const llrs_tensor *w, size_t nx, size_t ny) {
  if (nx != w->cols)
    return set_error(LLRS_E_INVALID, "matvec input mismatch: got %zu, expected %zu", nx, w->cols);
  if (ny != w->rows)
    return set_error(LLRS_E_INVALID, "matvec output mismatch: got %zu, expected %zu", ny, w->rows);
  return LLRS_OK;
}

int tensor_alloc(llrs_backend *b, uint32_t ty, size_t rows, size_t cols, llrs_tensor **out) {
  *out = nullptr;
  llrs_tensor *t = new (std::nothrow) llrs_tensor();
  if (!t) return set_error(LLRS_E_OOM, "out of host memory");
  t->b = b;
  backend_retain(b);
  t->type = ty;
  t->rows = rows;
  t->cols = cols;
  t->row_bytes = row_bytes(ty, cols);
  t->nbytes = t->row_bytes * rows;
  hipError_t e = hipMalloc(&t->dev, t->nbytes + kTensorTailPad);
  if (e != hipSuccess) {
    backend_release(b);
    delete t;
    return set_error(e == hipErrorOutOfMemory ? LLRS_E_OOM : LLRS_E_HIP,
                     "hipMalloc(%zu) failed: %s", rows * row_bytes(ty, cols) + kTensorTailPad,
                     hipGetErrorString(e));
  }
  e = hipMemsetAsync(t->dev + t->nbytes, 0, kTensorTailPad, b->stream);
  if (e != hipSuccess) {
    (void)hipFree(t->dev);
    backend_release(b);
    delete t;
    return set_error(LLRS_E_HIP, "hipMemsetAsync failed: %s", hipGetErrorString(e));
  }
  *out = t;
  return LLRS_OK;
}

void backend_retain(llrs_backend *b) { b->refs.fetch_add(1, std::memory_order_relaxed); }

void backend_release(llrs_backend *b) {
  if (b->refs.fetch_sub(1, std::memory_order_acq_rel) != 1) return;
  (void)hipSetDevice(b->device);
  (void)hipStreamSynchronize(b->stream);
  if (b->x_dev) (void)hipFree(b->x_dev);
  if (b->y_dev) (void)hipFree(b->y_dev);
  (void)hipStreamDestroy(b->stream);
  delete b;
}

}  // namespace llrs

using namespace llrs;

extern "C" {


int llrs_backend_create(const llrs_backend_config *cfg, llrs_backend **out) {
  clear_error();
  if (!out) return set_error(LLRS_E_INVALID, "out is NULL");
  *out = nullptr;
  int device = cfg ? cfg->device : 0;
  if (cfg && cfg->flags) return set_error(LLRS_E_INVALID, "llrs_backend_config.flags must be 0");
  int count = 0;
  LLRS_HIP(hipGetDeviceCount(&count));
  if (device < 0 || device >= count)
    return set_error(LLRS_E_INVALID, "HIP device %d out of range (%d devices)", device, count);
  LLRS_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  LLRS_HIP(hipGetDeviceProperties(&prop, device));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(LLRS_E_UNSUPPORTED, "device %d is %s; this backend is built for gfx950 only",
                     device, prop.gcnArchName);
  llrs_backend *b = new (std::nothrow) llrs_backend();
  if (!b) return set_error(LLRS_E_OOM, "out of host memory");
  b->device = device;
  b->cu_count = prop.multiProcessorCount;
  b->name = "hip-gfx950";
  hipError_t e = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete b;
    return set_error(LLRS_E_HIP, "hipStreamCreate failed: %s", hipGetErrorString(e));
  }
  *out = b;
  return LLRS_OK;
}

// Releases the creator's handle; models, caches and tensors made from the
// backend keep it alive until they are freed.
void llrs_backend_destroy(llrs_backend *b) {
  if (b) backend_release(b);
}

const char *llrs_backend_name(const llrs_backend *b) { return b ? b->name.c_str() : ""; }
size_t llrs_backend_threads(const llrs_backend *b) { return b ? (size_t)b->cu_count : 0; }

int llrs_backend_synchronize(llrs_backend *b) {
  clear_error();
  if (!b) return set_error(LLRS_E_INVALID, "backend is NULL");
  LLRS_HIP(hipStreamSynchronize(b->stream));
  return LLRS_OK;
}

int llrs_tensor_upload(llrs_backend *b, const void *bytes, size_t nbytes, uint32_t ty, size_t rows,
                       size_t cols, llrs_tensor **out) {
  clear_error();
  if (!b || !out) return set_error(LLRS_E_INVALID, "backend/out is NULL");
  *out = nullptr;
  int bs = block_size(ty);
  if (!bs)
    return set_error(LLRS_E_UNSUPPORTED,
                     "unsupported GGML tensor type %u; supported: F32, F16, BF16, Q4_0, Q4_1, "
                     "Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K",
                     ty);
  if (cols % (size_t)bs)
    return set_error(LLRS_E_INVALID, "last dimension %zu is not divisible by %d for %s", cols, bs,
                     type_name(ty));
  if (cols > (size_t)1 << 30 || rows > (size_t)1 << 31)
    return set_error(LLRS_E_INVALID, "tensor shape [%zu, %zu] is too large", rows, cols);
  size_t expected = rows * cols / (size_t)bs * (size_t)type_size(ty);
  if (nbytes != expected)
    return set_error(LLRS_E_INVALID, "bad %s tensor byte length: got %zu, expected %zu",
                     type_name(ty), nbytes, expected);
  if (nbytes && !bytes) return set_error(LLRS_E_INVALID, "bytes is NULL");
  LLRS_HIP(hipSetDevice(b->device));
  llrs_tensor *t = nullptr;
  LLRS_TRY(tensor_alloc(b, ty, rows, cols, &t));
  hipError_t e = hipSuccess;
  if (nbytes)
    e = hipMemcpyAsync(t->dev, bytes, nbytes, hipMemcpyHostToDevice, b->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(b->stream);
  if (e != hipSuccess) {
    llrs_tensor_free(t);
    return set_error(LLRS_E_HIP, "tensor upload failed: %s", hipGetErrorString(e));
  }
  *out = t;
  return LLRS_OK;
}

void llrs_tensor_free(llrs_tensor *t) {
  if (!t) return;
  llrs_backend *b = t->b;
  (void)hipSetDevice(b->device);
  (void)hipStreamSynchronize(b->stream);
  (void)hipFree(t->dev);
  delete t;
  backend_release(b);
}

int llrs_tensor_info(const llrs_tensor *t, uint32_t *ty, size_t *rows, size_t *cols,
                     size_t *nbytes) {
  clear_error();
  if (!t) return set_error(LLRS_E_INVALID, "tensor is NULL");
  if (ty) *ty = t->type;
  if (rows) *rows = t->rows;
  if (cols) *cols = t->cols;
  if (nbytes) *nbytes = t->nbytes;
  return LLRS_OK;
}

int llrs_tensor_download(const llrs_tensor *t, void *out, size_t nbytes) {
  clear_error();
  if (!t || (!out && nbytes)) return set_error(LLRS_E_INVALID, "tensor/out is NULL");
  if (nbytes != t->nbytes)
    return set_error(LLRS_E_INVALID, "download size %zu != tensor size %zu", nbytes, t->nbytes);
  LLRS_HIP(hipSetDevice(t->b->device));
  if (nbytes) LLRS_HIP(hipMemcpyAsync(out, t->dev, nbytes, hipMemcpyDeviceToHost, t->b->stream));
  LLRS_HIP(hipStreamSynchronize(t->b->stream));
  return LLRS_OK;
}

int llrs_matvec(llrs_backend *b, const llrs_tensor *w, const float *x, size_t nx, float *y,
                size_t ny) {
  clear_error();
  if (!b || !w) return set_error(LLRS_E_INVALID, "backend/tensor is NULL");
  LLRS_TRY(validate_matvec(w, nx, ny));
  if ((nx && !x) || (ny && !y)) return set_error(LLRS_E_INVALID, "x/y is NULL");
  if (ny == 0) return LLRS_OK;
  LLRS_HIP(hipSetDevice(b->device));
  LLRS_TRY(ensure_scratch(b, nx ? nx : 1, ny));
  if (nx) LLRS_HIP(hipMemcpyAsync(b->x_dev, x, nx * 4, hipMemcpyHostToDevice, b->stream));
  LLRS_TRY(launch_matvec(b, w, b->x_dev, b->y_dev));
  LLRS_HIP(hipMemcpyAsync(y, b->y_dev, ny * 4, hipMemcpyDeviceToHost, b->stream));
  LLRS_HIP(hipStreamSynchronize(b->stream));
  return LLRS_OK;
}

int llrs_matvec_dev(llrs_backend *b, const llrs_tensor *w, const float *x_dev, float *y_dev) {
  clear_error();
  if (!b || !w) return set_error(LLRS_E_INVALID, "backend/tensor is NULL");
  if (w->rows == 0) return LLRS_OK;
  if (!x_dev || !y_dev) return set_error(LLRS_E_INVALID, "x_dev/y_dev is NULL");
  LLRS_HIP(hipSetDevice(b->device));
  return launch_matvec(b, w, x_dev, y_dev);
}

int llrs_dequant_row(llrs_backend *b, const llrs_tensor *w, size_t row, float *out, size_t n) {
  clear_error();
  if (!b || !w) return set_error(LLRS_E_INVALID, "backend/tensor is NULL");
  if (row >= w->rows) return set_error(LLRS_E_INVALID, "row %zu out of bounds", row);
  if (n != w->cols) return set_error(LLRS_E_INVALID, "embedding output has wrong length");
  if (!out) return set_error(LLRS_E_INVALID, "out is NULL");
  LLRS_HIP(hipSetDevice(b->device));
  LLRS_TRY(ensure_scratch(b, 1, n));
  LLRS_TRY(launch_dequant_row(w, row, b->y_dev, b->stream));
  LLRS_HIP(hipMemcpyAsync(out, b->y_dev, n * 4, hipMemcpyDeviceToHost, b->stream));
  LLRS_HIP(hipStreamSynchronize(b->stream));
  return LLRS_OK;
}

int llrs_device_alloc(llrs_backend *b, size_t nbytes, void **out_dev) {
  clear_error();
  if (!b || !out_dev) return set_error(LLRS_E_INVALID, "backend/out is NULL");
  LLRS_HIP(hipSetDevice(b->device));
  LLRS_HIP(hipMalloc(out_dev, nbytes ? nbytes : 1));
  return LLRS_OK;
}

int llrs_device_free(llrs_backend *b, void *dev) {
  clear_error();
  if (!b) return set_error(LLRS_E_INVALID, "backend is NULL");
  LLRS_HIP(hipSetDevice(b->device));
  LLRS_HIP(hipStreamSynchronize(b->stream));
  LLRS_HIP(hipFree(dev));
  return LLRS_OK;
}

int llrs_copy_h2d(llrs_backend *b, void *dst_dev, const void *src, size_t nbytes) {
  clear_error();
  if (!b) return set_error(LLRS_E_INVALID, "backend is NULL");
  LLRS_HIP(hipSetDevice(b->device));
  LLRS_HIP(hipMemcpyAsync(dst_dev, src, nbytes, hipMemcpyHostToDevice, b->stream));
  LLRS_HIP(hipStreamSynchronize(b->stream));
  return LLRS_OK;
}

int llrs_copy_d2h(llrs_backend *b, void *dst, const void *src_dev, size_t nbytes) {
  clear_error();
  if (!b) return set_error(LLRS_E_INVALID, "backend is NULL");
  LLRS_HIP(hipSetDevice(b->device));
  LLRS_HIP(hipMemcpyAsync(dst, src_dev, nbytes, hipMemcpyDeviceToHost, b->stream));
  LLRS_HIP(hipStreamSynchronize(b->stream));
  return LLRS_OK;
}

int llrs_device_copy(llrs_backend *b, void *dst_dev, const void *src_dev, size_t nbytes) {
  clear_error();
  if (!b) return set_error(LLRS_E_INVALID, "backend is NULL");
  if (nbytes == 0) return LLRS_OK;
  if (!dst_dev || !src_dev) return set_error(LLRS_E_INVALID, "NULL device pointer");
  if ((reinterpret_cast<uintptr_t>(dst_dev) | reinterpret_cast<uintptr_t>(src_dev) | nbytes) & 15)
    return set_error(LLRS_E_INVALID, "device copy needs 16-byte aligned pointers and length");
  LLRS_HIP(hipSetDevice(b->device));
  LLRS_TRY(launch_copy(dst_dev, src_dev, nbytes, b->cu_count, b->stream));
  LLRS_HIP(hipStreamSynchronize(b->stream));
  return LLRS_OK;
}

}  // extern "C"
