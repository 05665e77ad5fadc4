// On-device sampling (InferenceEngine::sample_current_logits,
// src/engine.rs:253-325): repetition penalty and temperature per token, a
// descending sort of the candidates in f32::total_cmp order, top-k
// truncation, softmax, the top-p cutoff and the draw, with the uniform
// number supplied by the caller.
//
// The sort is hipCUB's radix sort of (order key, token) pairs; it is stable,
// so equal values keep ascending token order (the reference's
// sort_unstable_by leaves their order unspecified).  The softmax, the top-p
// cumulative sum and the draw run in one workgroup: each thread owns a
// contiguous slice of the sorted candidates, the slices' sums are scanned
// across the workgroup, and the thread whose slice holds a crossing walks it
// in order.  The sums are the reference's f32 sums in another association,
// so a draw can differ from the reference's only when it falls within
// rounding of a boundary between two candidates.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <mutex>

#include "common.h"
#include "sampling.h"

namespace llrs {

namespace {

// Monotone map of f32::total_cmp order onto uint32 (and back).
__device__ __forceinline__ uint32_t order_key(float f) {
  const int32_t b = __float_as_int(f);
  return (uint32_t)(b ^ (int32_t)((uint32_t)(b >> 31) >> 1)) ^ 0x80000000u;
}
__device__ __forceinline__ float key_value(uint32_t k) {
  const int32_t b = (int32_t)(k ^ 0x80000000u);
  return __int_as_float(b ^ (int32_t)((uint32_t)(b >> 31) >> 1));
}

// src/engine.rs:262-278: the penalty for tokens of the repeat window
// (positive values divided, the others multiplied), then the temperature;
// a non-finite result becomes -inf.
__global__ void sample_prepare_kernel(const float *__restrict__ logits, int n,
                                      const uint32_t *__restrict__ recent, int n_recent,
                                      float penalty, float temperature, uint32_t *__restrict__ keys,
                                      uint32_t *__restrict__ idx) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  float v = logits[t];
  if (penalty != 1.0f) {
    bool seen = false;
    for (int i = 0; i < n_recent; i++) seen |= recent[i] == (uint32_t)t;
    if (seen) v = v > 0.0f ? v / penalty : v * penalty;
  }
  if (temperature > 0.0f) v /= temperature;
  if (!isfinite(v)) v = -INFINITY;
  keys[t] = order_key(v);
  idx[t] = (uint32_t)t;
}

constexpr int kSelectThreads = 1024;

// Inclusive scan of one float per thread (Hillis-Steele in LDS).
__device__ float block_scan(float v, float *sh) {
  const int tid = threadIdx.x;
  sh[tid] = v;
  __syncthreads();
  for (int o = 1; o < kSelectThreads; o <<= 1) {
    const float a = tid >= o ? sh[tid - o] : 0.f;
    __syncthreads();
    sh[tid] += a;
    __syncthreads();
  }
  return sh[tid];
}

// src/engine.rs:286-324 over the sorted candidates.
__global__ __launch_bounds__(kSelectThreads) void sample_select_kernel(
    const uint32_t *__restrict__ keys, const uint32_t *__restrict__ idx, int n, int top_k, float top_p,
    float temperature, float u, uint32_t *__restrict__ out) {
  __shared__ float sh[kSelectThreads];
  __shared__ int cut, pick;
  __shared__ float kept_exp;
  const int tid = threadIdx.x;
  if (temperature <= 0.0f) {  // the first candidate
    if (tid == 0) *out = idx[0];
    return;
  }
  const int m = (top_k > 0 && top_k < n) ? top_k : n;
  const float top = key_value(keys[0]);
  const int per = (m + kSelectThreads - 1) / kSelectThreads;
  const int b = min(m, tid * per), e = min(m, b + per);
  float s = 0.f;
  for (int i = b; i < e; i++) s += expf(key_value(keys[i]) - top);
  const float incl = block_scan(s, sh);
  const float sum = sh[kSelectThreads - 1], before = incl - s;
  if (!isfinite(sum) || sum <= 0.0f) {  // src/engine.rs:299-301
    if (tid == 0) *out = idx[0];
    return;
  }
  if (tid == 0) {
    cut = m;
    pick = m;
  }
  __syncthreads();
  // The top-p cutoff: the first candidate whose cumulative probability
  // reaches top_p (all of them if none does).
  {
    float c = before;
    for (int i = b; i < e; i++) {
      c += expf(key_value(keys[i]) - top);
      if (c / sum >= top_p) {
        atomicMin(&cut, i + 1);
        break;
      }
    }
  }
  __syncthreads();
  const int kept = cut;
  // Probability mass of the kept candidates, from the slice that ends them.
  if (kept == m) {
    if (tid == 0) kept_exp = sum;
  } else if (b < kept && kept <= e) {
    float c = before;
    for (int i = b; i < kept; i++) c += expf(key_value(keys[i]) - top);
    kept_exp = c;
  }
  __syncthreads();
  // The draw: the first kept candidate whose cumulative mass reaches
  // u * (kept mass), i.e. where random - sum(p) first drops to <= 0.
  const float r = u * kept_exp;
  {
    float c = before;
    for (int i = b; i < min(e, kept); i++) {
      c += expf(key_value(keys[i]) - top);
      if (c >= r) {
        atomicMin(&pick, i);
        break;
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    const int i = pick < kept ? pick : kept - 1;  // no crossing: the last kept candidate
    *out = idx[i];
  }
}

}  // namespace

namespace {

// The allocation-free sampler's scratch: keys, sorted keys, indices, sorted
// indices (kNoAllocMaxVocab words each), the repeat window, the result word,
// then the radix sort's temporary storage.  In host code `scratch` names a
// host-side stand-in, never the device memory: kernels and copies get the
// address hipGetSymbolAddress returns for the current device.
constexpr size_t kNoAllocWords = 4 * (size_t)kNoAllocMaxVocab + kNoAllocMaxRecent + 64;
constexpr size_t kNoAllocBytes = kNoAllocWords * 4 + kNoAllocSortBytes;
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_dev[kMaxDevices] = {};  // per device: its copy of `scratch`

}  // namespace

int sample_noalloc_scratch(SampleScratch &w) {
  int dev = 0;
  LLRS_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return set_error(LLRS_E_UNSUPPORTED, "device %d", dev);
  uint8_t *base = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
      void *p = nullptr;
      LLRS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
      const size_t need = sample_sort_bytes(kNoAllocMaxVocab);
      if (need > kNoAllocSortBytes)
        return set_error(LLRS_E_UNSUPPORTED, "the radix sort needs %zu temporary bytes, %zu reserved", need,
                         kNoAllocSortBytes);
      g_scratch_dev[dev] = static_cast<uint8_t *>(p);
    }
    base = g_scratch_dev[dev];
  }
  uint32_t *words = reinterpret_cast<uint32_t *>(base);
  w.n = kNoAllocMaxVocab;
  w.max_recent = kNoAllocMaxRecent;
  w.keys = words;
  w.keys_sorted = words + kNoAllocMaxVocab;
  w.idx = words + 2 * (size_t)kNoAllocMaxVocab;
  w.idx_sorted = words + 3 * (size_t)kNoAllocMaxVocab;
  w.recent = words + 4 * (size_t)kNoAllocMaxVocab;
  w.token = w.recent + kNoAllocMaxRecent;
  w.tmp = base + kNoAllocWords * 4;
  w.tmp_bytes = kNoAllocSortBytes;
  return LLRS_OK;
}

size_t sample_sort_bytes(int n) {
  size_t bytes = 0;
  (void)hipcub::DeviceRadixSort::SortPairsDescending(nullptr, bytes, (const uint32_t *)nullptr,
                                                     (uint32_t *)nullptr, (const uint32_t *)nullptr,
                                                     (uint32_t *)nullptr, n, 0, 32);
  return bytes;
}

int launch_sample(const float *logits, int n, const SampleParams &p, int n_recent, float u,
                  SampleScratch &w, hipStream_t s) {
  if (n <= 0 || n > w.n || n_recent < 0 || n_recent > w.max_recent)
    return set_error(LLRS_E_INVALID, "sampling over %d tokens with %d recent ones", n, n_recent);
  hipLaunchKernelGGL(sample_prepare_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, logits,
                     n, w.recent, n_recent, p.penalty, p.temperature, w.keys, w.idx);
  LLRS_HIP(hipGetLastError());
  size_t bytes = w.tmp_bytes;
  LLRS_HIP(hipcub::DeviceRadixSort::SortPairsDescending(w.tmp, bytes, w.keys, w.keys_sorted, w.idx,
                                                        w.idx_sorted, n, 0, 32, s));
  hipLaunchKernelGGL(sample_select_kernel, dim3(1), dim3(kSelectThreads), 0, s, w.keys_sorted,
                     w.idx_sorted, n, p.top_k, p.top_p, p.temperature, u, w.token);
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

}  // namespace llrs
