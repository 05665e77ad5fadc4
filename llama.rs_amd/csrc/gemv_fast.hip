// Tuned batch-1 dequant-GEMV kernel and its launcher (device code in
// gemv_dev.h).
#include <hip/hip_runtime.h>

#include "common.h"
#include "gemv.h"
#include "gemv_dev.h"

namespace llrs {

namespace {

// LDSX: row sums through ds_bpermute (the LM head, whose waves stream ~37
// row steps each); otherwise through DPP and permlane swaps.
template <uint32_t TA, uint32_t TB, bool DUAL, bool BAL, int NT, bool LDSX = false>
__global__ __launch_bounds__(NT) void gemv_fast_kernel(FastGemvArgs a) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float red[16];
  GemvPhase<TA, TB, DUAL, false, BAL, LDSX> ph;
  ph.prefetch(a, blockIdx.x, gridDim.x, smem);
  ph.finish(a, smem, red);
}

}  // namespace

size_t fast_gemv_lds_bytes(const FastGemvArgs &a, int grid, int threads) {
  int most = 0;
  for (int w = 0; w < grid; w++) {
    int r0, r1;
    fast_gemv_rows(a, w, grid, r0, r1);
    most = r1 - r0 > most ? r1 - r0 : most;
  }
  return fast_gemv_digit_bytes(a.cols) + fast_gemv_ybuf_bytes(most) +
         (a.bal ? bal_slot_bytes(threads >> 6) : 0);
}

bool fast_gemv_supports(uint32_t type, size_t cols) {
  if (cols == 0 || cols % 64 || cols > 24576) return false;
  switch (type) {
    case LLRS_Q4_K: case LLRS_Q5_K: case LLRS_Q6_K: return cols % 256 == 0;
    case LLRS_Q8_0: case LLRS_Q5_0: case LLRS_Q4_0: case LLRS_Q4_1: case LLRS_Q5_1: return true;
    default: return false;
  }
}

// The ds_bpermute variant is built for single-type, single-matrix launches
// in 256-thread workgroups (the LM head's shape) only.
template <uint32_t TA, uint32_t TB, bool DUAL, bool BAL = false>
static void launch_one(const FastGemvArgs &args, int grid, int threads, bool ldsx, size_t lds, hipStream_t s) {
  if (threads == 512) {
    hipLaunchKernelGGL((gemv_fast_kernel<TA, TB, DUAL, BAL, 512>), dim3(grid), dim3(512), lds, s, args);
  } else if constexpr (TA == TB && !DUAL && !BAL) {
    if (ldsx)
      hipLaunchKernelGGL((gemv_fast_kernel<TA, TB, DUAL, BAL, 256, true>), dim3(grid), dim3(256), lds, s, args);
    else
      hipLaunchKernelGGL((gemv_fast_kernel<TA, TB, DUAL, BAL, 256>), dim3(grid), dim3(256), lds, s, args);
  } else {
    hipLaunchKernelGGL((gemv_fast_kernel<TA, TB, DUAL, BAL, 256>), dim3(grid), dim3(256), lds, s, args);
  }
}

int launch_gemv_fast(const FastGemvArgs &args, int grid, hipStream_t s, int threads, bool lds_exchange) {
  if (grid <= 0) return set_error(LLRS_E_INVALID, "GEMV grid must be positive");
  if (threads != 256 && threads != 512) return set_error(LLRS_E_INVALID, "GEMV blocks are 256 or 512 threads");
  if (lds_exchange && (threads != 256 || args.epi == kEpiSwiGlu || args.bal ||
                       args.seg[0].type != args.seg[args.nseg - 1].type))
    return set_error(LLRS_E_UNSUPPORTED, "ds_bpermute row sums are built for 256-thread single-type launches");
  if (args.dig_out && (args.part != 16 || args.rows % 64))
    return set_error(LLRS_E_INVALID, "a digitised output needs 16-row partitions of a multiple of 64 rows");
  if (args.part && args.part != 2 && args.part != 16)
    return set_error(LLRS_E_INVALID, "GEMV partition of %d rows is not supported", args.part);
  size_t lds = fast_gemv_lds_bytes(args, grid, threads);
  if (lds > kMaxLds) return set_error(LLRS_E_UNSUPPORTED, "GEMV needs %zu bytes of LDS (cols %d, rows %d, grid %d)", lds, args.cols, args.rows, grid);
  uint32_t ta = args.seg[0].type, tb = args.seg[args.nseg - 1].type;
  for (int i = 0; i + 1 < args.nseg; i++)
    if (args.seg[i].type != ta) return set_error(LLRS_E_UNSUPPORTED, "mixed leading segment types");
  if (args.epi == kEpiSwiGlu) {
    if (args.nseg != 1 || args.seg[1].type != ta)
      return set_error(LLRS_E_UNSUPPORTED, "gate and up must share a type");
#define DUAL1(A)                                  \
  if (ta == A) {                                  \
    launch_one<A, A, true>(args, grid, threads, lds_exchange, lds, s);   \
    LLRS_HIP(hipGetLastError());                  \
    return LLRS_OK;                               \
  }
    DUAL1(LLRS_Q4_K) DUAL1(LLRS_Q5_0) DUAL1(LLRS_Q8_0) DUAL1(LLRS_Q6_K)
    DUAL1(LLRS_Q4_0) DUAL1(LLRS_Q4_1) DUAL1(LLRS_Q5_1) DUAL1(LLRS_Q5_K)
#undef DUAL1
  }
#define PAIR(A, B)                                 \
  if (ta == A && tb == B) {                        \
    launch_one<A, B, false>(args, grid, threads, lds_exchange, lds, s);   \
    LLRS_HIP(hipGetLastError());                   \
    return LLRS_OK;                                \
  }
  // One type: the balanced split when asked for.
#define SAME(A)                                          \
  if (ta == A && tb == A) {                              \
    if (args.bal)                                        \
      launch_one<A, A, false, true>(args, grid, threads, lds_exchange, lds, s); \
    else                                                 \
      launch_one<A, A, false>(args, grid, threads, lds_exchange, lds, s);       \
    LLRS_HIP(hipGetLastError());                         \
    return LLRS_OK;                                      \
  }
  SAME(LLRS_Q4_K) SAME(LLRS_Q6_K) SAME(LLRS_Q8_0) SAME(LLRS_Q5_0)
  PAIR(LLRS_Q4_K, LLRS_Q8_0) PAIR(LLRS_Q5_0, LLRS_Q8_0)
  PAIR(LLRS_Q4_K, LLRS_Q6_K) PAIR(LLRS_Q4_K, LLRS_Q5_0)
  SAME(LLRS_Q4_0) SAME(LLRS_Q4_1) SAME(LLRS_Q5_1) SAME(LLRS_Q5_K)
#undef SAME
#undef PAIR
  return set_error(LLRS_E_UNSUPPORTED, "no tuned GEMV for %s + %s", type_name(ta), type_name(tb));
}

bool fast_gemv_packed(uint32_t type, int cols) {
  const int per_unit = (type == LLRS_Q4_K || type == LLRS_Q5_K || type == LLRS_Q6_K) ? 64 : 32;
  return cols / per_unit <= 32;
}

int fast_gemv_grid(int cu_count, int rows, int cols, bool dual, int part) {
  // Measured on the decode shapes: one workgroup per CU for rows of <= 8K
  // columns, two for longer rows (more loads in flight per row), three for the
  // dual gate/up kernel.
  const int per_cu = dual ? 3 : (cols > 8192 ? 2 : 1);
  if (part <= 0) part = 2;
  const int g = per_cu * cu_count, units = (rows + part - 1) / part;
  return units < g ? units : g;
}

bool fast_gemv_supports_pair(uint32_t ta, uint32_t tb) {
  auto ok = [](uint32_t a, uint32_t b) {
    return (a == b && (a == LLRS_Q4_K || a == LLRS_Q6_K || a == LLRS_Q8_0 || a == LLRS_Q5_0 ||
                       a == LLRS_Q4_0 || a == LLRS_Q4_1 || a == LLRS_Q5_1 || a == LLRS_Q5_K)) ||
           (a == LLRS_Q4_K && (b == LLRS_Q8_0 || b == LLRS_Q6_K || b == LLRS_Q5_0)) ||
           (a == LLRS_Q5_0 && b == LLRS_Q8_0);
  };
  return ok(ta, tb);
}

}  // namespace llrs
