// LDS access-pattern probe: kernels whose only work is LDS reads or writes
// of a known bank pattern, so that the SQ_LDS_BANK_CONFLICT and
// SQ_LDS_IDX_ACTIVE counters can be read against a known answer.  The
// prefill GEMMs report a bank-conflict share of exactly one third for their
// 128-bit LDS accesses; these kernels show what the counters report for
// conflict-free 32-, 64- and 128-bit accesses and for a pattern whose lanes
// all hit one bank.  No counterpart in the reference (measurement only).
#include <hip/hip_runtime.h>

#include "common.h"

namespace llrs {

namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeFloats = 8192;  // 32 KB of LDS per workgroup

// MODE 0: ds_read_b32, lane l reads dword l of a 64-dword row (all banks once
//         per half-wave: conflict-free).
// MODE 1: ds_read_b64, lane l reads dwords 2l, 2l + 1 (conflict-free).
// MODE 2: ds_read_b128, lane l reads dwords 4l .. 4l + 3 (conflict-free).
// MODE 3: ds_read_b32, lane l reads dword 64 l (every lane in bank 0).
// MODE 4: ds_write_b128, lane l writes dwords 4l .. 4l + 3 (conflict-free).
// MODE 5: ds_read_b128 of an MFMA 16x16x32 operand fragment from a tile with
//         rows 144 bytes apart (the prefill GEMMs' LDS row stride): lane l
//         reads row l % 16 at byte 16 (l / 16).
// MODE 6: as 5 with rows 176 bytes apart.
// MODE 7: ds_write_b128 of the prefill GEMMs' staging pattern: lane l writes
//         16 bytes at row l / 2, byte 64 (l % 2) (+16 per iteration's row),
//         rows 144 bytes apart.
// MODE 8: ds_read_b128, lanes 16g .. 16g + 15 read 256 contiguous bytes at
//         byte 2064 g + 16 (not 256-byte aligned).
// MODE 9: as 8 at byte 2048 g (256-byte aligned).
// MODE 10: ds_write_b128, lane l writes row l / 2 of chunk c = 4 (l % 2) +
//         (iteration % 4), chunks 2048 bytes apart, the row's 16-byte slot
//         XOR-swizzled by 2 (c / 2).
// MODE 11: as 10 without the swizzle.
// Each iteration moves to another row; the sums go to `out` so nothing is
// eliminated.
template <int MODE>
__global__ __launch_bounds__(kProbeThreads) void lds_probe_kernel(float *out, int iters) {
  __shared__ __align__(16) float buf[kProbeFloats];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < kProbeFloats; i += kProbeThreads) buf[i] = (float)(i & 255);
  __syncthreads();
  float acc = 0.f;
  for (int it = 0; it < iters; it++) {
    const int row = (it * 4 + wave) & 15;  // 16 rows of 512 dwords
    if constexpr (MODE == 0) {
      acc += buf[row * 512 + lane];
    } else if constexpr (MODE == 1) {
      const float2 v = *reinterpret_cast<const float2 *>(&buf[row * 512 + 2 * lane]);
      acc += v.x + v.y;
    } else if constexpr (MODE == 2) {
      const float4 v = *reinterpret_cast<const float4 *>(&buf[row * 512 + 4 * lane]);
      acc += v.x + v.y + v.z + v.w;
    } else if constexpr (MODE == 3) {
      acc += buf[(row * 8 + lane * 64) & (kProbeFloats - 1)];
    } else if constexpr (MODE == 5 || MODE == 6) {
      constexpr int RS = MODE == 5 ? 36 : 44;  // row stride in dwords
      const float4 v = *reinterpret_cast<const float4 *>(&buf[(row & 7) * 1024 + (lane & 15) * RS + 4 * (lane >> 4)]);
      acc += v.x + v.y + v.z + v.w;
    } else if constexpr (MODE == 8 || MODE == 9) {
      const int o = (MODE == 8 ? 516 * (lane >> 4) + 4 : 512 * (lane >> 4)) + 4 * (lane & 15);
      const float4 v = *reinterpret_cast<const float4 *>(&buf[o + (row & 3) * 64]);
      acc += v.x + v.y + v.z + v.w;
    } else if constexpr (MODE == 10 || MODE == 11) {
      const int c = 4 * (lane & 1) + (it & 3), r = lane >> 1;
      const int slot = MODE == 10 ? ((r & ~15) | ((r ^ (2 * (c >> 1))) & 15)) : r;
      *reinterpret_cast<float4 *>(&buf[c * 512 + slot * 4]) = make_float4(acc, acc, acc, acc);
      acc += 1.f;
    } else if constexpr (MODE == 7) {
      *reinterpret_cast<float4 *>(&buf[(lane >> 1) * 36 + 16 * (lane & 1) + 4 * (it & 3)]) =
          make_float4(acc, acc, acc, acc);
      acc += 1.f;
    } else {
      *reinterpret_cast<float4 *>(&buf[row * 512 + 4 * lane]) = make_float4(acc, acc, acc, acc);
      acc += 1.f;
    }
    // A compiler barrier: every iteration's access is emitted (the rows
    // repeat every four iterations, and LDS does not change in between).
    asm volatile("" ::: "memory");
  }
  if constexpr (MODE == 4 || MODE == 7 || MODE == 10 || MODE == 11) {  // the written rows are read back, so the stores are live
    __syncthreads();
    acc += buf[(tid * 17) & (kProbeFloats - 1)];
  }
  out[blockIdx.x * kProbeThreads + tid] = acc;
}

template <int MODE>
void launch_probe(float *out, int blocks, int iters, hipStream_t s) {
  hipLaunchKernelGGL(lds_probe_kernel<MODE>, dim3(blocks), dim3(kProbeThreads), 0, s, out, iters);
}

}  // namespace

}  // namespace llrs

using namespace llrs;

extern "C" int llrs_debug_lds_probe(llrs_backend *b, int mode, int blocks, int iters) {
  if (!b) return set_error(LLRS_E_INVALID, "null backend");
  if (mode < 0 || mode > 11 || blocks <= 0 || blocks > 65536 || iters <= 0)
    return set_error(LLRS_E_INVALID, "LDS probe: mode 0..11, 1..65536 blocks, iters > 0");
  float *out = nullptr;
  LLRS_HIP(hipMalloc((void **)&out, (size_t)blocks * kProbeThreads * sizeof(float)));
  switch (mode) {
    case 0: launch_probe<0>(out, blocks, iters, b->stream); break;
    case 1: launch_probe<1>(out, blocks, iters, b->stream); break;
    case 2: launch_probe<2>(out, blocks, iters, b->stream); break;
    case 3: launch_probe<3>(out, blocks, iters, b->stream); break;
    case 4: launch_probe<4>(out, blocks, iters, b->stream); break;
    case 5: launch_probe<5>(out, blocks, iters, b->stream); break;
    case 6: launch_probe<6>(out, blocks, iters, b->stream); break;
    case 7: launch_probe<7>(out, blocks, iters, b->stream); break;
    case 8: launch_probe<8>(out, blocks, iters, b->stream); break;
    case 9: launch_probe<9>(out, blocks, iters, b->stream); break;
    case 10: launch_probe<10>(out, blocks, iters, b->stream); break;
    default: launch_probe<11>(out, blocks, iters, b->stream); break;
  }
  const hipError_t e = hipGetLastError();
  const hipError_t e2 = hipStreamSynchronize(b->stream);
  (void)hipFree(out);
  LLRS_HIP(e);
  LLRS_HIP(e2);
  return LLRS_OK;
}
