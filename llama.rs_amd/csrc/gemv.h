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

// ------------------------------------------------------------ tuned GEMV path
enum FastEpi { kEpiStore = 0, kEpiAdd = 1, kEpiSwiGlu = 2, kEpiLogits = 3 };

// One weight matrix of a fused launch.  Row counts are multiples of 4.
struct FastSeg {
  const uint8_t *w;
  uint32_t type;
  int rows;
  long row_bytes;
  const float *bias;  // kEpiStore: added to the output (nullable)
  float *out;
};

// y = W x with x (times `norm` when given, the RMSNorm gain) digitised in LDS.
//   kEpiStore:  seg[i].out[r] = acc * inv_rms + bias[r] for every segment (rows concatenated)
//   kEpiAdd:    seg[0].out[r] += acc
//   kEpiSwiGlu: seg[2].out[r] = silu(gate) * up with gate = seg[0], up = seg[1]
//   kEpiLogits: seg[0].out[r] = acc, and the argmax of the whole output becomes
//               tok_by_pos[*pos + 1] = *next_token, with *pos advanced.
struct FastGemvArgs {
  FastSeg seg[3];
  int nseg;
  int rows;  // output rows covered by the grid
  int cols;
  const float *x;
  const float *norm;
  float eps;
  int epi;
  unsigned long long *amax_key;
  unsigned *done;
  int *pos;
  uint32_t *tok_by_pos;  // max_pos + 1 entries
  uint32_t *next_token;
  int max_pos;           // the context length: positions past it are never written
  int part;              // rows per partition unit: 4 (0 = default) or 16 with dig_out
  uint8_t *dig_out;      // when set: the output is also written digitised here
  const uint8_t *dig_in; // when set: x arrives digitised (x and norm are unused)
};

bool fast_gemv_supports(uint32_t type, size_t cols);
// Whether a launch whose leading segments have type ta and last segment tb
// has a tuned instantiation.
bool fast_gemv_supports_pair(uint32_t ta, uint32_t tb);
// Dynamic LDS of one workgroup: the digitised activation and its rows' results.
size_t fast_gemv_lds_bytes(int cols, int rows, int grid, int part);
// Bytes of a digitised activation of n elements (dig_out / dig_in).
inline size_t fast_gemv_digits_size(size_t n) { return 2 * n + (n / 16) * 8; }
int launch_gemv_fast(const FastGemvArgs &args, int grid, hipStream_t s);
// Workgroups for a launch over `rows` x `cols`, never more than the
// partition units (`part` rows each; 0 = row quads).
int fast_gemv_grid(int cu_count, int rows, int cols, bool dual, int part);

}  // namespace llrs
