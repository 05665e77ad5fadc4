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
//   kEpiAdd:    seg[0].out[r] = res_in[r] + acc (seg[0].out[r] += acc when res_in is null)
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
  int part;              // rows per partition unit: 2 (0 = default) or 16 with dig_out
  uint8_t *dig_out;      // when set: the output is also written digitised here
  const uint8_t *dig_in; // when set: x arrives digitised (x and norm are unused)
  const float *res_in;   // kEpiAdd: the residual added to (null: seg[0].out itself)
  // Balanced split: a workgroup whose rows lie in one segment and form fewer
  // row groups than twice its waves (and not a multiple of them) spreads the
  // (row group, unit iteration) steps evenly over all waves and sums each
  // row's per-wave partials in wave order.  The sums then depend on the grid
  // and the block size in their last bits.
  int bal;
};

// Rows [r0, r1) of workgroup wg of nwg: the launch's weight bytes split evenly
// over the grid, cut at whole partition units (`part` rows, pairs by default),
// so workgroups whose rows lie in a wider-typed segment get fewer of them.
// Segment row counts are multiples of 4 (of `part` when it is 16).
__host__ __device__ inline void fast_gemv_rows(const FastGemvArgs &a, int wg, int nwg, int &r0,
                                               int &r1) {
  const int part = a.part ? a.part : 2;
  const int ns = a.epi == kEpiSwiGlu ? 1 : a.nseg;
  long total = 0;
  for (int s = 0; s < ns; s++) total += (long)a.seg[s].rows * a.seg[s].row_bytes;
  auto row_at = [&](long b) -> int {
    int base = 0;
    for (int s = 0; s < ns; s++) {
      const long sb = (long)a.seg[s].rows * a.seg[s].row_bytes;
      if (b < sb) return base + (int)(b / a.seg[s].row_bytes) / part * part;
      b -= sb;
      base += a.seg[s].rows;
    }
    return a.rows;
  };
  r0 = row_at(total * wg / nwg);
  r1 = row_at(total * (wg + 1) / nwg);
}

bool fast_gemv_supports(uint32_t type, size_t cols);
// Whether a launch whose leading segments have type ta and last segment tb
// has a tuned instantiation.
bool fast_gemv_supports_pair(uint32_t ta, uint32_t tb);
// Dynamic LDS of one workgroup: the digitised activation and its rows' results.
// `threads`: the block size (the balanced split keeps partials per wave).
size_t fast_gemv_lds_bytes(const FastGemvArgs &a, int grid, int threads = 256);
// Bytes of a digitised activation of n elements (dig_out / dig_in).
inline size_t fast_gemv_digits_size(size_t n) { return 2 * n + (n / 16) * 8; }
// `threads`: 256 or 512 per workgroup (the digitised activation is built
// once per workgroup and shared by its waves).  `lds_exchange`: row sums
// through ds_bpermute rather than DPP / permlane swaps, for launches whose
// waves stream many row steps (the LM head); 256 threads, one weight type,
// no SwiGLU, no balanced split.
int launch_gemv_fast(const FastGemvArgs &args, int grid, hipStream_t s, int threads = 256,
                     bool lds_exchange = false);
// Whether rows of `cols` columns of `type` have at most 32 units of work, so
// that each 32-lane half of a wave takes its own row group (packed rows).
bool fast_gemv_packed(uint32_t type, int cols);
// Workgroups for a launch over `rows` x `cols`, never more than the
// partition units (`part` rows each; 0 = row pairs).
int fast_gemv_grid(int cu_count, int rows, int cols, bool dual, int part);

}  // namespace llrs
