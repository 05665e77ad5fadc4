// The persistent decode kernel: every layer of one token's step
// (Qwen2Model::forward_impl, src/model.rs:173-261) in one launch of one
// workgroup per CU, the phases separated by device-wide barriers.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"
#include "decode.h"
#include "gemv.h"

namespace llrs {

// One layer's GEMV phases (those of the kernel-per-phase path).  Every
// activation a phase writes has its own buffer per layer (the residual stream
// included), so within one launch no buffer is read before it is written and
// activations can be read with ordinary loads.
struct PersistentLayer {
  FastGemvArgs qkv, o, gate_up, down;
};

struct PersistentArgs {
  const PersistentLayer *layers;  // device array, one per layer
  int nlayers;
  // Layer 0's attention; layer l's q/k/v/out lie act_stride floats further
  // and its KV cache cache_stride floats further (kept as kernel arguments so
  // the attention's pointers stay in scalar registers).
  AttnArgs attn;
  long act_stride, cache_stride;
  unsigned *bar;  // kPersistentBarWords words of barrier counters, zero at launch (the embedding kernel clears them)
  unsigned *err;  // set when a barrier wait gives up; never cleared by the kernel
  int scalar_poll;  // the counters lie in uncached memory: polled by scalar loads
};

// Barrier counters, each on its own 128-byte line.
constexpr int kBarCounters = 16, kBarStride = 32;
constexpr int kPersistentBarWords = kBarCounters * kBarStride;
constexpr int kPersistentThreads = 512;
constexpr size_t kCuLds = 160 * 1024;  // LDS per CU on gfx950
// The dynamic LDS request is at least this, so no CU holds two workgroups.
constexpr size_t kPersistentMinLds = kCuLds / 2 + 1024;

// Static LDS of the kernel: per-wave attention staging (q and the new k row),
// the reduction scratch of the GEMV phases, and slack.
inline size_t persistent_static_lds(int head_dim) {
  return 2 * (size_t)(kPersistentThreads / 64) * head_dim * 4 + 512;
}

// A type argument meaning "chosen per layer" (V of the Q/K/V launch and
// ffn_down in the Q4_K family: the kernel reads each layer's type and branches).
constexpr uint32_t kTypePerLayer = 0xffffffffu;

// Whether the step's weight types and geometry have an instantiation.
bool decode_persistent_supports(uint32_t t_qkv, uint32_t t_v, uint32_t t_o, uint32_t t_gu,
                                uint32_t t_down, int head_dim);
int launch_decode_persistent(const PersistentArgs &p, uint32_t t_qkv, uint32_t t_v, uint32_t t_o,
                             uint32_t t_gu, uint32_t t_down, int head_dim, int grid, size_t lds,
                             hipStream_t s, bool long_items);
// Workgroups of the instantiation that fit one CU with `lds` bytes of dynamic
// LDS (hipOccupancyMaxActiveBlocksPerMultiprocessor).  The kernel's barriers
// need every workgroup resident at once: one per CU at least.
int decode_persistent_blocks_per_cu(uint32_t t_qkv, uint32_t t_v, uint32_t t_o, uint32_t t_gu,
                                    uint32_t t_down, int head_dim, size_t lds, bool long_items,
                                    int *blocks);
// Whether a step at position pos should launch the long_items instantiation.
inline bool persistent_long_items(size_t pos, int nh) { return attention_span((int)pos, nh) > 1; }

}  // namespace llrs
