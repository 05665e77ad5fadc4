// The persistent decode kernel: one launch runs every layer of a token's
// step (Qwen2Model::forward_impl, src/model.rs:173-261) with one workgroup
// per CU, all co-resident.  Per layer the phases are those of the
// kernel-per-phase path, with the same arithmetic: RMSNorm + Q/K/V (+bias),
// RoPE + KV append + attention, o_proj (+residual), RMSNorm + gate/up +
// SiLU*up, ffn_down (+residual).  A device-wide barrier separates the phases.
//
// Why: a separate launch per phase pays the ramp-up of its first weight
// loads and the drain of its last workgroups every time.  Here a workgroup
// issues the first weight loads of its next phase (they depend on nothing the
// current phase writes) before it waits at the barrier, so the wait overlaps
// HBM latency.
//
// Barrier: kBarCounters device-scope counters, 128 bytes apart; workgroup w
// increments counter w % kBarCounters (an atomic without return, so arriving
// costs no round trip) and the first wave of every workgroup polls all of
// them until their sum reaches the barrier's target.  Spread over several
// counters, the arrivals do not queue behind each other at one address (a
// single counter costs ~4 us per barrier at 256 workgroups, these ~1.7 us).
// The counters live in uncached memory (no L2 keeps a copy) and are polled
// with scalar loads: a wave's vector loads complete in issue order, so a
// vector poll would first wait for the weight loads the wave issued before
// the barrier (+2% end to end on the 7B shape).  The writer waits for its
// stores (device-scope stores) before arriving.  Every wait is bounded in
// time: on expiry the kernel sets *err (reported to the host as an error)
// and runs on rather than hang.
#include <hip/hip_runtime.h>

#include "attention_dev.h"
#include "common.h"
#include "decode_persistent.h"
#include "gemv_dev.h"

namespace llrs {

#ifdef LLRS_STAMPS
// Timing build only (build.py --stamps): per barrier interval k (5 per layer)
// and workgroup, wall-clock stamps (the 100 MHz clock) [0] released from
// barrier k, [1] activation staged, [2] weight streaming done, [3] stores
// done and arriving at barrier k + 1.  Interval 0 starts at kernel entry.
constexpr int kStampIntervals = 5 * 64, kStampWgs = 512;
__device__ unsigned long long g_stamps[kStampIntervals * kStampWgs * 4];
#define STAMP(k, i)                                                                        \
  do {                                                                                     \
    if (threadIdx.x == 0 && (k) < kStampIntervals && wg < kStampWgs)                      \
      g_stamps[((size_t)(k) * kStampWgs + wg) * 4 + (i)] = wall_clock64();                 \
  } while (0)
#define STAMP_PHASE(ph, k) ph.stamp = ((k) < kStampIntervals && wg < kStampWgs) ? g_stamps + ((size_t)(k) * kStampWgs + wg) * 4 : nullptr
#else
#define STAMP(k, i) do {} while (0)
#define STAMP_PHASE(ph, k) do {} while (0)
#endif

namespace {

__device__ __forceinline__ unsigned ld_u32_dev(unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The workgroup's stores are complete, then its arrival at the next barrier
// (interval k ends).
__device__ void bar_arrive(unsigned *bar, int wg, unsigned k) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  STAMP(k, 3);
  if (threadIdx.x == 0)
    __hip_atomic_fetch_add(bar + (wg % kBarCounters) * kBarStride, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// The sum of the kBarCounters counters, read by scalar loads (uncached
// memory): all sixteen in flight at once, then one wait.
static_assert(kBarCounters == 16 && kBarStride == 32, "the scalar poll reads 16 counters 128 bytes apart");
__device__ __forceinline__ unsigned bar_sum_scalar(const unsigned *bar) {
  unsigned v[16];
  asm volatile(
      "s_load_dword %0, %16, 0x0 glc\n\ts_load_dword %1, %16, 0x80 glc\n\t"
      "s_load_dword %2, %16, 0x100 glc\n\ts_load_dword %3, %16, 0x180 glc\n\t"
      "s_load_dword %4, %16, 0x200 glc\n\ts_load_dword %5, %16, 0x280 glc\n\t"
      "s_load_dword %6, %16, 0x300 glc\n\ts_load_dword %7, %16, 0x380 glc\n\t"
      "s_load_dword %8, %16, 0x400 glc\n\ts_load_dword %9, %16, 0x480 glc\n\t"
      "s_load_dword %10, %16, 0x500 glc\n\ts_load_dword %11, %16, 0x580 glc\n\t"
      "s_load_dword %12, %16, 0x600 glc\n\ts_load_dword %13, %16, 0x680 glc\n\t"
      "s_load_dword %14, %16, 0x700 glc\n\ts_load_dword %15, %16, 0x780 glc\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(v[0]), "=&s"(v[1]), "=&s"(v[2]), "=&s"(v[3]), "=&s"(v[4]), "=&s"(v[5]), "=&s"(v[6]),
        "=&s"(v[7]), "=&s"(v[8]), "=&s"(v[9]), "=&s"(v[10]), "=&s"(v[11]), "=&s"(v[12]), "=&s"(v[13]),
        "=&s"(v[14]), "=&s"(v[15])
      : "s"(uniform_ptr(bar))
      : "memory");
  unsigned t = 0;
#pragma unroll
  for (int i = 0; i < 16; i++) t += v[i];
  return t;
}

// Until every workgroup has arrived at barrier k (k >= 1), or ~20 ms passed.
// scalar: the counters are in uncached memory (scalar polls); otherwise each
// lane polls one with a device-scope vector load.
__device__ void bar_wait(unsigned *bar, unsigned *err, int nwg, unsigned k, bool scalar) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const unsigned target = k * (unsigned)nwg;
    // The clock read is a scalar memory access of its own, so the 20 ms
    // limit is checked every 16th poll, from the first check on.
    unsigned long long t0 = 0;
    for (unsigned it = 1;; it++) {
      unsigned v;
      if (scalar) {
        v = bar_sum_scalar(bar);
      } else {
        v = lane < kBarCounters ? ld_u32_dev(bar + lane * kBarStride) : 0u;
#pragma unroll
        for (int o = 1; o < kBarCounters; o <<= 1) v += __shfl_xor(v, o, 64);
      }
      if (__builtin_amdgcn_readfirstlane(v) >= target) break;
      if ((it & 15) == 0) {
        const unsigned long long t = wall_clock64();  // the 100 MHz wall clock
        if (!t0) {
          t0 = t;
        } else if (t - t0 > 2000000ull) {  // 20 ms
          if (lane == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
}

typedef const __attribute__((address_space(4))) PersistentLayer ConstLayer;

template <uint32_t T> struct TypeC { static constexpr uint32_t value = T; };

// LONG: the instantiation whose attention also has the multi-chunk items of
// long contexts (attention_span > 1); the other one keeps the single-chunk
// path's register allocation, and stays correct at any position, with more
// partials to merge.
template <uint32_t TQ, uint32_t TV, uint32_t TO, uint32_t TGU, uint32_t TD, int HD, bool LONG>
__global__ __launch_bounds__(kPersistentThreads) void decode_persistent_kernel(PersistentArgs p) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float red[16];
  __shared__ __align__(16) float aqs[kPersistentThreads / 64][HD], akn[kPersistentThreads / 64][HD];
  const int wg = blockIdx.x, nwg = gridDim.x;
  const int wave = threadIdx.x >> 6;
  static_assert(kPersistentThreads == 64 * kTaskItems, "an attention task is one item per wave");
  const int pos = bounded_pos(p.attn.pos, p.attn.max_seq);
  // Attention tasks (T items of one head, attention_task_items): the G query
  // heads that share a (KV head, task index) run on workgroups of one XCD
  // (workgroup w sits on XCD w % 8), so the items' keys and values come from
  // HBM once and from that XCD's L2 for the other heads.  Task t: XCD x =
  // t % 8, r = t / 8, head j = r % G of pair q * 8 + x with q = r / G; pair =
  // task index * nkv + kv head.  Workgroup w runs tasks w + j nwg in rounds
  // of kTaskItems / T, in increasing pair order (nwg >= 8 G, checked by the
  // host), and a head's last task waits only for tasks of lower pairs (or of
  // its own round, folded by other waves), so every wait ends.
  const int G = p.attn.nh / p.attn.nkv;
  const int span = LONG ? attention_span(pos, p.attn.nh) : 1;
  const int n_items_h = pos / (span * kChunk) + 1;
  const int task_items = attention_task_items(n_items_h, p.attn.fold_max);
  const int n_task_h = (n_items_h + task_items - 1) / task_items;
  const int per_round = kTaskItems / task_items;
  const int n_pairs = p.attn.nkv * n_task_h;
  const int n_tasks = (n_pairs + 7) / 8 * 8 * G;
  const unsigned epoch = *p.attn.epoch;  // advanced by this step's embedding launch
  unsigned k = 0;
  for (int l = 0; l < p.nlayers; l++) {
    // Through the constant address space: the arguments are never written
    // during the launch, so they load through the scalar cache.
    const PersistentLayer &L = *(const PersistentLayer *)(ConstLayer *)((uintptr_t)(p.layers + l));
    // The phase objects are value-initialised: a member that one path leaves
    // unset would otherwise be carried in registers from the previous layer.
    {  // RMSNorm + Q/K/V (+ bias)
      auto qkv = [&](auto tv) {
        GemvPhase<TQ, decltype(tv)::value, false, true> ph{};
        ph.prefetch(L.qkv, wg, nwg, smem);
        if (k) bar_wait(p.bar, p.err, nwg, k, p.scalar_poll);
        STAMP(k, 0);
        STAMP_PHASE(ph, k);
        ph.finish(L.qkv, smem, red);
        bar_arrive(p.bar, wg, k);
      };
      if constexpr (TV == kTypePerLayer) {  // V's type, read per layer (a uniform branch)
        switch (L.qkv.seg[L.qkv.nseg - 1].type) {
          case LLRS_Q6_K: qkv(TypeC<LLRS_Q6_K>{}); break;
          case LLRS_Q4_K: qkv(TypeC<LLRS_Q4_K>{}); break;
          default: qkv(TypeC<LLRS_Q8_0>{}); break;
        }
      } else {
        qkv(TypeC<TV>{});
      }
      k++;
    }
    {  // RoPE, KV append, attention: one item per wave, kTaskItems per task
      AttnArgs a = p.attn;
      a.q += l * p.act_stride;
      a.k += l * p.act_stride;
      a.v += l * p.act_stride;
      a.out += l * p.act_stride;
      a.k_cache += l * p.cache_stride;
      a.v_cache += l * p.cache_stride;
      a.tag = epoch * (unsigned)p.nlayers + (unsigned)l;
      // Every wave passes the barrier once: inside its first item, after that
      // item's cache loads are issued (rows written by earlier steps; from
      // kSplitLoadsFrom positions only the key rows), or in its first task
      // when it has no item there, or after the loop when the workgroup has
      // no task.
      bool waited = false;
      auto wait = [&] {
        if (!waited) {
          bar_wait(p.bar, p.err, nwg, k, p.scalar_poll);
          STAMP(k, 0);
          waited = true;
        }
      };
      const bool multi = span > 1;
      // The items' partials meet in LDS, two buffers alternating by task: a
      // buffer is written again only after the next task's workgroup barrier,
      // which wave 0 reaches after folding it.
      float *part = reinterpret_cast<float *>(smem);
      int nt = 0;
      for (int t0 = wg; t0 < n_tasks; t0 += per_round * nwg) {
        auto slot = [&](int s, int, int, int &h, int &task) {
          const int t = t0 + s * nwg;
          if (t >= n_tasks) return false;
          const int r = t >> 3, pair = (r / G) * 8 + (t & 7);
          if (pair >= n_pairs) return false;
          h = (pair % a.nkv) * G + r % G;
          task = pair / a.nkv;
          return true;
        };
        float *pb = part + (nt++ & 1) * kTaskItems * AttnGeom<HD>::kPart;
        if constexpr (LONG) {
          if (multi)
            attention_round<HD, true, true, true>(a, pos, slot, aqs[wave], akn[wave], pb, wait);
          else
            attention_round<HD, true, false, true>(a, pos, slot, aqs[wave], akn[wave], pb, wait);
        } else {
          attention_round<HD, true, false, true>(a, pos, slot, aqs[wave], akn[wave], pb, wait);
        }
      }
      wait();
      bar_arrive(p.bar, wg, k);
      k++;
    }
    {  // o_proj (+ residual)
      GemvPhase<TO, TO, false, true> ph{};
      ph.prefetch(L.o, wg, nwg, smem);
      bar_wait(p.bar, p.err, nwg, k, p.scalar_poll);
      STAMP(k, 0);
      STAMP_PHASE(ph, k);
      ph.finish(L.o, smem, red);
      bar_arrive(p.bar, wg, k);
      k++;
    }
    {  // RMSNorm + gate/up + SiLU*up
      GemvPhase<TGU, TGU, true, true> ph{};
      ph.prefetch(L.gate_up, wg, nwg, smem);
      bar_wait(p.bar, p.err, nwg, k, p.scalar_poll);
      STAMP(k, 0);
      STAMP_PHASE(ph, k);
      ph.finish(L.gate_up, smem, red);
      bar_arrive(p.bar, wg, k);
      k++;
    }
    {  // ffn_down (+ residual)
      auto down = [&](auto td) {
        GemvPhase<decltype(td)::value, decltype(td)::value, false, true> ph{};
        ph.prefetch(L.down, wg, nwg, smem);
        bar_wait(p.bar, p.err, nwg, k, p.scalar_poll);
        STAMP(k, 0);
        STAMP_PHASE(ph, k);
        ph.finish(L.down, smem, red);
        bar_arrive(p.bar, wg, k);
      };
      if constexpr (TD == kTypePerLayer) {
        if (L.down.seg[0].type == LLRS_Q4_K)
          down(TypeC<LLRS_Q4_K>{});
        else
          down(TypeC<LLRS_Q6_K>{});
      } else {
        down(TypeC<TD>{});
      }
      k++;
    }
  }
}

template <uint32_t TQ, uint32_t TV, uint32_t TO, uint32_t TGU, uint32_t TD>
int launch_types(const PersistentArgs &p, int head_dim, int grid, size_t lds, hipStream_t s, bool lng) {
  const dim3 g((unsigned)grid), b(kPersistentThreads);
#define PK(HD, L) hipLaunchKernelGGL((decode_persistent_kernel<TQ, TV, TO, TGU, TD, HD, L>), g, b, lds, s, p)
  switch (head_dim) {
    case 64: if (lng) PK(64, true); else PK(64, false); break;
    case 128: if (lng) PK(128, true); else PK(128, false); break;
    default: return set_error(LLRS_E_UNSUPPORTED, "persistent decode: head_dim %d", head_dim);
  }
#undef PK
  LLRS_HIP(hipGetLastError());
  return LLRS_OK;
}

template <uint32_t TQ, uint32_t TV, uint32_t TO, uint32_t TGU, uint32_t TD>
int occupancy_types(int head_dim, size_t lds, bool lng, int *blocks) {
#define OCC(HD, L)                                                                                      \
  LLRS_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(                                              \
      blocks, reinterpret_cast<const void *>(decode_persistent_kernel<TQ, TV, TO, TGU, TD, HD, L>), \
      kPersistentThreads, lds))
  switch (head_dim) {
    case 64: if (lng) OCC(64, true); else OCC(64, false); break;
    case 128: if (lng) OCC(128, true); else OCC(128, false); break;
    default: return set_error(LLRS_E_UNSUPPORTED, "persistent decode: head_dim %d", head_dim);
  }
#undef OCC
  return LLRS_OK;
}

}  // namespace

// The instantiated type sets: the q4km recipe at hidden sizes that are
// multiples of 256 (Q4_K, Q8_0 V, Q6_K down) and not (Q5_0 fallback), and
// the uniform q4k recipe.
bool decode_persistent_supports(uint32_t t_qkv, uint32_t t_v, uint32_t t_o, uint32_t t_gu,
                                uint32_t t_down, int head_dim) {
  if (head_dim != 64 && head_dim != 128) return false;
  const bool q4km = t_qkv == LLRS_Q4_K && t_v == LLRS_Q8_0 && t_o == LLRS_Q4_K && t_gu == LLRS_Q4_K &&
                    t_down == LLRS_Q6_K;
  const bool q4km_q5 = t_qkv == LLRS_Q5_0 && t_v == LLRS_Q8_0 && t_o == LLRS_Q5_0 &&
                       t_gu == LLRS_Q5_0 && t_down == LLRS_Q6_K;
  const bool q4k = t_qkv == LLRS_Q4_K && t_v == LLRS_Q4_K && t_o == LLRS_Q4_K && t_gu == LLRS_Q4_K &&
                   t_down == LLRS_Q4_K;
  // Q4_K q/k/o/gate/up with V and ffn_down types chosen per layer (V: Q8_0,
  // Q4_K or Q6_K; down: Q4_K or Q6_K), e.g. llama.cpp's Q4_K_M files.
  const bool mixed = t_qkv == LLRS_Q4_K && t_o == LLRS_Q4_K && t_gu == LLRS_Q4_K &&
                     t_v == kTypePerLayer && t_down == kTypePerLayer;
  return q4km || q4km_q5 || q4k || mixed;
}

int decode_persistent_blocks_per_cu(uint32_t t_qkv, uint32_t t_v, uint32_t t_o, uint32_t t_gu,
                                    uint32_t t_down, int head_dim, size_t lds, bool long_items,
                                    int *blocks) {
  *blocks = 0;
  if (t_qkv == LLRS_Q4_K && t_v == LLRS_Q8_0 && t_down == LLRS_Q6_K)
    return occupancy_types<LLRS_Q4_K, LLRS_Q8_0, LLRS_Q4_K, LLRS_Q4_K, LLRS_Q6_K>(head_dim, lds, long_items, blocks);
  if (t_qkv == LLRS_Q5_0)
    return occupancy_types<LLRS_Q5_0, LLRS_Q8_0, LLRS_Q5_0, LLRS_Q5_0, LLRS_Q6_K>(head_dim, lds, long_items, blocks);
  if (t_qkv == LLRS_Q4_K && t_v == LLRS_Q4_K)
    return occupancy_types<LLRS_Q4_K, LLRS_Q4_K, LLRS_Q4_K, LLRS_Q4_K, LLRS_Q4_K>(head_dim, lds, long_items, blocks);
  if (t_qkv == LLRS_Q4_K && t_v == kTypePerLayer)
    return occupancy_types<LLRS_Q4_K, kTypePerLayer, LLRS_Q4_K, LLRS_Q4_K, kTypePerLayer>(head_dim, lds, long_items,
                                                                                     blocks);
  return set_error(LLRS_E_UNSUPPORTED, "persistent decode: no instantiation for these weight types");
}

int launch_decode_persistent(const PersistentArgs &p, uint32_t t_qkv, uint32_t t_v, uint32_t t_o,
                             uint32_t t_gu, uint32_t t_down, int head_dim, int grid, size_t lds,
                             hipStream_t s, bool long_items) {
  if (grid < 1) return set_error(LLRS_E_INVALID, "persistent decode: grid %d", grid);
  if (lds + persistent_static_lds(head_dim) > kCuLds)
    return set_error(LLRS_E_UNSUPPORTED, "persistent decode needs %zu bytes of LDS", lds);
  if (t_qkv == LLRS_Q4_K && t_v == LLRS_Q8_0 && t_down == LLRS_Q6_K)
    return launch_types<LLRS_Q4_K, LLRS_Q8_0, LLRS_Q4_K, LLRS_Q4_K, LLRS_Q6_K>(p, head_dim, grid, lds, s, long_items);
  if (t_qkv == LLRS_Q5_0)
    return launch_types<LLRS_Q5_0, LLRS_Q8_0, LLRS_Q5_0, LLRS_Q5_0, LLRS_Q6_K>(p, head_dim, grid, lds, s, long_items);
  if (t_qkv == LLRS_Q4_K && t_v == LLRS_Q4_K)
    return launch_types<LLRS_Q4_K, LLRS_Q4_K, LLRS_Q4_K, LLRS_Q4_K, LLRS_Q4_K>(p, head_dim, grid, lds, s, long_items);
  if (t_qkv == LLRS_Q4_K && t_v == kTypePerLayer)
    return launch_types<LLRS_Q4_K, kTypePerLayer, LLRS_Q4_K, LLRS_Q4_K, kTypePerLayer>(p, head_dim, grid, lds, s,
                                                                                   long_items);
  return set_error(LLRS_E_UNSUPPORTED, "persistent decode: no instantiation for these weight types");
}

}  // namespace llrs

#ifdef LLRS_STAMPS
// Timing build only: copies the stamps of the last persistent launch
// ([interval][512 workgroup slots][4], 64-bit ticks of the 100 MHz clock).
extern "C" int llrs_debug_stamps(void *dst, size_t bytes) {
  if (bytes > sizeof(llrs::g_stamps)) bytes = sizeof(llrs::g_stamps);
  return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(llrs::g_stamps), bytes, 0, hipMemcpyDeviceToHost);
}
#endif
