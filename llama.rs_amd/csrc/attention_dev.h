// Device side of decode attention: one (query head, chunk of positions)
// item per wave, shared by the attention kernel and the persistent decode
// kernel.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"
#include "decode.h"
#include "quant_dev.h"
#include "wave_dev.h"

namespace llrs {

// *pos clamped into [0, max_seq): even a corrupted position never indexes
// outside the cache.
__device__ __forceinline__ int bounded_pos(const int *pos, int max_seq) {
  int p = *pos;
  return p < 0 ? 0 : p >= max_seq ? max_seq - 1 : p;
}

// ------------------------------------------------------------------ attention
//
// Items of attention_span(pos, nh) consecutive chunks of kChunk positions
// (one chunk while every head's items fit the wave slots), one per wave; the
// kTaskItems consecutive items of a head that one workgroup runs form a task.
// Per chunk: split-half RoPE (src/model.rs:87-95) on the head's query, scores
// q.k * 1/sqrt(hd), softmax partials (max, sum of exp) and exp-weighted V
// sums (src/model.rs:206-231, softmax_inplace 298-313).  The item holding the
// current position also rotates the new key, and the group's first head
// appends key and value to the cache (KVCache::update, src/cache.rs:38-53).
//
// Decode attention moves a few MB per layer, so latency bounds it: each wave
// issues all its K and V loads first.  A task's items meet in LDS behind one
// workgroup barrier; a head's tasks meet without counters (see
// attention_task): one round trip on the merging path, none on the others,
// no cache write-back.  Tasks past the current position are skipped, so one
// grid (sized for the whole context) serves every position of a captured
// graph.


// Whether a merge has waited ~20 ms for partials that never came; then *err
// is set and the merge goes on with what it read.
__device__ __forceinline__ bool merge_wait_over(unsigned long long &t0, unsigned *err) {
  return tagged_wait_over(t0, err);
}

// Per-lane geometry of an item.  Keys: LPR lanes hold a row as float4s, so
// one load covers RPI whole rows (contiguous bytes), NK4 loads a chunk.
// Values: VW floats per lane, VL lanes per row, RV rows per load, NVI loads.
template <int HD> struct AttnGeom {
  static constexpr int KH = HD / 2, LPR = HD / 4, RPI = 64 / LPR, NK4 = kChunk / RPI;
  static constexpr int VW = HD >= 64 ? HD / 64 : 1, VL = HD / VW, RV = 64 / VL, NVI = kChunk / RV;
  static_assert(NK4 >= 1 && NK4 * 2 == LPR && VW <= 2 && RV * VL == 64, "head_dim must be 16..128");
  // The lane holding the score of row p of a sub-chunk (lanes 2k and 2k+1 of
  // a row group hold row k * RPI + group).
  static __device__ __forceinline__ int score_lane(int p) { return (p % RPI) * LPR + (p / RPI) * 2; }
  // A partial in LDS or scratch: [HD] O sums, [HD] V sums, max, sum of exp.
  static constexpr int kPart = 2 * HD + 2;
};

// The softmax partial of one item or of several merged, held by a wave:
// running max m and sum of exp l in every lane, the exp-weighted V sums O and
// the plain V sums Vs (for the uniform fallback) of the lane's VW dimensions
// in lanes < VL.
template <int HD> struct AttnPart {
  float m, l, O[AttnGeom<HD>::VW], Vs[AttnGeom<HD>::VW];
};

// One (query head, item) of an attention task, run by one wave: its softmax
// partial over positions [item * span, min((item + 1) * span, pos + 1)),
// span = attention_span(pos, nh) chunks; the item holding pos also rotates
// the new key, and the group's first head appends key and value to the cache.
// qs and kn are the wave's own LDS (HD floats each).  MULTI: the
// instantiation for attention_span(pos, nh) > 1 (the other one assumes
// single-chunk items and keeps their code straight-line).
// EARLY (the persistent kernel): `wait` is the phase barrier, issued after the
// item's cache loads (rows written by earlier steps); the caller makes sure
// every wave passes it exactly once.  The phase barrier ends in a workgroup
// barrier that waves reach from different call sites (here, or after their
// task loop), which pairs up because s_barrier counts waves: so this
// function contains no workgroup barrier of its own and calls `wait` on
// every path, before any return.
struct NoWait {
  __device__ void operator()() const {}
};

template <int HD, bool MULTI, bool EARLY, class Wait>
__device__ void attention_item(const AttnArgs &a, int h, int chunk, int pos, float *qs, float *kn,
                               Wait &&wait, AttnPart<HD> &P) {
  // No contraction into FMAs: the attention kernel and the persistent kernel
  // compile this code in different contexts, and their results must agree
  // bit for bit.
#pragma clang fp contract(off)
  using Gm = AttnGeom<HD>;
  constexpr int KH = Gm::KH, LPR = Gm::LPR, RPI = Gm::RPI, NK4 = Gm::NK4;
  constexpr int VW = Gm::VW, VL = Gm::VL, RV = Gm::RV, NVI = Gm::NVI;
  using VT = typename std::conditional<VW == 2, float2, float>::type;

  const int G = a.nh / a.nkv, kvw = a.nkv * HD;
  const int kvh = h / G;
  const int S = MULTI ? attention_span(pos, a.nh) : 1, span = S * kChunk;
  const int c0 = chunk * span;  // this item: positions [c0, c0 + span), S sub-chunks
  const bool owns_new = pos < c0 + span;
  const int lane = thread_x() & 63, kcol = lane % LPR, kgrp = lane / LPR;
  // The sub-chunk row whose score this lane ends up holding.
  const int srow = (kcol >> 1) * RPI + kgrp;
  const float *kc = a.k_cache + (size_t)kvh * HD, *vc = a.v_cache + (size_t)kvh * HD;

  // 1. Loads, all issued up front: this lane's query and new-key pair
  //    (i, i + KH) with its RoPE factors and its dimensions of the new value;
  //    then the first sub-chunk's keys (load j: rows j * RPI + kgrp, the
  //    lane's float4 kcol of each) and
  //    values (lane = VW consecutive dims of row lane / VL, RV rows per
  //    load).  Rows past the sub-chunk's end are clamped onto its first row
  //    and masked later.
  const int ri = lane & (KH - 1);
  const float *cs = a.rope + (size_t)pos * HD, *sn = cs + KH;
  const float *qx = a.q + (size_t)h * HD, *kx = a.k + kvh * HD, *vx = a.v + kvh * HD;
  const int vd = (lane % VL) * VW, vr0 = lane / VL;
  float4 kr[NK4];
  VT vv[NVI];
  auto load_k = [&](int s0, int s1) {
#pragma unroll
    for (int j = 0; j < NK4; j++) {
      const int p = s0 + j * RPI + kgrp;
      kr[j] = *reinterpret_cast<const float4 *>(kc + (size_t)(p < s1 ? p : s0) * kvw + 4 * kcol);
    }
  };
  auto load_v = [&](int s0, int s1) {
#pragma unroll
    for (int i = 0; i < NVI; i++) {
      const int p = s0 + i * RV + vr0;
      vv[i] = *reinterpret_cast<const VT *>(vc + (size_t)(p < s1 ? p : s0) * kvw + vd);
    }
  };
  auto load_rows = [&](int s0, int s1) {
    load_k(s0, s1);
    load_v(s0, s1);
  };
  // This step's query, key and value (ordinary loads: no workgroup of the
  // launch reads them before they are written).
  float q_re, q_im, k_re, k_im, rc, rs;
  VT vnew;
  auto load_new = [&] {
    q_re = qx[ri];
    q_im = qx[ri + KH];
    k_re = kx[ri];
    k_im = kx[ri + KH];
    rc = cs[ri];
    rs = sn[ri];
    vnew = *reinterpret_cast<const VT *>(vx + vd);
  };
  if constexpr (EARLY) {
    // The cache rows before this step's position were written by earlier
    // steps, so their loads go out before the caller waits for this step's
    // query, key and value (`wait`: the persistent kernel's barrier; the row
    // at pos is taken from those, not from the cache).  From kSplitLoadsFrom
    // positions only the key rows do and the value rows follow the wait:
    // with both in flight (8 MB per layer at 4,000 positions of the 1.5B
    // shape) the barrier's release waits behind them.
    const int s1 = min(c0 + kChunk, pos + 1);
    if (pos >= kSplitLoadsFrom) {
      load_k(c0, s1);
      wait();
      load_new();
      load_v(c0, s1);
    } else {
      load_rows(c0, s1);
      wait();
      load_new();
    }
  } else {
    wait();
    load_new();
    load_rows(c0, min(c0 + kChunk, pos + 1));
  }

  // 2. Rotated query and new key in LDS; the group's first head appends the
  //    new key and value to the cache.
  if (lane < KH) {
    qs[ri] = q_re * rc - q_im * rs;
    qs[ri + KH] = q_re * rs + q_im * rc;
    const float r0 = k_re * rc - k_im * rs, r1 = k_re * rs + k_im * rc;
    kn[ri] = r0;
    kn[ri + KH] = r1;
    if (owns_new && h % G == 0) {
      float *krow = a.k_cache + (size_t)pos * kvw + kvh * HD;
      krow[ri] = r0;
      krow[ri + KH] = r1;
    }
  }
  if (owns_new && h % G == 0 && lane < VL)
    *reinterpret_cast<VT *>(a.v_cache + (size_t)pos * kvw + kvh * HD + vd) = vnew;
  // The wave's LDS writes complete before its reads below.
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();

  // 3-4. Per sub-chunk: scores (each lane's float4 of every row it loaded,
  //    then a reduce-scatter over the row's LPR lanes that leaves the score
  //    of row srow in the lane), the softmax partials, exp-weighted and plain
  //    V sums of the lane's VW dimensions; sub-chunks after the first fold in
  //    with the running-max rescaling (their rows load after the previous
  //    one's sums).
  float m = -INFINITY, l = 0.f, O[VW], Vs[VW];
#pragma unroll
  for (int k = 0; k < VW; k++) O[k] = Vs[k] = 0.f;
  const float4 qv = *reinterpret_cast<const float4 *>(qs + 4 * kcol);
  for (int sub = 0; sub < S; sub++) {
    const int s0 = c0 + sub * kChunk;
    if (s0 > pos) break;
    const int s1 = min(s0 + kChunk, pos + 1);  // exclusive
    if (sub > 0) load_rows(s0, s1);
    if (s0 <= pos && pos < s1) {  // the row this step appends, from registers / LDS
      const int pn = pos - s0;
      if (kgrp == pn % RPI) {
        const float4 nk = *reinterpret_cast<const float4 *>(kn + 4 * kcol);
#pragma unroll
        for (int j = 0; j < NK4; j++)
          if (j == pn / RPI) kr[j] = nk;
      }
#pragma unroll
      for (int i = 0; i < NVI; i++)
        if (s0 + i * RV + vr0 == pos) vv[i] = vnew;
    }
    float d[NK4];
#pragma unroll
    for (int j = 0; j < NK4; j++) d[j] = qv.x * kr[j].x + qv.y * kr[j].y + qv.z * kr[j].z + qv.w * kr[j].w;
    // Reduce-scatter: at mask mk (NK4, NK4 / 2, .., 2) the lane keeps the
    // half of its n values picked by its bit mk and adds its partner's copy
    // of that half; a last exchange with lane ^ 1 completes the sum.
#pragma unroll
    for (int n = NK4; n > 1; n >>= 1) {
      const bool hi = lane & n;
#pragma unroll
      for (int j = 0; j < n / 2; j++) {
        const float keep = hi ? d[j + n / 2] : d[j], give = hi ? d[j] : d[j + n / 2];
        d[j] = keep + lane_partner(give, n);
      }
    }
    float sc = d[0] + lane_partner(d[0], 1);
    const bool valid = s0 + srow < s1;
    sc = valid ? sc * a.scale : -INFINITY;
    float ms = sc;
    ms = wave_max(ms);
    const float x = valid ? expf(sc - ms) : 0.f;
    float ls = (lane & 1) ? 0.f : x;  // every row is held by two lanes
    ls = wave_total(ls);
    float Os[VW], Vss[VW];
#pragma unroll
    for (int k = 0; k < VW; k++) Os[k] = Vss[k] = 0.f;
#pragma unroll
    for (int i = 0; i < NVI; i++) {
      const int p = i * RV + vr0;  // position within the sub-chunk
      float wp;  // exp weight of position p, held by lane score_lane(p)
      if constexpr (RV == 1)
        wp = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), Gm::score_lane(i)));
      else
        wp = __shfl(x, Gm::score_lane(p), 64);
      const bool in = s0 + p < s1;  // a clamped row adds nothing, whatever it holds
      const float *e = reinterpret_cast<const float *>(&vv[i]);
#pragma unroll
      for (int k = 0; k < VW; k++) {
        Os[k] += in ? wp * e[k] : 0.f;
        Vss[k] += in ? e[k] : 0.f;
      }
    }
#pragma unroll
    for (int o = VL; o < 64; o <<= 1) {
#pragma unroll
      for (int k = 0; k < VW; k++) {
        Os[k] += lane_partner(Os[k], o);
        Vss[k] += lane_partner(Vss[k], o);
      }
    }
    if (sub == 0) {  // one sub-chunk: exactly its own partial
      m = ms;
      l = ls;
#pragma unroll
      for (int k = 0; k < VW; k++) {
        O[k] = Os[k];
        Vs[k] = Vss[k];
      }
    } else {
#pragma unroll
      for (int k = 0; k < VW; k++) Vs[k] += Vss[k];
      if (ms != -INFINITY) {
        const float mn = fmaxf(m, ms);
        const float sa = m == -INFINITY ? 0.f : expf(m - mn), sb = expf(ms - mn);
        l = l * sa + ls * sb;
#pragma unroll
        for (int k = 0; k < VW; k++) O[k] = O[k] * sa + Os[k] * sb;
        m = mn;
      }
    }
  }

  P.m = m;
  P.l = l;
#pragma unroll
  for (int k = 0; k < VW; k++) {
    P.O[k] = O[k];
    P.Vs[k] = Vs[k];
  }
}

// Folds partials first .. first + np - 1 of `slots` (scratch partials written
// by other workgroups of this step) into (M, L, R) and their V sums into V
// when `vsums`.  Per round of 64: their statistics one per lane load together
// with their first OB O partials; a load round is repeated until every tag is
// this step's.  The round's max by wave reduction, each partial's weight
// exp(m_c - M) in its lane, broadcast by readlane to weight the O partials;
// rounds fold with the running-max rescaling, and a partial whose max is -inf
// weighs 0.
template <int HD>
__device__ void fold_scratch(const AttnArgs &a, const unsigned long long *slots, int np, float &M, float &L,
                             float (&R)[AttnGeom<HD>::VW], unsigned long long &t0) {
#pragma clang fp contract(off)
  using Gm = AttnGeom<HD>;
  constexpr int VW = Gm::VW, VL = Gm::VL, OB = 32 / VW;
  const long stride = a.part_stride;
  const unsigned tag = a.tag;
  const int lane = thread_x() & 63, vd = (lane % VL) * VW;
  for (int cb = 0; cb < np; cb += 64) {
    const int nc = min(64, np - cb);
    float ov[OB][VW], mm, ll;
    const unsigned long long *pcl = slots + (size_t)(cb + min(lane, nc - 1)) * stride;
    while (true) {
      bool ok = true;
#pragma unroll
      for (int j = 0; j < OB; j++) {
        const unsigned long long *pc = slots + (size_t)(cb + min(j, nc - 1)) * stride + vd;
#pragma unroll
        for (int k = 0; k < VW; k++) ov[j][k] = load_tagged(pc + k, tag, ok);
      }
      mm = load_tagged(pcl + 2 * HD, tag, ok);
      ll = load_tagged(pcl + 2 * HD + 1, tag, ok);
      if (__all(ok) || merge_wait_over(t0, a.err)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    const bool in = lane < nc && mm != -INFINITY;
    float Mr = in ? mm : -INFINITY;
    Mr = wave_max(Mr);
    const float w = in ? expf(mm - Mr) : 0.f;
    float Lr = w * ll;
    Lr = wave_total(Lr);
    float Rr[VW];
#pragma unroll
    for (int k = 0; k < VW; k++) Rr[k] = 0.f;
    for (int jb = 0; jb < nc; jb += OB) {
      if (jb > 0) {
        while (true) {
          bool ok = true;
#pragma unroll
          for (int j = 0; j < OB; j++) {
            const unsigned long long *pc = slots + (size_t)(cb + min(jb + j, nc - 1)) * stride + vd;
#pragma unroll
            for (int k = 0; k < VW; k++) ov[j][k] = load_tagged(pc + k, tag, ok);
          }
          if (__all(ok) || merge_wait_over(t0, a.err)) break;
          __builtin_amdgcn_s_sleep(1);
        }
      }
#pragma unroll
      for (int j = 0; j < OB; j++) {
        if (jb + j >= nc) break;
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), jb + j));
#pragma unroll
        for (int k = 0; k < VW; k++) Rr[k] += wj * ov[j][k];
      }
    }
    if (Mr != -INFINITY) {
      const float Mn = fmaxf(M, Mr);
      const float sa = M == -INFINITY ? 0.f : expf(M - Mn), sb = expf(Mr - Mn);
      L = L * sa + Lr * sb;
#pragma unroll
      for (int k = 0; k < VW; k++) R[k] = R[k] * sa + Rr[k] * sb;
      M = Mn;
    }
  }
}

// One round of attention tasks in a workgroup of kTaskItems waves: slot s =
// wave / T takes task `task` of head h as given by slot(s, T, n_tasks, h,
// task) (false: none), its T items (T = attention_task_items) one per wave.  Each wave's
// partial goes to `part` (LDS, kTaskItems partials); the slot's first wave
// folds the slot's partials in item order into the task partial.  A head of
// one task writes its output from there.  Otherwise every task but the
// head's last publishes its partial with device-scope 64-bit stores that
// carry the step's tag beside each value; the last task (the one holding the
// current position) reads the others' until every tag is this step's and
// folds them with the running-max rescaling of flash decoding.  A partial
// whose scores are all -inf contributes exp(-inf) = 0; without a finite
// positive total the weights fall back to uniform, as softmax_inplace does
// (src/model.rs:298-313).  Every wave of the workgroup runs the round (its
// workgroup barrier is uniform).  COH: the output is read by other
// workgroups of the same launch (the persistent decode kernel), so it is
// stored at device scope.
template <int HD, bool COH, bool MULTI, bool EARLY = false, class Slot, class Wait = NoWait>
__device__ void attention_round(const AttnArgs &a, int pos, Slot &&slot, float *qs, float *kn, float *part,
                                Wait &&wait = Wait{}) {
#pragma clang fp contract(off)
  using Gm = AttnGeom<HD>;
  constexpr int VW = Gm::VW, VL = Gm::VL, PF = Gm::kPart;
  const int wave = thread_x() >> 6, lane = thread_x() & 63;
  const int vd = (lane % VL) * VW;
  const int S = MULTI ? attention_span(pos, a.nh) : 1;
  const int n_items = pos / (S * kChunk) + 1;
  const int T = attention_task_items(n_items, a.fold_max), lt = __builtin_ctz(T);  // T is a power of two
  const int n_tasks = (n_items + T - 1) >> lt;
  const int sl = wave >> lt, wi = wave & (T - 1);
  int h = 0, task = 0;
  const bool act = slot(sl, T, n_tasks, h, task);
  const int i0 = task << lt, n_in = act ? min(T, n_items - i0) : 0;
  if (wi < n_in) {
    AttnPart<HD> P;
    attention_item<HD, MULTI, EARLY>(a, h, i0 + wi, pos, qs, kn, wait, P);
    float *mine = part + wave * PF;
    if (lane < VL) {
#pragma unroll
      for (int k = 0; k < VW; k++) {
        mine[vd + k] = P.O[k];
        mine[HD + vd + k] = P.Vs[k];
      }
    }
    if (lane == 0) {
      mine[2 * HD] = P.m;
      mine[2 * HD + 1] = P.l;
    }
  } else {
    wait();
  }
  __syncthreads();
  if (wi != 0 || n_in == 0) return;

  // The task partial: items in order, weights exp(m_i - M).
  const float *pt = part + (wave - wi) * PF;
  float M = -INFINITY, L = 0.f, R[VW], V[VW];
  for (int i = 0; i < n_in; i++) M = fmaxf(M, pt[i * PF + 2 * HD]);
#pragma unroll
  for (int k = 0; k < VW; k++) R[k] = V[k] = 0.f;
  for (int i = 0; i < n_in; i++) {
    const float *pi = pt + i * PF;
    const float mi = pi[2 * HD];
    const float w = mi == -INFINITY ? 0.f : expf(mi - M);
    L += w * pi[2 * HD + 1];
#pragma unroll
    for (int k = 0; k < VW; k++) {
      R[k] += w * pi[vd + k];
      V[k] += pi[HD + vd + k];
    }
  }

  float *out = a.out + (size_t)h * HD;
  const long stride = a.part_stride;
  unsigned long long *const base = a.scratch + (size_t)h * (size_t)a.max_chunks * stride;
  const unsigned tag = a.tag;
  if (n_tasks > 1 && task != n_tasks - 1) {  // publish the task partial
    unsigned long long *pt = base + (size_t)task * stride;
    if (lane < VL) {
#pragma unroll
      for (int k = 0; k < VW; k++) {
        store_tagged(pt + vd + k, R[k], tag);
        store_tagged(pt + HD + vd + k, V[k], tag);
      }
    }
    if (lane == 0) {
      store_tagged(pt + 2 * HD, M, tag);
      store_tagged(pt + 2 * HD + 1, L, tag);
    }
    return;
  }
  unsigned long long t0 = 0;
  if (n_tasks > 1) fold_scratch<HD>(a, base, n_tasks - 1, M, L, R, t0);
  if (lane < VL) {
    if (isfinite(L) && L > 0.f) {
#pragma unroll
      for (int k = 0; k < VW; k++) st_act<COH>(out + vd + k, R[k] / L);
    } else {
      // Uniform weights: the V sums of the other tasks, in task order, then this one's.
      float Vt[VW];
#pragma unroll
      for (int k = 0; k < VW; k++) Vt[k] = 0.f;
      for (int c = 0; c < n_tasks - 1; c++) {
        float vc[VW];
        while (true) {
          bool ok = true;
#pragma unroll
          for (int k = 0; k < VW; k++) vc[k] = load_tagged(base + (size_t)c * stride + HD + vd + k, tag, ok);
          if (ok || merge_wait_over(t0, a.err)) break;
          __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int k = 0; k < VW; k++) Vt[k] += vc[k];
      }
#pragma unroll
      for (int k = 0; k < VW; k++) st_act<COH>(out + vd + k, (Vt[k] + V[k]) / (float)(pos + 1));
    }
  }
}

}  // namespace llrs
