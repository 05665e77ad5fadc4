// Device side of decode attention: one (query head, chunk of positions)
// item per wave, shared by the attention kernel and the persistent decode
// kernel.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "common.h"
#include "decode.h"
#include "quant_dev.h"

namespace llrs {

// *pos clamped into [0, max_seq): even a corrupted position never indexes
// outside the cache.
__device__ __forceinline__ int bounded_pos(const int *pos, int max_seq) {
  int p = *pos;
  return p < 0 ? 0 : p >= max_seq ? max_seq - 1 : p;
}

// ------------------------------------------------------------------ attention
//
// One wave per (query head, item of attention_span(pos, nh) consecutive
// chunks of kChunk positions: one chunk while every head's items fit the
// wave slots); items past the current position exit at once, so one grid
// (sized for the whole context) serves every position of a captured graph.  Per chunk: split-half RoPE
// (src/model.rs:87-95) on the head's query, scores q.k * 1/sqrt(hd), softmax
// partials (max, sum of exp) and exp-weighted V sums (src/model.rs:206-231,
// softmax_inplace 298-313).  The chunk holding the current position also
// rotates the new key, and the group's first head appends key and value to
// the cache (KVCache::update, src/cache.rs:38-53).
//
// Decode attention moves a few MB per layer, so latency bounds it: each wave
// issues all its K and V loads first and works without workgroup barriers.
// The chunks of a head meet without counters: every chunk but the last
// publishes its partial with device-scope 64-bit stores that carry the
// step's tag beside each value, and returns at once; the last chunk (the one
// holding the current position) computes its own partial, then reads the
// others' until every tag is this step's, and folds them with the running-max
// rescaling of flash decoding.  One round trip on the merging path, none on
// the others, no cache write-back.  A head of more than kGroupFrom items
// merges in two levels (groups of kGroup, see step 5 below).  A chunk whose scores are all -inf
// contributes exp(-inf) = 0; without a finite positive total the weights fall
// back to uniform, as softmax_inplace does.


// Whether a merge has waited ~20 ms for partials that never came; then *err
// is set and the merge goes on with what it read.
__device__ __forceinline__ bool merge_wait_over(unsigned long long &t0, unsigned *err) {
  return tagged_wait_over(t0, err);
}

// One (query head, chunk) item, run by one wave.  COH: the output is read by
// other workgroups of the same launch (the persistent decode kernel), so it is
// stored at device scope.  qs and kn are the wave's own LDS (HD floats each).
// MULTI: the instantiation for attention_span(pos, nh) > 1 (the other one
// assumes single-chunk items and keeps their code straight-line).
// EARLY (the persistent kernel): `wait` is the phase barrier, which ends in a
// workgroup barrier.  The hardware's s_barrier counts waves, not call sites,
// and waves run different numbers of items, so an item contains no
// workgroup barrier of its own and calls `wait` exactly once on every path
// past the c0 > pos check (a wave with no item waits after its item loop).
struct NoWait {
  __device__ void operator()() const {}
};

template <int HD, bool COH, bool MULTI, bool EARLY = false, class Wait = NoWait>
__device__ void attention_item(const AttnArgs &a, int h, int chunk, int pos, float *qs, float *kn,
                               Wait &&wait = Wait{}) {
  constexpr int KH = HD / 2;              // dimensions per score lane
  constexpr int NK4 = KH / 4;             // their float4s
  constexpr int VW = HD >= 64 ? HD / 64 : 1;  // V floats per lane
  constexpr int VL = HD / VW;             // lanes covering one V row
  constexpr int RV = 64 / VL;             // V rows per load instruction
  constexpr int NVI = kChunk / RV;        // V load instructions
  static_assert(NK4 >= 1 && VW <= 2 && RV * VL == 64, "head_dim must be 16..128");
  using VT = typename std::conditional<VW == 2, float2, float>::type;

  const int G = a.nh / a.nkv, kvw = a.nkv * HD;
  const int kvh = h / G;
  const int S = MULTI ? attention_span(pos, a.nh) : 1, span = S * kChunk;
  const int c0 = chunk * span;  // this item: positions [c0, c0 + span), S sub-chunks
  if (c0 > pos) return;
  const int n_active = pos / span + 1;  // items of the head
  const bool owns_new = pos < c0 + span;
  const int lane = thread_x() & 63, half = lane >> 5, pl = lane & 31;
  const float *kc = a.k_cache + (size_t)kvh * HD, *vc = a.v_cache + (size_t)kvh * HD;

  // 1. Loads, all issued up front: this lane's query and new-key pair
  //    (i, i + KH) with its RoPE factors and its dimensions of the new value;
  //    then the first sub-chunk's keys (lane = half x position, KH dims) and
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
    const float *kp = kc + (size_t)(s0 + pl < s1 ? s0 + pl : s0) * kvw + half * KH;
#pragma unroll
    for (int j = 0; j < NK4; j++) kr[j] = *reinterpret_cast<const float4 *>(kp + 4 * j);
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

  // 3-4. Per sub-chunk: scores of positions pl (both halves end with the
  //    full dot), the softmax partials, exp-weighted and plain V sums of the
  //    lane's VW dimensions; sub-chunks after the first fold in with the
  //    running-max rescaling (their rows load after the previous one's sums).
  float m = -INFINITY, l = 0.f, O[VW], Vs[VW];
#pragma unroll
  for (int k = 0; k < VW; k++) O[k] = Vs[k] = 0.f;
  for (int sub = 0; sub < S; sub++) {
    const int s0 = c0 + sub * kChunk;
    if (s0 > pos) break;
    const int s1 = min(s0 + kChunk, pos + 1);  // exclusive
    if (sub > 0) load_rows(s0, s1);
    if (s0 <= pos && pos < s1) {  // the row this step appends, from registers / LDS
      if (s0 + pl == pos) {
#pragma unroll
        for (int j = 0; j < NK4; j++) kr[j] = *reinterpret_cast<const float4 *>(kn + half * KH + 4 * j);
      }
#pragma unroll
      for (int i = 0; i < NVI; i++)
        if (s0 + i * RV + vr0 == pos) vv[i] = vnew;
    }
    float sc = 0.f;
#pragma unroll
    for (int j = 0; j < NK4; j++) {
      const float4 q4 = *reinterpret_cast<const float4 *>(qs + half * KH + 4 * j);
      sc += q4.x * kr[j].x + q4.y * kr[j].y + q4.z * kr[j].z + q4.w * kr[j].w;
    }
    sc += __shfl_xor(sc, 32, 64);
    const bool valid = s0 + pl < s1;
    sc = valid ? sc * a.scale : -INFINITY;
    float ms = sc;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) ms = fmaxf(ms, __shfl_xor(ms, o, 64));
    const float x = valid ? expf(sc - ms) : 0.f;
    float ls = x;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) ls += __shfl_xor(ls, o, 64);
    float Os[VW], Vss[VW];
#pragma unroll
    for (int k = 0; k < VW; k++) Os[k] = Vss[k] = 0.f;
#pragma unroll
    for (int i = 0; i < NVI; i++) {
      const int p = i * RV + vr0;  // position within the sub-chunk
      float wp;  // exp weight of position p, held by lane p
      if constexpr (RV == 1)
        wp = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), i));
      else
        wp = __shfl(x, p, 64);
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
        Os[k] += __shfl_xor(Os[k], o, 64);
        Vss[k] += __shfl_xor(Vss[k], o, 64);
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

  float *out = a.out + (size_t)h * HD;
  if (n_active == 1) {  // the only chunk: finish here
    if (lane < VL) {
      const bool ok = isfinite(l) && l > 0.f;
#pragma unroll
      for (int k = 0; k < VW; k++) st_act<COH>(out + vd + k, ok ? O[k] / l : Vs[k] / (float)(pos + 1));
    }
    return;
  }

  // 5. Every chunk but the last publishes [HD] O sums, [HD] V sums, max, sum.
  //    Past kGroupFrom items a head merges in two levels: the last item of
  //    each group of kGroup chunks also folds its group's other partials into
  //    a group partial (slot max_chunks + group), and the head's last item
  //    folds its own group's partials, then the group partials.
  const long stride = a.part_stride;
  unsigned long long *const base =
      a.scratch + (size_t)h * (size_t)(a.max_chunks + attention_groups(a.max_chunks)) * stride;
  unsigned long long *const gbase = base + (size_t)a.max_chunks * stride;
  const unsigned tag = a.tag;
  const bool last = chunk == n_active - 1;
  const bool grouped = n_active > kGroupFrom;
  const int grp = chunk / kGroup;
  const bool leader = grouped && !last && chunk % kGroup == kGroup - 1;
  auto publish = [&](unsigned long long *part, float mv, float lv, const float (&o)[VW], const float (&vsum)[VW]) {
    if (lane < VL) {
#pragma unroll
      for (int k = 0; k < VW; k++) {
        store_tagged(part + vd + k, o[k], tag);
        store_tagged(part + HD + vd + k, vsum[k], tag);
      }
    }
    if (lane == 0) {
      store_tagged(part + 2 * HD, mv, tag);
      store_tagged(part + 2 * HD + 1, lv, tag);
    }
  };
  if (!last) {
    publish(base + (size_t)chunk * stride, m, l, O, Vs);
    if (!leader) return;
  }

  // 6. Merge, starting from the own partial.  Partials `first .. first + n`
  //    of `slots`: their statistics one per lane (64 a round) load together
  //    with their first OB O partials; a load round is repeated until every
  //    tag is this step's.  The round's max by wave reduction, each partial's
  //    weight exp(m_c - M) in its lane, broadcast by readlane to weight the O
  //    partials.  Rounds fold with the running-max rescaling; a partial whose
  //    max is -inf weighs 0.
  constexpr int OB = 32 / VW;  // O partials per load round
  float M = m, L = l, R[VW];
#pragma unroll
  for (int k = 0; k < VW; k++) R[k] = O[k];
  unsigned long long t0 = 0;
  const int g0 = grouped ? grp * kGroup : 0;  // the first chunk partial this item folds
  // Level 0: chunk partials g0 .. chunk - 1 (the leader then publishes the
  // group partial and returns); level 1 (the head's last item when grouped):
  // group partials 0 .. grp - 1.  One loop, so the merge code exists once.
  for (int level = 0; level < (grouped && !leader ? 2 : 1); level++) {
    const unsigned long long *slots = level ? gbase : base + (size_t)g0 * stride;
    const int np = level ? grp : chunk - g0;
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
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) Mr = fmaxf(Mr, __shfl_xor(Mr, o, 64));
      const float w = in ? expf(mm - Mr) : 0.f;
      float Lr = w * ll;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) Lr += __shfl_xor(Lr, o, 64);
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
  if (leader) {  // the group partial; the V sums stay in the chunk slots
    publish(gbase + (size_t)grp * stride, M, L, R, Vs);
    return;
  }
  const int np = n_active - 1;  // the chunk partials (the uniform fallback reads their V sums)
  if (lane < VL) {
    if (isfinite(L) && L > 0.f) {
#pragma unroll
      for (int k = 0; k < VW; k++) st_act<COH>(out + vd + k, R[k] / L);
    } else {
      float V[VW];
#pragma unroll
      for (int k = 0; k < VW; k++) V[k] = Vs[k];
      for (int c = 0; c < np; c++) {
        float vc[VW];
        while (true) {
          bool ok = true;
#pragma unroll
          for (int k = 0; k < VW; k++) vc[k] = load_tagged(base + (size_t)c * stride + HD + vd + k, tag, ok);
          if (ok || merge_wait_over(t0, a.err)) break;
          __builtin_amdgcn_s_sleep(1);
        }
#pragma unroll
        for (int k = 0; k < VW; k++) V[k] += vc[k];
      }
#pragma unroll
      for (int k = 0; k < VW; k++) st_act<COH>(out + vd + k, V[k] / (float)(pos + 1));
    }
  }
}

}  // namespace llrs
