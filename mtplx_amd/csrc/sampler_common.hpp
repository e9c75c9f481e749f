// Shared pieces of the sampler's vocabulary reduction: the chunk partial
// record (one 4096-id chunk of one row), the order-preserving u64 keys
// ("value desc, id asc" as one unsigned max) and the wave reductions. Used
// by sampler.hip and by the lm_head epilogue that writes chunk partials
// directly (qmv_stream.hpp, E_STORE_TOPK).
#pragma once

#include "common.hpp"

#include <math.h>

namespace mtp {

constexpr int kSampThreads = 512;
constexpr int kEPT = 8;                           // logits per thread per chunk
constexpr int kChunk = kSampThreads * kEPT;       // 4096
constexpr int kMaxTopK = 64;
constexpr int kTopkStageKeys = 16 * kMaxTopK;   // a merging wave's LDS: up to 16 lists of kMaxTopK keys
constexpr int kTopkParts = 64;                   // partial records per row from the fused lm_head

struct ChunkPart {
  double m;             // max of l/T over the chunk (-inf if all -inf)
  double s;             // sum exp(l/T - m)
  int nonfinite;        // NaN or +inf seen
  int pad;
  uint64_t keys[kMaxTopK];
};

__device__ __forceinline__ uint32_t ordered_bits(float v) {
  uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint64_t key) {
  uint32_t o = (uint32_t)(key >> 32);
  uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}

__device__ __forceinline__ int key_id(uint64_t key) { return (int)(~(uint32_t)key); }

__device__ __forceinline__ uint64_t make_key(float v, int id) {
  return ((uint64_t)ordered_bits(v) << 32) | (uint64_t)(~(uint32_t)id);
}

// Wave-uniform lane reads (v_readlane: the lane index must be uniform) and
// DPP row steps, so the wave reductions below use no LDS permutes. Call them
// from uniform control flow.
__device__ __forceinline__ uint32_t rl32(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ uint64_t rl64(uint64_t v, int l) {
  return ((uint64_t)rl32((uint32_t)(v >> 32), l) << 32) | rl32((uint32_t)v, l);
}
__device__ __forceinline__ double rlf64(double v, int l) {
  return __longlong_as_double((long long)rl64((uint64_t)__double_as_longlong(v), l));
}
__device__ __forceinline__ int rli(int v, int l) { return (int)rl32((uint32_t)v, l); }

template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}
template <int CTRL>
__device__ __forceinline__ double dppf64(double v) {
  return __longlong_as_double((long long)dpp64<CTRL>((uint64_t)__double_as_longlong(v)));
}
// Row (16-lane) steps: quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror.
constexpr int kDppX1 = 0xB1, kDppX2 = 0x4E, kDppHalf = 0x141, kDppRow = 0x140;

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = umax64(v, dpp64<kDppX1>(v));
  v = umax64(v, dpp64<kDppX2>(v));
  v = umax64(v, dpp64<kDppHalf>(v));
  v = umax64(v, dpp64<kDppRow>(v));
  return umax64(umax64(rl64(v, 0), rl64(v, 16)), umax64(rl64(v, 32), rl64(v, 48)));
}

__device__ __forceinline__ double wave_max_f64(double v) {
  v = fmax(v, dppf64<kDppX1>(v));
  v = fmax(v, dppf64<kDppX2>(v));
  v = fmax(v, dppf64<kDppHalf>(v));
  v = fmax(v, dppf64<kDppRow>(v));
  return fmax(fmax(rlf64(v, 0), rlf64(v, 16)), fmax(rlf64(v, 32), rlf64(v, 48)));
}

// Fixed tree: pairs, quads, eights, rows (each step commutative, so every
// lane of a row holds the same sum), then the four rows.
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dppf64<kDppX1>(v);
  v += dppf64<kDppX2>(v);
  v += dppf64<kDppHalf>(v);
  v += dppf64<kDppRow>(v);
  return (rlf64(v, 0) + rlf64(v, 16)) + (rlf64(v, 32) + rlf64(v, 48));
}

// Agent-scope 64-bit stores/loads of the records another workgroup merges.
__device__ __forceinline__ void st_u64_agent(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_u64_agent(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_f64_agent(double* p, double v) {
  st_u64_agent(reinterpret_cast<uint64_t*>(p), (uint64_t)__double_as_longlong(v));
}
__device__ __forceinline__ double ld_f64_agent(const double* p) {
  return __longlong_as_double((long long)ld_u64_agent(reinterpret_cast<const uint64_t*>(p)));
}

// One wave: the partial record of n <= 1024 values vals[0..n) held in LDS,
// in 32-value tiles: value i has id id0 + (i / 32) * tstride + i % 32 (ids
// >= V are outside the vocabulary). Stored to out with agent-scope stores.
// The sampler's per-chunk arithmetic on another set of ids: fp64 l/T, the
// maximum, sum exp(l/T - max), the non-finite flag, and the top-ksel keys by
// repeated wave maxima over cached per-lane bests.
__device__ inline void wave_sub_partial(const float* vals, int n, int id0, int tstride, int V, double temp,
                                        int ksel, int greedy, ChunkPart* out) {
  constexpr int kPer = 16;
  const int lane = threadIdx.x & 63;
  float v[kPer];
  double qv[kPer];
  uint64_t keys[kPer];
  bool ok[kPer];
  const int ne = (n + 63) >> 6;   // slots holding any value (wave-uniform): the rest are skipped
  int nonfinite = 0;
  double mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    ok[e] = false;
    keys[e] = 0ull;
    qv[e] = -INFINITY;
    if (e < ne) {
      const int i = e * 64 + lane;
      const int id = id0 + (i >> 5) * tstride + (i & 31);
      const bool valid = i < n && id < V;
      ok[e] = valid;
      v[e] = valid ? vals[i] : -INFINITY;
      if (valid && (isnan(v[e]) || (isinf(v[e]) && v[e] > 0))) nonfinite = 1;
      if (!greedy) {
        qv[e] = (double)v[e] / temp;
        mloc = fmax(mloc, qv[e]);
      }
      keys[e] = (valid && !isnan(v[e])) ? make_key(v[e], id) : 0ull;
    }
  }
  double m = -INFINITY, s = 0.0;
  if (!greedy) {
    m = wave_max_f64(mloc);
    double sl = 0.0;
    if (m > -INFINITY) {
#pragma unroll
      for (int e = 0; e < kPer; ++e)
        if (e < ne && ok[e]) sl += exp(qv[e] - m);
    }
    s = wave_sum_f64(sl);
  }
  const int nf = __any(nonfinite) ? 1 : 0;
  uint64_t best = 0ull;
#pragma unroll
  for (int e = 0; e < kPer; ++e) best = keys[e] > best ? keys[e] : best;
  for (int r = 0; r < ksel; ++r) {
    const uint64_t win = wave_max_u64(best);
    if (lane == 0) st_u64_agent(&out->keys[r], win);
    if (win != 0ull && best == win) {
      uint64_t nb = 0ull;
#pragma unroll
      for (int e = 0; e < kPer; ++e)
        if (e < ne && keys[e] < win && keys[e] > nb) nb = keys[e];
      best = nb;
    }
  }
  if (lane == 0) {
    st_f64_agent(&out->m, m);
    st_f64_agent(&out->s, s);
    __hip_atomic_store(&out->nonfinite, nf, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// One wave: merge n <= 16 partial records subs[0..n) (agent-scope loads) of
// consecutive id ranges into the record out: the maximum of the maxima, the
// sum of s_i exp(m_i - m) in record order, the OR of the flags, and the
// top-ksel keys by a k-way merge of the sorted lists. The lists are first
// copied into the wave's LDS area stage (n * ksel keys, all loads in flight
// at once), so the merge rounds read LDS (lanes 0..n-1 hold the list heads;
// a 16-lane DPP maximum picks the winner).
__device__ inline void wave_merge_subs(const ChunkPart* subs, int n, int ksel, int greedy, ChunkPart* out,
                                       uint64_t* stage) {
  const int lane = threadIdx.x & 63;
  for (int i = lane; i < n * ksel; i += 64) {
    const int l = i / ksel;
    stage[i] = ld_u64_agent(&subs[l].keys[i - l * ksel]);
  }
  double mi = -INFINITY, si = 0.0;
  int nfi = 0;
  if (lane < n) {
    mi = ld_f64_agent(&subs[lane].m);
    si = ld_f64_agent(&subs[lane].s);
    nfi = __hip_atomic_load(&subs[lane].nonfinite, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  int ptr = 0;
  uint64_t h = lane < n ? stage[lane * ksel] : 0ull;
  for (int r = 0; r < ksel; ++r) {
    uint64_t w = h;
    w = umax64(w, dpp64<kDppX1>(w));
    w = umax64(w, dpp64<kDppX2>(w));
    w = umax64(w, dpp64<kDppHalf>(w));
    w = umax64(w, dpp64<kDppRow>(w));
    const uint64_t win = rl64(w, 0);
    if (lane == 0) out->keys[r] = win;
    if (lane < n && win != 0ull && h == win) {
      ++ptr;
      h = ptr < ksel ? stage[lane * ksel + ptr] : 0ull;
    }
  }
  // maxima, flags and sums in record order (lanes 0..n-1 hold record lane)
  double m = -INFINITY;
  int nf = 0;
  for (int i = 0; i < n; ++i) {
    m = fmax(m, rlf64(mi, i));
    nf |= rli(nfi, i);
  }
  double s = 0.0;
  if (!greedy && m > -INFINITY) {
    for (int i = 0; i < n; ++i) {
      const double mm = rlf64(mi, i);
      if (mm > -INFINITY) s += rlf64(si, i) * exp(mm - m);
    }
  }
  if (lane == 0) {
    out->m = m;
    out->s = s;
    out->nonfinite = nf;
  }
}

}  // namespace mtp
