// Shared pieces of the sampler's vocabulary reduction: the chunk partial
// record (one 4096-id chunk of one row), the order-preserving u64 keys
// ("value desc, id asc" as one unsigned max) and the wave reductions. Used
// by sampler.hip.
#pragma once

#include "common.hpp"

#include <math.h>

namespace mtp {

constexpr int kSampThreads = 512;
constexpr int kEPT = 8;                           // logits per thread per chunk
constexpr int kChunk = kSampThreads * kEPT;       // 4096
constexpr int kMaxTopK = 64;

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

__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v, uint32_t w) { return v > w ? v : w; }
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = dpp_max_u32(v, dpp32<kDppX1>(v));
  v = dpp_max_u32(v, dpp32<kDppX2>(v));
  v = dpp_max_u32(v, dpp32<kDppHalf>(v));
  v = dpp_max_u32(v, dpp32<kDppRow>(v));
  return dpp_max_u32(dpp_max_u32(rl32(v, 0), rl32(v, 16)), dpp_max_u32(rl32(v, 32), rl32(v, 48)));
}

// The u64 maximum as 32-bit ones: the high words, then, when more than one
// lane holds the maximal high word, the low words of those lanes
// (lexicographic, so the same value as a 64-bit reduction, with
// single-instruction DPP steps). A single holder's key is read directly.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  const uint32_t hi = (uint32_t)(v >> 32);
  const uint32_t mh = wave_max_u32(hi);
  const uint64_t at = __ballot(hi == mh);
  if (__popcll(at) == 1) return ((uint64_t)mh << 32) | rl32((uint32_t)v, __ffsll((unsigned long long)at) - 1);
  const uint32_t ml = wave_max_u32(hi == mh ? (uint32_t)v : 0u);
  return ((uint64_t)mh << 32) | ml;
}

// Bitonic sort of one key per lane across the wave, descending (lane 0 the
// largest). Call from uniform control flow.
__device__ __forceinline__ uint64_t wave_sort_desc_u64(uint64_t kv) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(kv >> 32), stride, 64) << 32) |
                         (uint32_t)__shfl_xor((int)(uint32_t)kv, stride, 64);
      const bool lower = (lane & stride) == 0;
      const bool desc = (lane & size) == 0;   // the last pass (size 64) orders all 64 descending
      const bool take_max = lower == desc;
      kv = take_max ? (kv > o ? kv : o) : (kv < o ? kv : o);
    }
  }
  return kv;
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



}  // namespace mtp
