// Expert-sorted MoE dispatch around the gathered quantized matmul, gfx950.
//
//  * mtp_moe_route: per token, top-k of the router logits plus an optional
//    per-expert skew (value desc, id asc) and the softmax weights
//    renormalised over the chosen k (softmax over all experts, top-k of the
//    probabilities, renormalised: mtplx/models/qwen4_exp.py:1430-1437).
//  * mtp_moe_sort: stable counting sort of the flattened top-k expert ids —
//    the closed form of mtplx/moe_sorted_gather.py:221-238 sort_rows:
//      order = stable_argsort(flat), inv_order = argsort(order),
//      row_map = order // top_k, sorted = flat[order]
//    plus expert row offsets and the compact list of experts that got rows
//    (the gathered matmul launches one workgroup column per active expert).
//  * mtp_moe_segments: expert offsets and the active list from ids already
//    in sorted order (the reference entry points take sorted indices).
//  * mtp_moe_combine: unsort + route-weighted sum over top_k, plus the
//    sigmoid-gated shared expert and the residual: the block tail of
//    mtplx/models/qwen4_exp.py:1438-1445 and :1544-1577.
#include "common.hpp"
#include "sampler_common.hpp"

namespace mtp {

constexpr int kSortThreads = 1024;
constexpr int kMaxSortRows = 8192;
constexpr int kMaxExperts = 4096;

__global__ __launch_bounds__(kSortThreads) void moe_sort_kernel(const int32_t* ids, int R, int top_k, int E,
                                                                uint32_t* row_map, uint32_t* sorted_ids,
                                                                uint32_t* inv_order, int32_t* expert_off,
                                                                int32_t* active) {
  __shared__ int s_ids[kMaxSortRows];
  __shared__ int s_cnt[kMaxExperts + 1];
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  if (tid == 0) s_bad = 0;
  for (int e = tid; e <= E; e += kSortThreads) s_cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < R; i += kSortThreads) {
    const int e = ids[i];
    s_ids[i] = e;
    if (e < 0 || e >= E)
      s_bad = 1;
    else
      atomicAdd(&s_cnt[e], 1);
  }
  __syncthreads();
  if (s_bad) {
    // An id outside [0, E): flag it and leave outputs that index only inside
    // their buffers (identity order, empty expert ranges), so a consumer that
    // does not check the flag reads valid rows and runs no expert.
    for (int i = tid; i < R; i += kSortThreads) {
      row_map[i] = (uint32_t)(i / top_k);
      sorted_ids[i] = 0;
      inv_order[i] = (uint32_t)i;
    }
    for (int e = tid; e <= E; e += kSortThreads) expert_off[e] = 0;
    if (tid == 0) active[0] = -1;
    return;
  }
  // Exclusive scans of the counts and of the active flags (E <= 4096: each
  // thread takes 4 consecutive experts; integer sums, so any order is exact).
  {
    constexpr int kPer = kMaxExperts / kSortThreads;   // 4
    int c[kPer], rows = 0, acts = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid * kPer + j;
      c[j] = e < E ? s_cnt[e] : 0;
      rows += c[j];
      acts += c[j] > 0;
    }
    // inclusive scans over the workgroup: waves by shuffles, then the wave totals
    int ir = rows, ia = acts;
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int r = __shfl_up(ir, off, 64), a = __shfl_up(ia, off, 64);
      if (lane >= off) {
        ir += r;
        ia += a;
      }
    }
    __shared__ int s_wr[kSortThreads / 64], s_wa[kSortThreads / 64];
    if (lane == 63) {
      s_wr[wave] = ir;
      s_wa[wave] = ia;
    }
    __syncthreads();
    int br = 0, ba = 0;
    for (int w2 = 0; w2 < wave; ++w2) {
      br += s_wr[w2];
      ba += s_wa[w2];
    }
    int run = br + ir - rows, na = ba + ia - acts;   // exclusive prefix of this thread's first expert
    __syncthreads();   // every thread has read its counts: s_cnt may take the offsets
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int e = tid * kPer + j;
      if (e < E) {
        expert_off[e] = run;
        if (c[j] > 0) active[1 + na++] = e;
        s_cnt[e] = run;
        run += c[j];
      }
    }
    if (tid == kSortThreads - 1) {
      expert_off[E] = run;
      active[0] = na;
    }
  }
  __syncthreads();
  // Stable positions, 64 rows (one wave) at a time in row order: within a
  // wave the rows routed to the same expert are matched by ballots over the
  // id's bits, and each group's first lane takes the group's run of positions
  // from the expert's running offset (s_cnt); the rounds run in row order,
  // one workgroup barrier each, so earlier rows always come first.
  const int lane = tid & 63, wave = tid >> 6;
  for (int c0 = 0; c0 < R; c0 += kSortThreads) {
    const int i = c0 + tid;
    const bool valid = i < R;
    const int e = valid ? s_ids[i] : 0;
    unsigned long long m = __ballot(valid);
    for (int b = 0; (1 << b) < E; ++b) {   // uniform
      const bool bit = ((e >> b) & 1) != 0;
      const unsigned long long bal = __ballot(valid && bit);
      m &= bit ? bal : ~bal;
    }
    if (!valid) m = 0ull;
    const int leader = m ? __ffsll(m) - 1 : lane;
    int base = 0;
    const int nwav = (R - c0 + 63) >> 6 < kSortThreads / 64 ? (R - c0 + 63) >> 6 : kSortThreads / 64;
    for (int w = 0; w < nwav; ++w) {
      if (wave == w && valid && lane == leader) {
        base = s_cnt[e];
        s_cnt[e] = base + __popcll(m);
      }
      __syncthreads();
    }
    base = __shfl(base, leader, 64);
    if (valid) {
      const int pos = base + __popcll(m & ((1ull << lane) - 1ull));
      row_map[pos] = (uint32_t)(i / top_k);
      sorted_ids[pos] = (uint32_t)e;
      inv_order[i] = (uint32_t)pos;
    }
  }
}

// One wave per token: top-k experts and renormalised softmax weights.
// Each candidate is the u64 key (order-preserving value bits << 32 | ~id),
// so "value desc, id asc" is one unsigned max; -0 is folded into +0 first,
// so equal values tie on the id as the float comparison does, and NaN never
// wins (key 0). Up to kRouteRegE experts the keys stay in registers and
// each of the k rounds is a DPP wave max; wider rows go through LDS.
constexpr int kRouteMaxE = 4096;
constexpr int kRouteRegE = 512;

__device__ __forceinline__ uint64_t route_key(float v, int e) {
  if (v != v) return 0ull;
  return make_key(v + 0.0f, e);   // -0 + 0 = +0
}

__device__ __forceinline__ void route_finish(const float* s_val, const int* s_id, int t, int top_k, int32_t* ids,
                                             float* weights) {
  const float mx = s_val[0];
  float sum = 0.f;
  for (int r = 0; r < top_k; ++r) sum += __expf(s_val[r] - mx);
  for (int r = 0; r < top_k; ++r) {
    ids[(size_t)t * top_k + r] = s_id[r];
    weights[(size_t)t * top_k + r] = __expf(s_val[r] - mx) / sum;
  }
}

__global__ __launch_bounds__(64) void moe_route_kernel(const float* logits, long long ld, const float* skew, int E,
                                                       int top_k, int32_t* ids, float* weights) {
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const float* grow = logits + (size_t)t * ld;
  __shared__ float s_val[64];
  __shared__ int s_id[64];
  if (E <= kRouteRegE) {
    constexpr int kPer = kRouteRegE / 64;
    uint64_t key[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int e = lane + 64 * i;
      key[i] = e < E ? route_key(skew ? grow[e] + skew[e] : grow[e], e) : 0ull;
    }
    uint64_t taken = ~0ull;
    for (int r = 0; r < top_k; ++r) {   // uniform: the DPP max needs every lane
      uint64_t best = 0ull;
#pragma unroll
      for (int i = 0; i < kPer; ++i)
        if (key[i] < taken && key[i] > best) best = key[i];
      best = wave_max_u64(best);
      if (lane == 0) {
        s_val[r] = best ? key_value(best) : -INFINITY;
        s_id[r] = best ? key_id(best) : 0x7fffffff;
      }
      taken = best;
    }
    __syncthreads();
    if (lane == 0) route_finish(s_val, s_id, t, top_k, ids, weights);
    return;
  }
  __shared__ float row[kRouteMaxE];
  for (int e = lane; e < E; e += 64) row[e] = skew ? grow[e] + skew[e] : grow[e];
  __syncthreads();
  int taken_id = -1;
  float taken_val = INFINITY;
  for (int r = 0; r < top_k; ++r) {
    // best below the previous winner in (value desc, id asc) order
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int e = lane; e < E; e += 64) {
      const float v = row[e];
      const bool below = (v < taken_val) || (v == taken_val && e > taken_id);
      if (!below) continue;
      if (v > bv || (v == bv && e < bi)) {
        bv = v;
        bi = e;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      s_val[r] = bv;
      s_id[r] = bi;
    }
    taken_val = bv;
    taken_id = bi;
  }
  __syncthreads();
  if (lane == 0) route_finish(s_val, s_id, t, top_k, ids, weights);
}

// routed = bf16(sum_j w[t,j] * y_sorted[inv_order[t*k + j], :]);
// sh = bf16(sigmoid(gate[t]) * shared[t, :]) (no gate: shared itself);
// out[t, :] = bf16(resid[t, :] + bf16(routed + sh)) (no resid: the block output).
// Each stored tensor of the reference chain is rounded where it stores it.
// One column per thread (grid.x * 256 >= H). ss_out (H % 32 == 0, T <= 32):
// per 32-column block j, ss_out[j * 32 + t] = the sum of the squared stored
// values in column order (the residual epilogue's statistics, read by the
// next fused RMSNorm).
constexpr int kCombineThreads = 256;
__global__ __launch_bounds__(kCombineThreads) void moe_combine_kernel(
    const uint16_t* y_sorted, const uint32_t* inv_order, const float* w, const uint16_t* shared, const float* gate,
    long long gate_ld, const uint16_t* resid, uint16_t* out, float* ss_out, int T, int k, int H) {
  const int t = blockIdx.y;
  const int h = blockIdx.x * kCombineThreads + threadIdx.x;
  const float sg = gate ? 1.0f / (1.0f + __expf(-gate[(size_t)t * gate_ld])) : 1.0f;
  float stored = 0.f;
  if (h < H) {
    float acc = 0.f;
    for (int j = 0; j < k; ++j) {
      const uint32_t r = inv_order[(size_t)t * k + j];
      acc += w[(size_t)t * k + j] * bf2f(y_sorted[(size_t)r * H + h]);
    }
    float v = round_bf(acc);
    if (shared) {
      const float sh = bf2f(shared[(size_t)t * H + h]);
      v = round_bf(v + (gate ? round_bf(sg * sh) : sh));
    }
    if (resid) v = bf2f(resid[(size_t)t * H + h]) + v;
    out[(size_t)t * H + h] = f2bf(v);
    stored = round_bf(v);
  }
  if (ss_out) {   // uniform over the grid
    __shared__ float s_sq[kCombineThreads];
    s_sq[threadIdx.x] = stored * stored;
    __syncthreads();
    const int j = blockIdx.x * (kCombineThreads / 32) + (int)threadIdx.x;
    if (threadIdx.x < kCombineThreads / 32 && j * 32 < H) {
      float a = 0.f;
      for (int c = 0; c < 32; ++c) a += s_sq[threadIdx.x * 32 + c];
      ss_out[(size_t)j * 32 + t] = a;
    }
  }
}

// Offsets of each expert's rows in ids already sorted ascending, and the
// active list; active[0] = -1 flags an id outside [0, E) or a descent.
__global__ __launch_bounds__(kSortThreads) void moe_segments_kernel(const int32_t* sorted_ids, int R, int E,
                                                                    int32_t* expert_off, int32_t* active) {
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  for (int i = tid; i < R; i += kSortThreads) {
    const int e = sorted_ids[i];
    if (e < 0 || e >= E || (i > 0 && sorted_ids[i - 1] > e)) s_bad = 1;
  }
  __syncthreads();
  if (s_bad) {   // empty expert ranges: a consumer that does not check the flag runs no expert
    for (int e = tid; e <= E; e += kSortThreads) expert_off[e] = 0;
    if (tid == 0) active[0] = -1;
    return;
  }
  // off[e] = first i with sorted_ids[i] >= e (binary search per expert).
  for (int e = tid; e <= E; e += kSortThreads) {
    int lo = 0, hi = R;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (sorted_ids[mid] < e) lo = mid + 1; else hi = mid;
    }
    expert_off[e] = lo;
  }
  __syncthreads();
  if (tid == 0) {
    int na = 0;
    for (int e = 0; e < E; ++e)
      if (expert_off[e + 1] > expert_off[e]) active[1 + na++] = e;
    active[0] = na;
  }
}

}  // namespace mtp

using namespace mtp;

MTP_API size_t mtp_moe_workspace_bytes(int T, int top_k, int E) {
  (void)T;
  (void)top_k;
  (void)E;
  return 0;
}

MTP_API int mtp_moe_sort(const int32_t* topk_ids, int T, int top_k, int E, uint32_t* row_map, uint32_t* sorted_ids,
                         uint32_t* inv_order, int32_t* expert_off, int32_t* active, void* ws, size_t ws_bytes,
                         void* stream) {
  (void)ws;
  (void)ws_bytes;
  const int R = T * top_k;
  if (!topk_ids || !row_map || !sorted_ids || !inv_order || !expert_off || !active || T < 1 || top_k < 1 || E < 1) {
    set_error("mtp_moe_sort: bad arguments");
    return MTP_ERR_ARG;
  }
  if (R > kMaxSortRows || E > kMaxExperts) {
    set_error("mtp_moe_sort: %d routed rows / %d experts exceed the single-workgroup sort (%d / %d)", R, E,
              kMaxSortRows, kMaxExperts);
    return MTP_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(kSortThreads), 0, (hipStream_t)stream, topk_ids, R, top_k, E,
                     row_map, sorted_ids, inv_order, expert_off, active);
  return launch_check("mtp_moe_sort");
}

MTP_API int mtp_moe_route(const float* logits, int ld, const float* skew, int T, int E, int top_k, int32_t* ids,
                          float* weights, void* stream) {
  if (ld <= 0) ld = E;
  if (!logits || !ids || !weights || T < 1 || E < 1 || E > kRouteMaxE || ld < E || top_k < 1 || top_k > 64 ||
      top_k > E) {
    set_error("mtp_moe_route: bad arguments (1 <= top_k <= min(64, E), E <= %d, ld >= E)", kRouteMaxE);
    return MTP_ERR_ARG;
  }
  hipLaunchKernelGGL(moe_route_kernel, dim3(T), dim3(64), 0, (hipStream_t)stream, logits, (long long)ld, skew, E,
                     top_k, ids, weights);
  return launch_check("mtp_moe_route");
}

MTP_API int mtp_moe_segments(const int32_t* sorted_ids, int R, int E, int32_t* expert_off, int32_t* active,
                             void* stream) {
  if (!sorted_ids || !expert_off || !active || R < 1 || E < 1) {
    set_error("mtp_moe_segments: bad arguments");
    return MTP_ERR_ARG;
  }
  hipLaunchKernelGGL(moe_segments_kernel, dim3(1), dim3(kSortThreads), 0, (hipStream_t)stream, sorted_ids, R, E,
                     expert_off, active);
  return launch_check("mtp_moe_segments");
}

static int moe_combine_run(const void* y_sorted, const uint32_t* inv_order, const float* route_w, const void* shared,
                           const float* shared_gate, int gate_ld, const void* resid, void* out, float* ss_out, int T,
                           int top_k, int H, void* stream, const char* who) {
  if (!y_sorted || !inv_order || !route_w || !out || T < 1 || top_k < 1 || H < 1 ||
      (shared_gate && (!shared || gate_ld < 1))) {
    set_error("%s: bad arguments", who);
    return MTP_ERR_ARG;
  }
  if (ss_out && (H % 32 || T > 32)) {
    set_error("%s: the sums of squares need H %% 32 == 0 and T <= 32 (got H=%d T=%d)", who, H, T);
    return MTP_ERR_ARG;
  }
  dim3 grid(cdiv(H, kCombineThreads), T);
  hipLaunchKernelGGL(moe_combine_kernel, grid, dim3(kCombineThreads), 0, (hipStream_t)stream,
                     (const uint16_t*)y_sorted, inv_order, route_w, (const uint16_t*)shared, shared_gate,
                     (long long)gate_ld, (const uint16_t*)resid, (uint16_t*)out, ss_out, T, top_k, H);
  return launch_check(who);
}

MTP_API int mtp_moe_combine(const void* y_sorted, const uint32_t* inv_order, const float* route_w,
                            const void* shared, const float* shared_gate, int gate_ld, const void* resid, void* out,
                            int T, int top_k, int H, void* stream) {
  return moe_combine_run(y_sorted, inv_order, route_w, shared, shared_gate, gate_ld, resid, out, nullptr, T, top_k, H,
                         stream, "mtp_moe_combine");
}

MTP_API int mtp_moe_combine_ss(const void* y_sorted, const uint32_t* inv_order, const float* route_w,
                               const void* shared, const float* shared_gate, int gate_ld, const void* resid, void* out,
                               float* ss_out, int T, int top_k, int H, void* stream) {
  return moe_combine_run(y_sorted, inv_order, route_w, shared, shared_gate, gate_ld, resid, out, ss_out, T, top_k, H,
                         stream, "mtp_moe_combine_ss");
}
