// Exact speculative accept/reject over full-vocabulary logits, gfx950.
//
// Law (mtplx/sampling.py:131-391, uniform order mtplx/generation.py:15560-15790
// and :16085-16110):
//   p = renorm( topk(value desc, id asc) ∩ nucleus(cumulative_before < top_p over
//               the full-vocab fp64 softmax of logits/T) ), ids ascending;
//   depth d: a = min(1, p/q) (q<=0: 1 if p>0 else 0); accept iff u_d <= a;
//   first reject: residual max(p-q,0) over the union, renormalised (target if
//   empty), sampled with the next uniform; all accepted: bonus from row K with
//   the next uniform. Sampling is NumPy's Generator.choice rule:
//   idx = #{cdf <= u} with cdf = cumsum(p)/cdf[-1]
//   (mtplx/qwen4_draft_device_chain.py:294-305).
//
// Two kernels:
//  1. vocab_partials: grid (rows, chunks). Each 512-thread workgroup reads a
//     4096-logit chunk once (coalesced), and emits the chunk's fp64 max of
//     l/T, fp64 sum exp(l/T - max), a non-finite flag, and its top-k keys.
//     A key is (order-preserving float bits << 32) | ~id, so one u64 max is
//     "value desc, id asc". Top-k: each wave selects from its 512 logits
//     with per-thread cached bests (each round only the winning thread
//     rescans its 8 registers), then wave 0 merges the eight sorted lists.
//     Target and draft rows go through one launch.
//  2. accept_laws: one workgroup per request, one wave per row law: merges
//     the row's chunks (max/sum-exp combine in fixed chunk order, top-k as a
//     k-way merge of the chunks' sorted lists), builds the sparse law in fp64
//     with the per-candidate work spread over lanes; wave 0 then runs the
//     accept loop. (Vocabularies over 64 chunks use accept_finish, one wave
//     per request building the laws in turn.)
// Deterministic: fixed reduction trees, no float atomics.
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

// grid: (n_chunks, rows). logits row r at logits + r * ld.
// Rows below nrows1 come from logits, the rest from logits2 (row - nrows1).
__global__ __launch_bounds__(kSampThreads) void vocab_partials(const float* __restrict__ logits,
                                                               const float* __restrict__ logits2, int nrows1,
                                                               long long ld, int V, int n_chunks, double temp,
                                                               int ksel, int greedy, ChunkPart* __restrict__ parts) {
  constexpr int NWV = kSampThreads / 64;
  static_assert(NWV == 8, "the list merge reduces over 8 lanes");
  const int chunk = blockIdx.x;
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const float* lr = row < nrows1 ? logits + (size_t)row * ld : logits2 + (size_t)(row - nrows1) * ld;
  const int base = chunk * kChunk;

  float v[kEPT];
  double qv[kEPT];   // l / T in fp64, computed once
  int nonfinite = 0;
  double mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < kEPT; ++e) {
    const int id = base + e * kSampThreads + tid;
    v[e] = (id < V) ? lr[id] : -INFINITY;
  }
#pragma unroll
  for (int e = 0; e < kEPT; ++e) {
    const int id = base + e * kSampThreads + tid;
    const float x = v[e];
    if (id < V && (isnan(x) || (isinf(x) && x > 0))) nonfinite = 1;
    qv[e] = greedy ? 0.0 : (double)x / temp;
    if (!greedy) mloc = fmax(mloc, qv[e]);
  }
  __shared__ double s_red[NWV];
  __shared__ uint64_t s_wkey[NWV][kMaxTopK];
  __shared__ int s_nf[NWV];

  double mchunk = -INFINITY, schunk = 0.0;
  if (!greedy) {
    const double wm = wave_max_f64(mloc);
    if (lane == 0) s_red[wave] = wm;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NWV; ++w) mchunk = fmax(mchunk, s_red[w]);
    __syncthreads();
    double sl = 0.0;
    if (mchunk > -INFINITY) {
#pragma unroll
      for (int e = 0; e < kEPT; ++e) {
        const int id = base + e * kSampThreads + tid;
        if (id < V) sl += exp(qv[e] - mchunk);
      }
    }
    const double ws = wave_sum_f64(sl);
    if (lane == 0) s_red[wave] = ws;
    __syncthreads();
    schunk = ((s_red[0] + s_red[1]) + (s_red[2] + s_red[3])) + ((s_red[4] + s_red[5]) + (s_red[6] + s_red[7]));
  }
  {
    const int nf = __any(nonfinite) ? 1 : 0;
    if (lane == 0) s_nf[wave] = nf;
  }

  // Top-k: each wave selects the top ksel of its own 512 logits (cached
  // per-thread bests, no barriers), then wave 0 merges the NWV sorted lists.
  uint64_t keys[kEPT];
#pragma unroll
  for (int e = 0; e < kEPT; ++e) {
    const int id = base + e * kSampThreads + tid;
    keys[e] = (id < V && !isnan(v[e])) ? make_key(v[e], id) : 0ull;
  }
  uint64_t best = 0ull;
#pragma unroll
  for (int e = 0; e < kEPT; ++e) best = keys[e] > best ? keys[e] : best;

  for (int r = 0; r < ksel; ++r) {
    const uint64_t win = wave_max_u64(best);
    if (lane == 0) s_wkey[wave][r] = win;
    if (win != 0ull && best == win) {
      uint64_t nb = 0ull;
#pragma unroll
      for (int e = 0; e < kEPT; ++e)
        if (keys[e] < win && keys[e] > nb) nb = keys[e];
      best = nb;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  ChunkPart* out = parts + (size_t)row * n_chunks + chunk;
  int ptr = 0;
  uint64_t h = lane < NWV ? s_wkey[lane][0] : 0ull;
  for (int r = 0; r < ksel; ++r) {
    uint64_t w = h;   // max over lanes 0..7 (NWV = 8)
    w = umax64(w, dpp64<kDppX1>(w));
    w = umax64(w, dpp64<kDppX2>(w));
    w = umax64(w, dpp64<kDppHalf>(w));
    const uint64_t win = rl64(w, 0);
    if (lane == 0) out->keys[r] = win;
    if (lane < NWV && win != 0ull && h == win) {
      ++ptr;
      h = ptr < ksel ? s_wkey[lane][ptr] : 0ull;
    }
  }
  if (lane == 0) {
    int nf = 0;
#pragma unroll
    for (int w = 0; w < NWV; ++w) nf |= s_nf[w];
    out->m = mchunk;
    out->s = schunk;
    out->nonfinite = nf;
  }
}

// NumPy's pairwise sum for n <= 128 (numpy/core/src/umath/loops_utils.h):
// sequential below 8, else 8 strided accumulators combined as a tree, then
// the tail added in order.
__device__ double np_sum_small(const double* a, int n) {
  if (n < 8) {
    double r = 0.0;
    for (int i = 0; i < n; ++i) r += a[i];
    return r;
  }
  double r[8];
  for (int j = 0; j < 8; ++j) r[j] = a[j];
  int i = 8;
  for (; i < n - (n % 8); i += 8)
    for (int j = 0; j < 8; ++j) r[j] += a[i + j];
  double res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) res += a[i];
  return res;
}

// np_sum_small of n <= 64 values in LDS, run by a whole wave (same order:
// lanes 0..7 hold the 8 strided accumulators); the result is uniform.
__device__ double np_sum_wave(const double* a, int n) {
  const int lane = threadIdx.x & 63;
  if (n < 8) {
    double r = 0.0;
    for (int i = 0; i < n; ++i) r += a[i];
    return r;
  }
  const int full = n - (n % 8);
  double r = 0.0;
  if (lane < 8) {
    r = a[lane];
    for (int i = 8; i < full; i += 8) r += a[i + lane];
  }
  double res = ((rlf64(r, 0) + rlf64(r, 1)) + (rlf64(r, 2) + rlf64(r, 3))) +
               ((rlf64(r, 4) + rlf64(r, 5)) + (rlf64(r, 6) + rlf64(r, 7)));
  for (int i = full; i < n; ++i) res += a[i];
  return res;
}

struct RowLaw {
  int n;                    // support size (ids ascending)
  int ids[kMaxTopK];
  double probs[kMaxTopK];
  int nonfinite;
};

// Merge one row's chunk partials into its sparse law. Executed by one wave;
// results valid in lane 0's view of *law (law lives in LDS).
__device__ void build_law(const ChunkPart* parts, int n_chunks, int ksel, int greedy, double temp, double top_p,
                          RowLaw* law, uint64_t* s_sel) {
  const int lane = threadIdx.x & 63;
  // fp64 max / sum-exp combine in fixed chunk order.
  int nf = 0;
  double M = -INFINITY;
  for (int c = 0; c < n_chunks; ++c) {
    M = fmax(M, parts[c].m);
    nf |= parts[c].nonfinite;
  }
  double S = 0.0;
  if (!greedy)
    for (int c = 0; c < n_chunks; ++c)
      if (parts[c].m > -INFINITY) S += parts[c].s * exp(parts[c].m - M);

  // Global top-k over n_chunks * ksel candidate keys, cached bests per lane.
  const int ncand = n_chunks * ksel;
  uint64_t best = 0ull;
  for (int i = lane; i < ncand; i += 64) {
    uint64_t k = parts[i / ksel].keys[i % ksel];
    best = k > best ? k : best;
  }
  for (int r = 0; r < ksel; ++r) {
    uint64_t win = wave_max_u64(best);
    if (lane == 0) s_sel[r] = win;
    if (win != 0ull && best == win) {
      uint64_t nb = 0ull;
      for (int i = lane; i < ncand; i += 64) {
        uint64_t k = parts[i / ksel].keys[i % ksel];
        if (k < win && k > nb) nb = k;
      }
      best = nb;
    }
  }
  __syncthreads();
  if (lane != 0) return;
  law->nonfinite = nf || !(greedy || (isfinite(S) && S > 0.0));
  if (law->nonfinite) {
    law->n = 0;
    return;
  }
  if (greedy) {
    law->n = 1;
    law->ids[0] = key_id(s_sel[0]);
    law->probs[0] = 1.0;
    return;
  }
  // Full-vocab probabilities of the top-k in (value desc, id asc) order.
  double pk[kMaxTopK];
  int idk[kMaxTopK];
  int nk = 0;
  for (int r = 0; r < ksel; ++r) {
    if (s_sel[r] == 0ull) break;
    idk[nk] = key_id(s_sel[r]);
    pk[nk] = exp((double)key_value(s_sel[r]) / temp - M) / S;
    ++nk;
  }
  // Nucleus in top-k order: keep while cumulative_before < top_p.
  int keep[kMaxTopK];
  double before = 0.0;
  for (int r = 0; r < nk; ++r) {
    keep[r] = (top_p > 0.0 && top_p < 1.0) ? (before < top_p) : 1;
    before += pk[r];
  }
  // Support sorted by id ascending (ids unique).
  int n = 0;
  int sid[kMaxTopK];
  double sp[kMaxTopK];
  for (int r = 0; r < nk; ++r) {
    if (!keep[r] || !(pk[r] > 0.0)) continue;
    int pos = n++;
    while (pos > 0 && sid[pos - 1] > idk[r]) {
      sid[pos] = sid[pos - 1];
      sp[pos] = sp[pos - 1];
      --pos;
    }
    sid[pos] = idk[r];
    sp[pos] = pk[r];
  }
  if (n == 0) {  // empty filter -> argmax one-hot (mtplx/sampling.py:197-199)
    law->n = 1;
    law->ids[0] = key_id(s_sel[0]);
    law->probs[0] = 1.0;
    return;
  }
  // filtered / total, then the SparseDistribution renormalisation.
  double t1 = np_sum_small(sp, n);
  for (int i = 0; i < n; ++i) sp[i] = sp[i] / t1;
  double t2 = np_sum_small(sp, n);
  law->n = n;
  for (int i = 0; i < n; ++i) {
    law->ids[i] = sid[i];
    law->probs[i] = sp[i] / t2;
  }
}

__device__ double law_prob(const RowLaw& L, int tok) {
  for (int i = 0; i < L.n; ++i)
    if (L.ids[i] == tok) return L.probs[i];
  return 0.0;
}

// Generator.choice(ids, p) given its uniform.
__device__ int law_choice(const int* ids, const double* p, int n, double u) {
  double cdf[2 * kMaxTopK];
  double run = 0.0;
  for (int i = 0; i < n; ++i) {
    run += p[i];
    cdf[i] = run;
  }
  const double last = cdf[n - 1];
  int idx = 0;
  for (int i = 0; i < n; ++i) {
    cdf[i] = cdf[i] / last;
    if (cdf[i] <= u) idx = i + 1;
  }
  if (idx > n - 1) idx = n - 1;
  return ids[idx];
}

// One wave per request b. Rows of request b: target rows [b*(K+1), b*(K+1)+K],
// draft rows [b*K, b*K+K-1] in the draft partial array.
__global__ __launch_bounds__(64) void accept_finish(const ChunkPart* __restrict__ tparts,
                                                    const ChunkPart* __restrict__ dparts, int n_chunks,
                                                    const int32_t* __restrict__ draft_ids,
                                                    const double* __restrict__ uniforms, int K, int ksel,
                                                    int greedy, double temp, double top_p,
                                                    int32_t* __restrict__ out_tokens,
                                                    int32_t* __restrict__ n_accepted,
                                                    double* __restrict__ accept_probs, int32_t* __restrict__ status) {
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  __shared__ RowLaw s_p, s_q;
  __shared__ uint64_t s_sel[kMaxTopK];
  __shared__ int s_done, s_ui, s_nacc;
  if (lane == 0) {
    s_done = 0;
    s_ui = 0;
    s_nacc = 0;
    status[b] = 0;
    for (int d = 0; d <= K; ++d) out_tokens[(size_t)b * (K + 1) + d] = -1;
    for (int d = 0; d < K; ++d) accept_probs[(size_t)b * K + d] = -1.0;
  }
  __syncthreads();
  const double* u = uniforms + (size_t)b * (K + 1);
  for (int d = 0; d <= K; ++d) {
    build_law(tparts + ((size_t)b * (K + 1) + d) * n_chunks, n_chunks, ksel, greedy, temp, top_p, &s_p, s_sel);
    __syncthreads();
    if (d < K) {
      build_law(dparts + ((size_t)b * K + d) * n_chunks, n_chunks, ksel, greedy, temp, top_p, &s_q, s_sel);
      __syncthreads();
    }
    if (lane == 0) {
      int32_t* ot = out_tokens + (size_t)b * (K + 1);
      if (s_p.nonfinite || (d < K && s_q.nonfinite)) {
        status[b] = 1;
        s_done = 1;
      } else if (d == K) {
        // all drafts accepted: bonus from row K
        ot[K] = greedy ? s_p.ids[0] : law_choice(s_p.ids, s_p.probs, s_p.n, u[s_ui++]);
        s_nacc = K;
        s_done = 1;
      } else {
        const int tok = draft_ids[(size_t)b * K + d];
        const double p = law_prob(s_p, tok);
        const double q = law_prob(s_q, tok);
        double a;
        bool acc;
        if (greedy) {
          acc = (tok == s_p.ids[0]);
          a = acc ? 1.0 : 0.0;
        } else {
          a = (q <= 0.0) ? (p > 0.0 ? 1.0 : 0.0) : fmin(1.0, p / q);
          acc = u[s_ui++] <= a;
        }
        accept_probs[(size_t)b * K + d] = a;
        if (acc) {
          ot[d] = tok;
        } else {
          int corr;
          if (greedy) {
            corr = s_p.ids[0];
          } else {
            // residual over the union of supports, ids ascending
            int rid[2 * kMaxTopK];
            double rp[2 * kMaxTopK];
            int n = 0, i = 0, j = 0;
            while (i < s_p.n || j < s_q.n) {
              int id;
              double pv = 0.0, qv = 0.0;
              if (j >= s_q.n || (i < s_p.n && s_p.ids[i] < s_q.ids[j])) {
                id = s_p.ids[i];
                pv = s_p.probs[i++];
              } else if (i >= s_p.n || s_q.ids[j] < s_p.ids[i]) {
                id = s_q.ids[j];
                qv = s_q.probs[j++];
              } else {
                id = s_p.ids[i];
                pv = s_p.probs[i++];
                qv = s_q.probs[j++];
              }
              const double r = fmax(pv - qv, 0.0);
              if (r > 0.0 && isfinite(r)) {
                rid[n] = id;
                rp[n] = r;
                ++n;
              }
            }
            const double tot = np_sum_small(rp, n);
            if (n == 0 || !(isfinite(tot) && tot > 0.0)) {
              corr = law_choice(s_p.ids, s_p.probs, s_p.n, u[s_ui++]);
            } else {
              for (int t = 0; t < n; ++t) rp[t] = rp[t] / tot;
              const double t2 = np_sum_small(rp, n);
              for (int t = 0; t < n; ++t) rp[t] = rp[t] / t2;
              corr = law_choice(rid, rp, n, u[s_ui++]);
            }
          }
          ot[d] = corr;
          s_nacc = d;
          s_done = 1;
        }
      }
    }
    __syncthreads();
    if (s_done) break;
  }
  if (lane == 0) n_accepted[b] = s_nacc;
}

// ---------------------------------------------------------------------------
// Wave-parallel law construction (n_chunks <= 64): the same law as build_law,
// the same operations in the same order wherever an order matters, but with
// every load issued up front and the per-candidate work spread over lanes:
//   lane c owns chunk c (max / sum-exp statistics, head of its sorted keys);
//   the top-k is a k-way merge of the chunks' sorted key lists (each chunk's
//   keys are its top-ksel in descending order), keys staged in LDS;
//   lane r owns candidate r (probability, nucleus prefix, id rank).
constexpr int kLawKeys = 768;   // staged candidate keys per wave (38 chunks x 20)

__device__ __forceinline__ void wave_sync_lds() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup"); }

__device__ void build_law_wave(const ChunkPart* parts, int n_chunks, int ksel, int greedy, double temp, double top_p,
                               RowLaw* law, uint64_t* s_keys) {
  const int lane = threadIdx.x & 63;
  const bool own = lane < n_chunks;
  double m = -INFINITY, sc = 0.0;
  int nf = 0;
  if (own) {
    m = parts[lane].m;
    sc = parts[lane].s;
    nf = parts[lane].nonfinite;
  }
  // Candidate keys: staged in LDS when they fit, else read in place.
  const int ncand = n_chunks * ksel;
  const uint64_t* kp;
  int kstride;
  if (ncand <= kLawKeys) {
    for (int i = lane; i < ncand; i += 64) {
      const int c = i / ksel;
      s_keys[i] = parts[c].keys[i - c * ksel];
    }
    wave_sync_lds();
    kp = s_keys;
    kstride = ksel;
  } else {
    kp = parts[0].keys;
    kstride = (int)(sizeof(ChunkPart) / sizeof(uint64_t));
  }
  // fp64 max / sum-exp combine, the sum in chunk order.
  const double M = wave_max_f64(m);
  nf = __any(nf) ? 1 : 0;
  double S = 0.0;
  if (!greedy) {
    const double term = (own && m > -INFINITY) ? sc * exp(m - M) : 0.0;
    for (int c = 0; c < n_chunks; ++c) S += rlf64(term, c);
  }
  // Top-k: k-way merge of the sorted chunk lists; head h0 and next h1 per lane.
  uint64_t h0 = 0ull, h1 = 0ull;
  int ptr = 0;
  if (own) {
    h0 = kp[(size_t)lane * kstride];
    h1 = ksel > 1 ? kp[(size_t)lane * kstride + 1] : 0ull;
  }
  uint64_t mysel = 0ull;
  for (int r = 0; r < ksel; ++r) {
    const uint64_t win = wave_max_u64(h0);
    if (lane == r) mysel = win;
    if (win == 0ull) break;   // uniform: every list is exhausted
    if (h0 == win) {
      h0 = h1;
      ++ptr;
      h1 = ptr + 1 < ksel ? kp[(size_t)lane * kstride + ptr + 1] : 0ull;
    }
  }
  const uint64_t sel0 = rl64(mysel, 0);
  const int nonfinite = nf || !(greedy || (isfinite(S) && S > 0.0));
  if (nonfinite || greedy) {
    if (lane == 0) {
      law->nonfinite = nonfinite;
      law->n = nonfinite ? 0 : 1;
      law->ids[0] = key_id(sel0);
      law->probs[0] = 1.0;
    }
    wave_sync_lds();
    return;
  }
  const bool has = lane < ksel && mysel != 0ull;
  const int nk = __popcll(__ballot(has));   // zero keys only trail
  const int myid = key_id(mysel);
  const double pk = has ? exp((double)key_value(mysel) / temp - M) / S : 0.0;
  // Nucleus in top-k order: keep while the cumulative sum before is < top_p.
  double run = 0.0, before = 0.0;
  for (int i = 0; i < nk; ++i) {
    if (lane == i) before = run;
    run += rlf64(pk, i);
  }
  const bool keep = has && ((top_p > 0.0 && top_p < 1.0) ? (before < top_p) : true) && pk > 0.0;
  const int n = __popcll(__ballot(keep));
  if (n == 0) {   // empty filter -> argmax one-hot (mtplx/sampling.py:197-199)
    if (lane == 0) {
      law->nonfinite = 0;
      law->n = 1;
      law->ids[0] = key_id(sel0);
      law->probs[0] = 1.0;
    }
    wave_sync_lds();
    return;
  }
  // Support ordered by id ascending (ids unique): rank among the kept.
  int rank = 0;
  for (int i = 0; i < nk; ++i) {
    const int idi = rli(myid, i);
    const int ki = rli(keep ? 1 : 0, i);
    rank += (ki && idi < myid) ? 1 : 0;
  }
  if (keep) {
    law->ids[rank] = myid;
    law->probs[rank] = pk;
  }
  wave_sync_lds();
  // filtered / total, then the SparseDistribution renormalisation.
  const double t1 = np_sum_wave(law->probs, n);
  if (lane < n) law->probs[lane] = law->probs[lane] / t1;
  wave_sync_lds();
  const double t2 = np_sum_wave(law->probs, n);
  if (lane < n) law->probs[lane] = law->probs[lane] / t2;
  if (lane == 0) {
    law->nonfinite = 0;
    law->n = n;
  }
  wave_sync_lds();
}

// Probability of tok under law L (0 if absent); whole wave, uniform result.
__device__ double law_prob_wave(const RowLaw& L, int tok) {
  const int lane = threadIdx.x & 63;
  const uint64_t hit = __ballot(lane < L.n && L.ids[lane] == tok);
  return hit ? L.probs[__ffsll((unsigned long long)hit) - 1] : 0.0;
}

// Generator.choice(ids, p) given its uniform (n <= 64, arrays in LDS); whole
// wave. cdf = cumsum(p) / cdf[-1] in order; idx = #{cdf <= u}, at most n-1.
__device__ int law_choice_wave(const int* ids, const double* p, int n, double u) {
  const int lane = threadIdx.x & 63;
  const double pv = lane < n ? p[lane] : 0.0;
  double run = 0.0, mine = 0.0;
  for (int i = 0; i < n; ++i) {
    run += rlf64(pv, i);
    if (lane == i) mine = run;
  }
  const double last = run;
  const int idx0 = __popcll(__ballot(lane < n && mine / last <= u));
  const int idx = idx0 > n - 1 ? n - 1 : idx0;
  return ids[idx];
}

// The accept loop of one request over its prebuilt laws (target rows 0..K,
// draft rows 0..K-1); run by one whole wave. s_rid / s_rp: LDS scratch of
// kMaxTopK entries for the residual law.
__device__ void accept_loop_wave(const RowLaw* tl, const RowLaw* dl, int b, int K, int greedy,
                                 const int32_t* __restrict__ draft_ids, const double* __restrict__ uniforms,
                                 int32_t* __restrict__ out_tokens, int32_t* __restrict__ n_accepted,
                                 double* __restrict__ accept_probs, int32_t* __restrict__ status, int* s_rid,
                                 double* s_rp) {
  const int lane = threadIdx.x & 63;
  int32_t* ot = out_tokens + (size_t)b * (K + 1);
  for (int d = lane; d <= K; d += 64) ot[d] = -1;
  for (int d = lane; d < K; d += 64) accept_probs[(size_t)b * K + d] = -1.0;
  const double* u = uniforms + (size_t)b * (K + 1);
  int ui = 0, nacc = 0, bad = 0;
  for (int d = 0; d <= K; ++d) {
    const RowLaw& P = tl[d];
    if (P.nonfinite || (d < K && dl[d].nonfinite)) {
      bad = 1;
      break;
    }
    if (d == K) {   // all drafts accepted: bonus from row K
      const int tok = greedy ? P.ids[0] : law_choice_wave(P.ids, P.probs, P.n, u[ui++]);
      if (lane == 0) ot[K] = tok;
      nacc = K;
      break;
    }
    const RowLaw& Qd = dl[d];
    const int tok = draft_ids[(size_t)b * K + d];
    const double p = law_prob_wave(P, tok);
    const double q = law_prob_wave(Qd, tok);
    double a;
    bool acc;
    if (greedy) {
      acc = (tok == P.ids[0]);
      a = acc ? 1.0 : 0.0;
    } else {
      a = (q <= 0.0) ? (p > 0.0 ? 1.0 : 0.0) : fmin(1.0, p / q);
      acc = u[ui++] <= a;
    }
    if (lane == 0) accept_probs[(size_t)b * K + d] = a;
    if (acc) {
      if (lane == 0) ot[d] = tok;
      continue;
    }
    int corr;
    if (greedy) {
      corr = P.ids[0];
    } else {
      // Residual max(p - q, 0) over the union of supports, ids ascending:
      // an id outside P's support has p = 0 and a zero residual, so the
      // positive residuals are P's entries in P's (ascending) order.
      int myid = 0;
      double r = 0.0;
      if (lane < P.n) {
        myid = P.ids[lane];
        double qv = 0.0;
        for (int j = 0; j < Qd.n; ++j)
          if (Qd.ids[j] == myid) qv = Qd.probs[j];
        r = fmax(P.probs[lane] - qv, 0.0);
      }
      const bool keep = lane < P.n && r > 0.0 && isfinite(r);
      const uint64_t km = __ballot(keep);
      const int n = __popcll(km);
      if (keep) {
        const int pos = __popcll(km & ((1ull << lane) - 1ull));
        s_rid[pos] = myid;
        s_rp[pos] = r;
      }
      wave_sync_lds();
      const double tot = np_sum_wave(s_rp, n);
      if (n == 0 || !(isfinite(tot) && tot > 0.0)) {
        corr = law_choice_wave(P.ids, P.probs, P.n, u[ui++]);
      } else {
        if (lane < n) s_rp[lane] = s_rp[lane] / tot;
        wave_sync_lds();
        const double t2 = np_sum_wave(s_rp, n);
        if (lane < n) s_rp[lane] = s_rp[lane] / t2;
        wave_sync_lds();
        corr = law_choice_wave(s_rid, s_rp, n, u[ui++]);
      }
    }
    if (lane == 0) ot[d] = corr;
    nacc = d;
    break;
  }
  if (lane == 0) {
    status[b] = bad;
    n_accepted[b] = nacc;
  }
}

// One workgroup per request, one wave per law (2K+1 of them, up to 16 waves,
// each wave taking every nwv-th law), then the accept loop on wave 0.
// Dynamic LDS: laws [2K+1] then candidate keys [nwv][kLawKeys].
__global__ __launch_bounds__(1024) void accept_laws(const ChunkPart* __restrict__ tparts,
                                                    const ChunkPart* __restrict__ dparts, int n_chunks,
                                                    const int32_t* __restrict__ draft_ids,
                                                    const double* __restrict__ uniforms, int K, int ksel,
                                                    int greedy, double temp, double top_p,
                                                    int32_t* __restrict__ out_tokens,
                                                    int32_t* __restrict__ n_accepted,
                                                    double* __restrict__ accept_probs, int32_t* __restrict__ status) {
  extern __shared__ __align__(16) unsigned char s_lds[];
  const int b = blockIdx.x;
  const int nwv = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6;
  const int nlaw = 2 * K + 1;
  RowLaw* laws = reinterpret_cast<RowLaw*>(s_lds);
  uint64_t* keys = reinterpret_cast<uint64_t*>(s_lds + (size_t)nlaw * sizeof(RowLaw)) + (size_t)wave * kLawKeys;
  for (int li = wave; li < nlaw; li += nwv) {
    const ChunkPart* rp = li <= K ? tparts + ((size_t)b * (K + 1) + li) * n_chunks
                                  : dparts + ((size_t)b * K + (li - K - 1)) * n_chunks;
    build_law_wave(rp, n_chunks, ksel, greedy, temp, top_p, &laws[li], keys);
  }
  __syncthreads();
  if (wave == 0) {   // the residual scratch reuses wave 0's key area
    double* s_rp = reinterpret_cast<double*>(keys);
    int* s_rid = reinterpret_cast<int*>(s_rp + kMaxTopK);
    accept_loop_wave(laws, laws + K + 1, b, K, greedy, draft_ids, uniforms, out_tokens, n_accepted, accept_probs,
                     status, s_rid, s_rp);
  }
}

static size_t accept_laws_lds(int K, int nwv) {
  return (size_t)(2 * K + 1) * sizeof(RowLaw) + (size_t)nwv * kLawKeys * sizeof(uint64_t);
}

// One wave per row: sparse law of the row (ids ascending) and optionally a draw.
__global__ __launch_bounds__(64) void row_laws(const ChunkPart* __restrict__ parts, int n_chunks, int ksel,
                                               int greedy, double temp, double top_p,
                                               const double* __restrict__ uniforms, int32_t* __restrict__ out_ids,
                                               double* __restrict__ out_probs, int32_t* __restrict__ out_count,
                                               int32_t* __restrict__ sampled, int32_t* __restrict__ status) {
  const int r = blockIdx.x;
  __shared__ RowLaw s_p;
  __shared__ uint64_t s_sel[kMaxTopK];
  __shared__ uint64_t s_keys[kLawKeys];
  if (n_chunks <= 64)
    build_law_wave(parts + (size_t)r * n_chunks, n_chunks, ksel, greedy, temp, top_p, &s_p, s_keys);
  else
    build_law(parts + (size_t)r * n_chunks, n_chunks, ksel, greedy, temp, top_p, &s_p, s_sel);
  __syncthreads();
  const int lane = threadIdx.x;
  if (lane == 0) {
    status[r] = s_p.nonfinite ? 1 : 0;
    if (out_count) out_count[r] = s_p.n;
  }
  if (out_ids)
    for (int i = lane; i < ksel; i += 64) {
      out_ids[(size_t)r * ksel + i] = i < s_p.n ? s_p.ids[i] : -1;
      out_probs[(size_t)r * ksel + i] = i < s_p.n ? s_p.probs[i] : 0.0;
    }
  if (sampled) {
    const int tok = s_p.nonfinite ? -1 : law_choice_wave(s_p.ids, s_p.probs, s_p.n, uniforms[r]);
    if (lane == 0) sampled[r] = tok;
  }
}

static int sampler_plan(int V, int top_k, double temperature, int* ksel, int* greedy, int* n_chunks,
                        const char* who) {
  if (V < 1) {
    set_error("%s: vocabulary size %d < 1", who, V);
    return MTP_ERR_ARG;
  }
  *greedy = !(temperature > 0.0);
  if (*greedy) {
    *ksel = 1;
  } else {
    if (top_k < 1 || top_k > kMaxTopK) {
      set_error("%s: top_k=%d unsupported on the GPU law (1..%d)", who, top_k, kMaxTopK);
      return MTP_ERR_UNSUPPORTED;
    }
    *ksel = top_k < V ? top_k : V;
  }
  *n_chunks = cdiv(V, kChunk);
  return MTP_OK;
}

}  // namespace mtp

using namespace mtp;

MTP_API size_t mtp_sampler_workspace_bytes(int rows, int V) {
  if (rows < 1 || V < 1) return 0;
  return (size_t)rows * cdiv(V, kChunk) * sizeof(ChunkPart);
}

MTP_API int mtp_spec_accept(const float* target_logits, const float* draft_logits, const int32_t* draft_ids,
                            const double* uniforms, int B, int K, int V, double temperature, int top_k,
                            double top_p, int32_t* out_tokens, int32_t* n_accepted, double* accept_probs, int32_t* status,
                            void* ws, size_t ws_bytes, void* stream) {
  const char* who = "mtp_spec_accept";
  int ksel, greedy, n_chunks;
  int rc = sampler_plan(V, top_k, temperature, &ksel, &greedy, &n_chunks, who);
  if (rc) return rc;
  if (B < 1 || K < 1 || !target_logits || !draft_logits || !draft_ids || !uniforms || !out_tokens ||
      !n_accepted || !accept_probs || !status) {
    set_error("%s: need B>=1, K>=1 and non-null buffers", who);
    return MTP_ERR_ARG;
  }
  const size_t need = mtp_sampler_workspace_bytes(B * (2 * K + 1), V);
  if (!ws || ws_bytes < need) {
    set_error("%s: workspace %zu B < required %zu B", who, ws_bytes, need);
    return MTP_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  ChunkPart* tparts = reinterpret_cast<ChunkPart*>(ws);
  ChunkPart* dparts = tparts + (size_t)B * (K + 1) * n_chunks;
  const double temp = greedy ? 1.0 : temperature;
  // target rows then draft rows, one launch (dparts follows tparts)
  hipLaunchKernelGGL(vocab_partials, dim3(n_chunks, B * (2 * K + 1)), dim3(kSampThreads), 0, st, target_logits,
                     draft_logits, B * (K + 1), (long long)V, V, n_chunks, temp, ksel, greedy, tparts);
  if ((rc = launch_check(who))) return rc;
  if (n_chunks <= 64) {
    const int nwv = 2 * K + 1 < 16 ? 2 * K + 1 : 16;
    const size_t lds = accept_laws_lds(K, nwv);
    if (lds > 160 * 1024) {
      set_error("%s: K=%d needs %zu B of LDS", who, K, lds);
      return MTP_ERR_UNSUPPORTED;
    }
    // A failure here surfaces as a launch error, checked below.
    if (lds > 65536) (void)hipFuncSetAttribute((const void*)accept_laws, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds);
    hipLaunchKernelGGL(accept_laws, dim3(B), dim3(nwv * 64), lds, st, tparts, dparts, n_chunks, draft_ids, uniforms,
                       K, ksel, greedy, temp, top_p, out_tokens, n_accepted, accept_probs, status);
  } else {
    hipLaunchKernelGGL(accept_finish, dim3(B), dim3(64), 0, st, tparts, dparts, n_chunks, draft_ids, uniforms, K,
                       ksel, greedy, temp, top_p, out_tokens, n_accepted, accept_probs, status);
  }
  return launch_check(who);
}

MTP_API int mtp_sample_rows(const float* logits, int rows, int V, double temperature, int top_k, double top_p,
                            const double* uniforms, int32_t* out_ids, double* out_probs, int32_t* out_count,
                            int32_t* sampled, int32_t* status, void* ws, size_t ws_bytes, void* stream) {
  const char* who = "mtp_sample_rows";
  int ksel, greedy, n_chunks;
  int rc = sampler_plan(V, top_k, temperature, &ksel, &greedy, &n_chunks, who);
  if (rc) return rc;
  if (rows < 1 || !logits || !status || (sampled && !uniforms) || (out_ids && !out_probs)) {
    set_error("%s: need rows>=1, logits, status, and uniforms when sampling", who);
    return MTP_ERR_ARG;
  }
  const size_t need = mtp_sampler_workspace_bytes(rows, V);
  if (!ws || ws_bytes < need) {
    set_error("%s: workspace %zu B < required %zu B", who, ws_bytes, need);
    return MTP_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  ChunkPart* parts = reinterpret_cast<ChunkPart*>(ws);
  const double temp = greedy ? 1.0 : temperature;
  hipLaunchKernelGGL(vocab_partials, dim3(n_chunks, rows), dim3(kSampThreads), 0, st, logits, logits, rows,
                     (long long)V, V, n_chunks, temp, ksel, greedy, parts);
  if ((rc = launch_check(who))) return rc;
  hipLaunchKernelGGL(row_laws, dim3(rows), dim3(64), 0, st, parts, n_chunks, ksel, greedy, temp, top_p,
                     uniforms, out_ids, out_probs, out_count, sampled, status);
  return launch_check(who);
}
