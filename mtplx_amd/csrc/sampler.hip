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
//  1. vocab_partials: grid (rows, chunks). Each 256-thread workgroup reads a
//     4096-logit chunk once (coalesced), and emits the chunk's fp64 max of
//     l/T, fp64 sum exp(l/T - max), a non-finite flag, and its top-k keys.
//     A key is (order-preserving float bits << 32) | ~id, so one u64 max is
//     "value desc, id asc". Top-k uses per-thread cached bests: each round
//     only the winning thread rescans its 16 registers.
//  2. accept_finish: one wave per request merges the chunks of its 2K+1 rows
//     (max/sum-exp combine in fixed chunk order, top-k over the candidates),
//     builds the sparse laws in fp64 and runs the accept loop on lane 0.
// Deterministic: fixed reduction trees, no float atomics.
#include "common.hpp"

#include <math.h>

namespace mtp {

constexpr int kSampThreads = 256;
constexpr int kEPT = 16;                          // logits per thread per chunk
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

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    uint64_t o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ double wave_max_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmax(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// grid: (n_chunks, rows). logits row r at logits + r * ld.
__global__ __launch_bounds__(kSampThreads) void vocab_partials(const float* __restrict__ logits, long long ld,
                                                               int V, int n_chunks, double temp, int ksel,
                                                               int greedy, ChunkPart* __restrict__ parts) {
  const int chunk = blockIdx.x;
  const int row = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const float* lr = logits + (size_t)row * ld;
  const int base = chunk * kChunk;

  float v[kEPT];
  int nonfinite = 0;
  double mloc = -INFINITY;
#pragma unroll
  for (int e = 0; e < kEPT; ++e) {
    const int id = base + e * kSampThreads + tid;
    float x = (id < V) ? lr[id] : -INFINITY;
    v[e] = x;
    if (id < V && (isnan(x) || (isinf(x) && x > 0))) nonfinite = 1;
    if (!greedy) mloc = fmax(mloc, (double)x / temp);
  }
  __shared__ double s_red[4];
  __shared__ uint64_t s_key[4];
  __shared__ int s_nf[4];

  double mchunk = -INFINITY, schunk = 0.0;
  if (!greedy) {
    double wm = wave_max_f64(mloc);
    if (lane == 0) s_red[wave] = wm;
    __syncthreads();
    mchunk = fmax(fmax(s_red[0], s_red[1]), fmax(s_red[2], s_red[3]));
    __syncthreads();
    double sl = 0.0;
    if (mchunk > -INFINITY) {
#pragma unroll
      for (int e = 0; e < kEPT; ++e) {
        const int id = base + e * kSampThreads + tid;
        if (id < V) sl += exp((double)v[e] / temp - mchunk);
      }
    }
    double ws = wave_sum_f64(sl);
    if (lane == 0) s_red[wave] = ws;
    __syncthreads();
    schunk = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
  }
  {
    int nf = __any(nonfinite) ? 1 : 0;
    if (lane == 0) s_nf[wave] = nf;
  }

  // Top-k selection with cached per-thread bests.
  uint64_t keys[kEPT];
#pragma unroll
  for (int e = 0; e < kEPT; ++e) {
    const int id = base + e * kSampThreads + tid;
    keys[e] = (id < V && !isnan(v[e])) ? make_key(v[e], id) : 0ull;
  }
  uint64_t best = 0ull;
#pragma unroll
  for (int e = 0; e < kEPT; ++e) best = keys[e] > best ? keys[e] : best;

  ChunkPart* out = parts + (size_t)row * n_chunks + chunk;
  for (int r = 0; r < ksel; ++r) {
    uint64_t wmax = wave_max_u64(best);
    __syncthreads();
    if (lane == 0) s_key[wave] = wmax;
    __syncthreads();
    uint64_t a = s_key[0] > s_key[1] ? s_key[0] : s_key[1];
    uint64_t b = s_key[2] > s_key[3] ? s_key[2] : s_key[3];
    uint64_t win = a > b ? a : b;
    if (tid == 0) out->keys[r] = win;
    if (win != 0ull && best == win) {
      uint64_t nb = 0ull;
#pragma unroll
      for (int e = 0; e < kEPT; ++e)
        if (keys[e] < win && keys[e] > nb) nb = keys[e];
      best = nb;
    }
  }
  if (tid == 0) {
    out->m = mchunk;
    out->s = schunk;
    out->nonfinite = s_nf[0] | s_nf[1] | s_nf[2] | s_nf[3];
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

// One wave per row: sparse law of the row (ids ascending) and optionally a draw.
__global__ __launch_bounds__(64) void row_laws(const ChunkPart* __restrict__ parts, int n_chunks, int ksel,
                                               int greedy, double temp, double top_p,
                                               const double* __restrict__ uniforms, int32_t* __restrict__ out_ids,
                                               double* __restrict__ out_probs, int32_t* __restrict__ out_count,
                                               int32_t* __restrict__ sampled, int32_t* __restrict__ status) {
  const int r = blockIdx.x;
  __shared__ RowLaw s_p;
  __shared__ uint64_t s_sel[kMaxTopK];
  build_law(parts + (size_t)r * n_chunks, n_chunks, ksel, greedy, temp, top_p, &s_p, s_sel);
  __syncthreads();
  if (threadIdx.x != 0) return;
  status[r] = s_p.nonfinite ? 1 : 0;
  if (out_count) out_count[r] = s_p.n;
  if (out_ids)
    for (int i = 0; i < ksel; ++i) {
      out_ids[(size_t)r * ksel + i] = i < s_p.n ? s_p.ids[i] : -1;
      out_probs[(size_t)r * ksel + i] = i < s_p.n ? s_p.probs[i] : 0.0;
    }
  if (sampled) sampled[r] = s_p.nonfinite ? -1 : law_choice(s_p.ids, s_p.probs, s_p.n, uniforms[r]);
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
  hipLaunchKernelGGL(vocab_partials, dim3(n_chunks, B * (K + 1)), dim3(kSampThreads), 0, st, target_logits,
                     (long long)V, V, n_chunks, temp, ksel, greedy, tparts);
  if ((rc = launch_check(who))) return rc;
  hipLaunchKernelGGL(vocab_partials, dim3(n_chunks, B * K), dim3(kSampThreads), 0, st, draft_logits, (long long)V,
                     V, n_chunks, temp, ksel, greedy, dparts);
  if ((rc = launch_check(who))) return rc;
  hipLaunchKernelGGL(accept_finish, dim3(B), dim3(64), 0, st, tparts, dparts, n_chunks, draft_ids, uniforms, K, ksel,
                     greedy, temp, top_p, out_tokens, n_accepted, accept_probs, status);
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
  hipLaunchKernelGGL(vocab_partials, dim3(n_chunks, rows), dim3(kSampThreads), 0, st, logits, (long long)V, V,
                     n_chunks, temp, ksel, greedy, parts);
  if ((rc = launch_check(who))) return rc;
  hipLaunchKernelGGL(row_laws, dim3(rows), dim3(64), 0, st, parts, n_chunks, ksel, greedy, temp, top_p,
                     uniforms, out_ids, out_probs, out_count, sampled, status);
  return launch_check(who);
}
