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
//     "value desc, id asc". Top-k: a radix select finds the k-th largest key
//     eight bits at a time (LDS digit histograms); the keys at or above it
//     are gathered and one wave sorts them (bitonic across its 64 lanes).
//     Target and draft rows go through one launch.
//  2. accept_laws: one workgroup per request, one wave per row law: merges
//     the row's chunks (max/sum-exp combine in fixed chunk order, top-k as a
//     k-way merge of the chunks' sorted lists), builds the sparse law in fp64
//     with the per-candidate work spread over lanes; wave 0 then runs the
//     accept loop. (Vocabularies over 64 chunks use accept_finish, one wave
//     per request building the laws in turn.)
// Laws whose support may exceed 64 ids (top_k = 0 or > 64: pure nucleus, or
// no truncation at all) take the wide path: one 1024-thread workgroup per row
// finds the support's cut by a radix descent over the logits' order-preserving
// bits (four 8-bit passes of per-digit counts and probability mass, the mass
// in 2^-62 fixed point so integer atomics keep it exact and order-free),
// resolves the cut inside the final tie group by id, and writes the support in
// id order with a block scan. The accept loop and draws then run over those
// laws with binary-searched lookups and block-wide scans.
// Penalties (presence/frequency, steering overlays) are sparse fp32 deltas
// added to the raw logits before any of this (mtp_apply_logit_deltas).
// Deterministic: fixed reduction trees, no float atomics.
#include "common.hpp"
#include "sampler_common.hpp"

#include <math.h>

#include <mutex>

namespace mtp {


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

  // Top-k by radix select: the ksel-th largest key K* of the chunk is found
  // eight bits at a time from the top (an LDS histogram of the next digit
  // among the keys that share the digits found so far; wave 0 finds the digit
  // holding rank r from the top), stopping as soon as the boundary digit's
  // keys all belong to the top ksel. Keys are distinct (the id is part of
  // the key), so the selected set is exact; its at most 64 keys are then
  // gathered in LDS and sorted descending by one wave (bitonic over 64 lanes).
  uint64_t keys[kEPT];
#pragma unroll
  for (int e = 0; e < kEPT; ++e) {
    const int id = base + e * kSampThreads + tid;
    keys[e] = (id < V && !isnan(v[e])) ? make_key(v[e], id) : 0ull;
  }
  __shared__ int s_hist[256];
  __shared__ uint64_t s_sel[kMaxTopK];
  __shared__ int s_rank, s_cnt, s_nsel, s_nvalid;
  __shared__ uint64_t s_prefix;
  {
    // valid keys: a ballot count per key slot, one LDS add per wave
    int nv = 0;
#pragma unroll
    for (int e = 0; e < kEPT; ++e) nv += __popcll(__ballot(keys[e] != 0ull));
    if (tid == 0) {
      s_nvalid = 0;
      s_nsel = 0;
    }
    __syncthreads();
    if (lane == 0 && nv) atomicAdd(&s_nvalid, nv);
  }
  __syncthreads();
  const int nvalid = s_nvalid;
  // Keys >= thr are selected; with at most ksel valid keys, all of them.
  uint64_t thr = 1ull;
  if (nvalid > ksel) {
    uint64_t prefix = 0ull;
    int rank = ksel;
    for (int shift = 56; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += kSampThreads) s_hist[i] = 0;
      __syncthreads();
      const uint64_t hi_mask = shift == 56 ? 0ull : ~((1ull << (shift + 8)) - 1ull);
#pragma unroll
      for (int e = 0; e < kEPT; ++e)
        if (keys[e] != 0ull && (keys[e] & hi_mask) == prefix) atomicAdd(&s_hist[(keys[e] >> shift) & 255u], 1);
      __syncthreads();
      if (wave == 0) {
        // lane l holds digits 255 - 4l .. 252 - 4l (descending); the
        // inclusive prefix over lanes counts the keys at or above each block
        int c[4], tot = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          c[j] = s_hist[255 - 4 * lane - j];
          tot += c[j];
        }
        int incl = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(incl, o, 64);
          if (lane >= o) incl += y;
        }
        const int above = incl - tot;
        if (above < rank && rank <= incl) {   // exactly one lane holds the rank
          int d = 0, a = above, cnt = 0;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (cnt == 0 && a + c[j] >= rank) {
              d = 255 - 4 * lane - j;
              cnt = c[j];
            } else if (cnt == 0) {
              a += c[j];
            }
          }
          s_prefix = prefix | ((uint64_t)d << shift);
          s_rank = rank - a;
          s_cnt = cnt;
        }
      }
      __syncthreads();
      // (wave 0 rewrites these only after the next pass's two barriers,
      // which every thread reaches after reading them here)
      prefix = s_prefix;
      rank = s_rank;
      const int cnt = s_cnt;
      if (cnt == rank || shift == 0) {
        // every key under the boundary prefix is in (cnt == rank), or the
        // prefix is the full key K* itself: select the keys >= prefix
        thr = prefix;
        break;
      }
    }
  }
  // Gather the selected keys (at most ksel <= 64), then sort them descending.
#pragma unroll
  for (int e = 0; e < kEPT; ++e)
    if (keys[e] != 0ull && keys[e] >= thr) {
      const int at = atomicAdd(&s_nsel, 1);
      if (at < kMaxTopK) s_sel[at] = keys[e];   // at most ksel <= kMaxTopK by construction
    }
  __syncthreads();
  if (wave != 0) return;
  ChunkPart* out = parts + (size_t)row * n_chunks + chunk;
  const int nsel = s_nsel < kMaxTopK ? s_nsel : kMaxTopK;
  const uint64_t kv = wave_sort_desc_u64(lane < nsel ? s_sel[lane] : 0ull);
  if (lane < ksel) out->keys[lane] = kv;
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
__device__ __forceinline__ double np_sum_wave(const double* a, int n) {
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

// Rows of request b: target rows t_off[b] .. t_off[b] + K_b, draft rows (and
// draft ids) d_off[b] .. d_off[b] + K_b - 1, K_b = k_lens[b]; all null: the
// uniform batch (K_b = K, t_off = b (K + 1), d_off = b K). Outputs keep the
// uniform strides ([B, K+1] tokens, [B, K] accept probabilities, K = the
// largest K_b).
struct AcceptRows {
  const int32_t* t_off;
  const int32_t* d_off;
  const int32_t* k_lens;
  int nt;   // target rows in all (the draft rows follow them)
  int nd;   // draft rows (and draft ids) in all
};
__device__ __forceinline__ int req_k(const AcceptRows& r, int b, int K) { return r.k_lens ? r.k_lens[b] : K; }
__device__ __forceinline__ int req_t(const AcceptRows& r, int b, int K) { return r.t_off ? r.t_off[b] : b * (K + 1); }
__device__ __forceinline__ int req_d(const AcceptRows& r, int b, int K) { return r.d_off ? r.d_off[b] : b * K; }

// Whether request b's rows lie inside the buffers: 0 <= K_b <= K, its K_b + 1
// target rows inside the nt target rows and its K_b draft rows inside the nd
// draft rows. The offsets of a ragged batch are device data the host never
// reads, so every accept kernel checks them before touching a row: a request
// that fails gets status 2, tokens and accept probabilities -1 and no accepted
// drafts, and nothing of it is read or written past its own output rows.
__device__ __forceinline__ bool req_in_bounds(const AcceptRows& r, int Kb, int tb, int db, int K) {
  return Kb >= 0 && Kb <= K && tb >= 0 && (long long)tb + Kb < (long long)r.nt && db >= 0 &&
         (long long)db + Kb <= (long long)r.nd;
}

// Outputs of a request whose rows fail req_in_bounds (one thread writes them).
__device__ __forceinline__ void req_reject(int b, int K, int32_t* out_tokens, int32_t* n_accepted,
                                           double* accept_probs, int32_t* status) {
  for (int d = 0; d <= K; ++d) out_tokens[(size_t)b * (K + 1) + d] = -1;
  for (int d = 0; d < K; ++d) accept_probs[(size_t)b * K + d] = -1.0;
  n_accepted[b] = 0;
  status[b] = 2;
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
                                                    double* __restrict__ accept_probs, int32_t* __restrict__ status,
                                                    AcceptRows rr) {
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int Kb = req_k(rr, b, K), tb = req_t(rr, b, K), db = req_d(rr, b, K);
  if (!req_in_bounds(rr, Kb, tb, db, K)) {   // uniform over the block
    if (lane == 0) req_reject(b, K, out_tokens, n_accepted, accept_probs, status);
    return;
  }
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
  for (int d = 0; d <= Kb; ++d) {
    build_law(tparts + ((size_t)tb + d) * n_chunks, n_chunks, ksel, greedy, temp, top_p, &s_p, s_sel);
    __syncthreads();
    if (d < Kb) {
      build_law(dparts + ((size_t)db + d) * n_chunks, n_chunks, ksel, greedy, temp, top_p, &s_q, s_sel);
      __syncthreads();
    }
    if (lane == 0) {
      int32_t* ot = out_tokens + (size_t)b * (K + 1);
      if (s_p.nonfinite || (d < Kb && s_q.nonfinite)) {
        status[b] = 1;
        s_done = 1;
      } else if (d == Kb) {
        // all drafts accepted: bonus from row K_b
        ot[Kb] = greedy ? s_p.ids[0] : law_choice(s_p.ids, s_p.probs, s_p.n, u[s_ui++]);
        s_nacc = Kb;
        s_done = 1;
      } else {
        const int tok = draft_ids[(size_t)db + d];
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

// Top-k of the chunks' sorted key lists (list c at kp + c * kstride; lane c
// holds list c's head h0 and next h1): k rounds of wave maxima. Returns the
// lane's winner (lane r: the r-th largest key). Templated on the pointer so
// that the staged case reads LDS (ds loads), not generic memory.
template <typename KeyPtr>
__device__ __forceinline__ uint64_t merge_sorted_lists(KeyPtr kp, int kstride, bool own, int ksel) {
  const int lane = threadIdx.x & 63;
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
  return mysel;
}

__device__ __forceinline__ void build_law_wave(const ChunkPart* parts, int n_chunks, int ksel, int greedy,
                                               double temp, double top_p, RowLaw* law, uint64_t* s_keys) {
  const int lane = threadIdx.x & 63;
  const bool own = lane < n_chunks;
  double m = -INFINITY, sc = 0.0;
  int nf = 0;
  if (own) {
    m = parts[lane].m;
    sc = parts[lane].s;
    nf = parts[lane].nonfinite;
  }
  // Candidate keys: staged in LDS when they fit (their loads issued with the
  // statistics' loads above, one round trip for both), else read in place.
  const int ncand = n_chunks * ksel;
  const bool staged = ncand <= kLawKeys;
  if (staged) {
    // All of the lane's loads in flight at once, then the LDS stores. Key i
    // is key i % ksel of chunk i / ksel; (c, r) follow i in steps of 64.
    constexpr int kPer = kLawKeys / 64;
    uint64_t kv[kPer];
    int c = lane / ksel, r = lane - (lane / ksel) * ksel;
    const int dc = 64 / ksel, dr = 64 - (64 / ksel) * ksel;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      kv[j] = lane + 64 * j < ncand ? parts[c].keys[r] : 0ull;
      c += dc;
      r += dr;
      if (r >= ksel) {
        r -= ksel;
        ++c;
      }
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (lane + 64 * j < ncand) s_keys[lane + 64 * j] = kv[j];
    wave_sync_lds();
  }
  // fp64 max / sum-exp combine, the sum in chunk order.
  const double M = wave_max_f64(m);
  nf = __any(nf) ? 1 : 0;
  double S = 0.0;
  if (!greedy) {
    const double term = (own && m > -INFINITY) ? sc * exp(m - M) : 0.0;
    for (int c = 0; c < n_chunks; ++c) S += rlf64(term, c);
  }
  // The k-way merge of the sorted chunk lists.
  const uint64_t mysel = staged ? merge_sorted_lists(s_keys, ksel, own, ksel)
                                : merge_sorted_lists(parts[0].keys, (int)(sizeof(ChunkPart) / sizeof(uint64_t)), own,
                                                     ksel);
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
__device__ __forceinline__ double law_prob_wave(const RowLaw& L, int tok) {
  const int lane = threadIdx.x & 63;
  const uint64_t hit = __ballot(lane < L.n && L.ids[lane] == tok);
  return hit ? L.probs[__ffsll((unsigned long long)hit) - 1] : 0.0;
}

// Generator.choice(ids, p) given its uniform (n <= 64, arrays in LDS); whole
// wave. cdf = cumsum(p) / cdf[-1] in order; idx = #{cdf <= u}, at most n-1.
__device__ __forceinline__ int law_choice_wave(const int* ids, const double* p, int n, double u) {
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
// Kb: this request's depth; K: the row stride of the outputs; db: the index
// of its first draft id.
// tok_l / u_l: lane d holds draft token d and uniform d of the request
// (loaded at kernel start, so the chain reads registers, not memory).
__device__ __forceinline__ void accept_loop_wave(const RowLaw* tl, const RowLaw* dl, int b, int Kb, int K, int greedy,
                                 int tok_l, double u_l,
                                 int32_t* __restrict__ out_tokens, int32_t* __restrict__ n_accepted,
                                 double* __restrict__ accept_probs, int32_t* __restrict__ status, int* s_rid,
                                 double* s_rp) {
  const int lane = threadIdx.x & 63;
  int32_t* ot = out_tokens + (size_t)b * (K + 1);
  for (int d = lane; d <= K; d += 64) ot[d] = -1;
  for (int d = lane; d < K; d += 64) accept_probs[(size_t)b * K + d] = -1.0;
  int ui = 0, nacc = 0, bad = 0;
  for (int d = 0; d <= Kb; ++d) {
    const RowLaw& P = tl[d];
    if (P.nonfinite || (d < Kb && dl[d].nonfinite)) {
      bad = 1;
      break;
    }
    if (d == Kb) {   // all drafts accepted: bonus from row K_b
      const int tok = greedy ? P.ids[0] : law_choice_wave(P.ids, P.probs, P.n, rlf64(u_l, ui++));
      if (lane == 0) ot[Kb] = tok;
      nacc = Kb;
      break;
    }
    const RowLaw& Qd = dl[d];
    const int tok = rli(tok_l, d);
    const double p = law_prob_wave(P, tok);
    const double q = law_prob_wave(Qd, tok);
    double a;
    bool acc;
    if (greedy) {
      acc = (tok == P.ids[0]);
      a = acc ? 1.0 : 0.0;
    } else {
      a = (q <= 0.0) ? (p > 0.0 ? 1.0 : 0.0) : fmin(1.0, p / q);
      acc = rlf64(u_l, ui++) <= a;
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
      // q of each of P's ids: lane j holds Q's entry j; a ballot per id of P
      // finds its lane (ids are unique in a law), no LDS scan per lane.
      const int pn = __builtin_amdgcn_readfirstlane(P.n);
      const int qid = lane < Qd.n ? Qd.ids[lane] : -1;
      const double qp = lane < Qd.n ? Qd.probs[lane] : 0.0;
      const int myid = lane < pn ? P.ids[lane] : -2;
      double qv = 0.0;
      for (int i = 0; i < pn; ++i) {
        const uint64_t hit = __ballot(qid == rli(myid, i));
        const double v = hit ? rlf64(qp, __ffsll((unsigned long long)hit) - 1) : 0.0;
        if (lane == i) qv = v;
      }
      double r = 0.0;
      if (lane < pn) r = fmax(P.probs[lane] - qv, 0.0);
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
        corr = law_choice_wave(P.ids, P.probs, P.n, rlf64(u_l, ui++));
      } else {
        if (lane < n) s_rp[lane] = s_rp[lane] / tot;
        wave_sync_lds();
        const double t2 = np_sum_wave(s_rp, n);
        if (lane < n) s_rp[lane] = s_rp[lane] / t2;
        wave_sync_lds();
        corr = law_choice_wave(s_rid, s_rp, n, rlf64(u_l, ui++));
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
__global__ __launch_bounds__(1024) void accept_laws(const ChunkPart* __restrict__ tparts, int t_chunks,
                                                    const ChunkPart* __restrict__ dparts, int n_chunks,
                                                    const int32_t* __restrict__ draft_ids,
                                                    const double* __restrict__ uniforms, int K, int ksel,
                                                    int greedy, double temp, double top_p,
                                                    int32_t* __restrict__ out_tokens,
                                                    int32_t* __restrict__ n_accepted,
                                                    double* __restrict__ accept_probs, int32_t* __restrict__ status,
                                                    AcceptRows rr) {
  extern __shared__ __align__(16) unsigned char s_lds[];
  const int b = blockIdx.x;
  const int nwv = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6;
  const int Kb = req_k(rr, b, K), tb = req_t(rr, b, K), db = req_d(rr, b, K);
  if (!req_in_bounds(rr, Kb, tb, db, K)) {   // uniform over the block
    if (threadIdx.x == 0) req_reject(b, K, out_tokens, n_accepted, accept_probs, status);
    return;
  }
  // The accept chain's inputs, loaded now (K + 1 <= 64: the host's bound).
  double u_l = 0.0;
  int tok_l = -1;
  if (wave == 0) {
    const int lane = threadIdx.x & 63;
    if (lane <= Kb) u_l = uniforms[(size_t)b * (K + 1) + lane];
    if (lane < Kb) tok_l = draft_ids[(size_t)db + lane];
  }
  const int nlaw = 2 * Kb + 1;
  RowLaw* laws = reinterpret_cast<RowLaw*>(s_lds);   // sized for 2K + 1 laws
  uint64_t* keys = reinterpret_cast<uint64_t*>(s_lds + (size_t)(2 * K + 1) * sizeof(RowLaw)) + (size_t)wave * kLawKeys;
  for (int li = wave; li < nlaw; li += nwv) {
    const ChunkPart* rp = li <= Kb ? tparts + ((size_t)tb + li) * t_chunks
                                   : dparts + ((size_t)db + (li - Kb - 1)) * n_chunks;
    build_law_wave(rp, li <= Kb ? t_chunks : n_chunks, ksel, greedy, temp, top_p, &laws[li], keys);
  }
  __syncthreads();
  if (wave == 0) {   // the residual scratch reuses wave 0's key area
    double* s_rp = reinterpret_cast<double*>(keys);
    int* s_rid = reinterpret_cast<int*>(s_rp + kMaxTopK);
    accept_loop_wave(laws, laws + Kb + 1, b, Kb, K, greedy, tok_l, u_l, out_tokens, n_accepted, accept_probs,
                     status, s_rid, s_rp);
  }
}

static size_t accept_laws_lds(int K, int nwv) {
  return (size_t)(2 * K + 1) * sizeof(RowLaw) + (size_t)nwv * kLawKeys * sizeof(uint64_t);
}

// One wave per row: sparse law of the row (ids ascending) and optionally a draw.
// out_ids / out_probs rows are ld_out apart; slots past the support hold -1 / 0.
__global__ __launch_bounds__(64) void row_laws(const ChunkPart* __restrict__ parts, int n_chunks, int ksel,
                                               int greedy, double temp, double top_p,
                                               const double* __restrict__ uniforms, int32_t* __restrict__ out_ids,
                                               double* __restrict__ out_probs, int ld_out,
                                               int32_t* __restrict__ out_count,
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
    for (int i = lane; i < ld_out; i += 64) {
      out_ids[(size_t)r * ld_out + i] = i < s_p.n ? s_p.ids[i] : -1;
      out_probs[(size_t)r * ld_out + i] = i < s_p.n ? s_p.probs[i] : 0.0;
    }
  if (sampled) {
    const int tok = s_p.nonfinite ? -1 : law_choice_wave(s_p.ids, s_p.probs, s_p.n, uniforms[r]);
    if (lane == 0) sampled[r] = tok;
  }
}

// k_eff: the top-k bound of mtplx/sampling.py:176 (0 < top_k < V, else no
// bound = V). Laws with k_eff <= 64 take the narrow path (ksel = k_eff keys
// per chunk); wider ones the wide path (ksel = 1: the argmax only).
struct SamplerPlan {
  int ksel, greedy, n_chunks, k_eff, wide;
};

static int sampler_plan(int V, int top_k, double temperature, SamplerPlan* pl, const char* who) {
  if (V < 1) {
    set_error("%s: vocabulary size %d < 1", who, V);
    return MTP_ERR_ARG;
  }
  if (top_k < 0) {
    set_error("%s: top_k=%d < 0", who, top_k);
    return MTP_ERR_ARG;
  }
  pl->greedy = !(temperature > 0.0);
  pl->k_eff = (top_k > 0 && top_k < V) ? top_k : V;
  pl->wide = !pl->greedy && pl->k_eff > kMaxTopK;
  pl->ksel = pl->greedy ? 1 : (pl->wide ? 1 : pl->k_eff);
  pl->n_chunks = cdiv(V, kChunk);
  return MTP_OK;
}


// ---------------------------------------------------------------------------
// Wide laws (support bound above 64 ids). Per-row storage in the workspace:
// a 16-byte header {n, nonfinite}, ids int32 [V], then probs fp64 [V].
constexpr int kWideThreads = 1024;
constexpr int kWideWaves = kWideThreads / 64;
constexpr double kFix62 = 4611686018427387904.0;   // 2^62: fixed-point probability mass

struct WideHdr {
  int n;
  int nonfinite;
  int pad[2];
};

__host__ __device__ inline size_t wide_ids_off() { return 16; }
__host__ __device__ inline size_t wide_probs_off(int V) { return (16 + 4 * (size_t)V + 15) & ~(size_t)15; }
__host__ __device__ inline size_t wide_row_bytes(int V) { return (wide_probs_off(V) + 8 * (size_t)V + 255) & ~(size_t)255; }

struct WideLaw {
  const int* ids;
  const double* probs;
  int n;
  int nonfinite;
};

__device__ __forceinline__ WideLaw wide_law(const unsigned char* base, size_t row_bytes, int V, int row) {
  const unsigned char* r = base + (size_t)row * row_bytes;
  const WideHdr* h = reinterpret_cast<const WideHdr*>(r);
  WideLaw L;
  L.ids = reinterpret_cast<const int*>(r + wide_ids_off());
  L.probs = reinterpret_cast<const double*>(r + wide_probs_off(V));
  L.n = h->n;
  L.nonfinite = h->nonfinite;
  return L;
}

__device__ __forceinline__ float ordered_value(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// Exclusive block scan of a 0/1 flag; *total receives the block's count.
// s_w: [kWideWaves + 1] LDS words. All threads must call it.
__device__ __forceinline__ int block_scan_flag(bool f, uint32_t* s_w, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t m = __ballot(f);
  const int in_wave = __popcll(m & ((1ull << lane) - 1ull));
  if (lane == 0) s_w[wave] = (uint32_t)__popcll(m);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int w = 0; w < kWideWaves; ++w) {
      const uint32_t t = s_w[w];
      s_w[w] = run;
      run += t;
    }
    s_w[kWideWaves] = run;
  }
  __syncthreads();
  const int r = (int)s_w[wave] + in_wave;
  *total = (int)s_w[kWideWaves];
  __syncthreads();
  return r;
}

// Deterministic block sum of a[0..n): each thread adds its strided elements
// in order, then the fixed wave tree, then the waves in order. Uniform result.
__device__ double block_sum_f64(const double* a, int n, double* s_d) {
  double v = 0.0;
  for (int i = threadIdx.x; i < n; i += kWideThreads) v += a[i];
  v = wave_sum_f64(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) s_d[wave] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < kWideWaves; ++w) t += s_d[w];
  __syncthreads();
  return t;
}

// Inclusive prefix of tile element x within the block (fixed order): wave
// Hillis-Steele scan, then the waves' totals in order. *tile_tot: the tile's
// sum (waves in order).
__device__ double block_incl_scan_f64(double x, double* s_d, double* tile_tot) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int o = 1; o < 64; o <<= 1) {
    const double y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_d[wave] = x;
  __syncthreads();
  double before = 0.0, tot = 0.0;
  for (int w = 0; w < kWideWaves; ++w) {
    if (w == wave) before = tot;
    tot += s_d[w];
  }
  __syncthreads();
  *tile_tot = tot;
  return before + x;
}

// Generator.choice(ids, p) given its uniform, for n up to the vocabulary:
// cdf = cumsum(p) (a fixed-order block scan), idx = #{cdf / cdf[n-1] <= u},
// at most n - 1. Two passes recompute the same cdf (the first only for its
// last value). Uniform result.
__device__ int block_choice(const int* ids, const double* p, int n, double u, double* s_d, double* s_last,
                            uint32_t* s_w) {
  double carry = 0.0;
  for (int base = 0; base < n; base += kWideThreads) {
    const int i = base + threadIdx.x;
    double tt;
    const double c = carry + block_incl_scan_f64(i < n ? p[i] : 0.0, s_d, &tt);
    if (i == n - 1) *s_last = c;
    carry += tt;
  }
  __syncthreads();
  const double last = *s_last;
  carry = 0.0;
  int count = 0;
  for (int base = 0; base < n; base += kWideThreads) {
    const int i = base + threadIdx.x;
    double tt;
    const double c = carry + block_incl_scan_f64(i < n ? p[i] : 0.0, s_d, &tt);
    carry += tt;
    int t;
    block_scan_flag(i < n && c / last <= u, s_w, &t);
    count += t;
  }
  const int idx = count > n - 1 ? n - 1 : count;
  return ids[idx];
}

// Probability of tok under a law with ids ascending (0 if absent).
__device__ __forceinline__ double wide_prob(const WideLaw& L, int tok) {
  int lo = 0, hi = L.n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (L.ids[mid] < tok) lo = mid + 1; else hi = mid;
  }
  return (lo < L.n && L.ids[lo] == tok) ? L.probs[lo] : 0.0;
}

// One workgroup per row: the sparse law p = renorm(topk(k_eff) ∩ nucleus(top_p))
// of the full-vocabulary softmax of logits/T (the narrow path's formula for
// each probability), ids ascending. Rows below nrows1 come from logits.
__global__ __launch_bounds__(kWideThreads) void wide_law_kernel(const float* __restrict__ logits,
                                                                const float* __restrict__ logits2, int nrows1,
                                                                long long ld, int V,
                                                                const ChunkPart* __restrict__ parts, int n_chunks,
                                                                double temp, int k_eff, double top_p,
                                                                unsigned char* __restrict__ lawbuf, size_t row_bytes) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const float* lr = row < nrows1 ? logits + (size_t)row * ld : logits2 + (size_t)(row - nrows1) * ld;
  const ChunkPart* pp = parts + (size_t)row * n_chunks;
  unsigned char* rb = lawbuf + (size_t)row * row_bytes;
  WideHdr* hdr = reinterpret_cast<WideHdr*>(rb);
  int* ids = reinterpret_cast<int*>(rb + wide_ids_off());
  double* probs = reinterpret_cast<double*>(rb + wide_probs_off(V));

  __shared__ uint32_t h_cnt[256];
  __shared__ unsigned long long h_mass[256];
  __shared__ double s_M, s_S;
  __shared__ int s_nf, s_all, s_argmax;
  __shared__ uint32_t s_prefix, s_cabove, s_w[kWideWaves + 1];
  __shared__ unsigned long long s_mabove;
  __shared__ double s_d[kWideWaves];

  if (tid == 0) {   // fp64 max / sum-exp combine in fixed chunk order (as build_law)
    double M = -INFINITY;
    int nf = 0;
    uint64_t best = 0ull;
    for (int c = 0; c < n_chunks; ++c) {
      M = fmax(M, pp[c].m);
      nf |= pp[c].nonfinite;
      best = pp[c].keys[0] > best ? pp[c].keys[0] : best;
    }
    double S = 0.0;
    for (int c = 0; c < n_chunks; ++c)
      if (pp[c].m > -INFINITY) S += pp[c].s * exp(pp[c].m - M);
    s_M = M;
    s_S = S;
    s_nf = nf || !(isfinite(S) && S > 0.0);
    s_argmax = key_id(best);
    s_prefix = 0u;
    s_cabove = 0u;
    s_mabove = 0ull;
    s_all = 0;
  }
  __syncthreads();
  if (s_nf) {
    if (tid == 0) {
      hdr->n = 0;
      hdr->nonfinite = 1;
    }
    return;
  }
  const double M = s_M, S = s_S;
  const bool nuc = top_p > 0.0 && top_p < 1.0;
  const unsigned long long TP = nuc ? (unsigned long long)(top_p * kFix62) : ~0ull;

  // Radix descent: after pass j the top 8(j+1) bits of the cut's key are
  // fixed, with the count and mass of everything ordered before its bin.
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (tid < 256) {
      h_cnt[tid] = 0u;
      h_mass[tid] = 0ull;
    }
    __syncthreads();
    const uint32_t prefix = s_prefix;
    for (int id = tid; id < V; id += kWideThreads) {
      const float l = lr[id];
      const uint32_t key = ordered_bits(l);
      if (pass == 0 || (key >> (shift + 8)) == prefix) {
        const int dgt = (key >> shift) & 255;
        atomicAdd(&h_cnt[dgt], 1u);
        const double pv = exp((double)l / temp - M) / S;
        const unsigned long long P = (unsigned long long)(pv * kFix62);
        if (P) atomicAdd(&h_mass[dgt], P);
      }
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t ca = s_cabove;
      unsigned long long ma = s_mabove;
      int sel = -1;
      for (int dgt = 255; dgt >= 0; --dgt) {
        const uint32_t c = h_cnt[dgt];
        if (!c) continue;
        const uint32_t ac = ca + c;
        const unsigned long long am = ma + h_mass[dgt];
        // The position after this bin is excluded (top-k full or nucleus
        // mass reached): the cut lies in this bin.
        if ((int)ac >= k_eff || (nuc && am >= TP)) {
          sel = dgt;
          break;
        }
        ca = ac;
        ma = am;
      }
      if (sel < 0) {
        s_all = 1;   // only in pass 0: every id is inside the cut
      } else {
        s_prefix = (prefix << 8) | (uint32_t)sel;
        s_cabove = ca;
        s_mabove = ma;
      }
    }
    __syncthreads();
    if (s_all) break;
  }

  // Inside the tie group (every logit equal to the cut's): members in id
  // order, each of the same fixed-point mass Pt; the first is included.
  const uint32_t tau = s_prefix;
  int t_cut = 0x7fffffff;
  if (!s_all) {
    const double pt = exp((double)ordered_value(tau) / temp - M) / S;
    const unsigned long long Pt = (unsigned long long)(pt * kFix62);
    const long long t_k = (long long)k_eff - (long long)s_cabove;
    long long t_n = 0x7fffffff;
    if (nuc && Pt) t_n = (long long)((TP - s_mabove + Pt - 1ull) / Pt);
    const long long t = t_k < t_n ? t_k : t_n;
    t_cut = (int)(t < 0x7fffffff ? t : 0x7fffffff);
  }

  // Support in id order: key above the cut, or a tie member before t_cut; p > 0.
  int out = 0, grank = 0;
  for (int base = 0; base < V; base += kWideThreads) {
    const int id = base + tid;
    const bool valid = id < V;
    const float l = valid ? lr[id] : -INFINITY;
    const uint32_t key = ordered_bits(l);
    const double pv = valid ? exp((double)l / temp - M) / S : 0.0;
    const bool isg = !s_all && valid && key == tau;
    int gtot;
    const int gr = grank + block_scan_flag(isg, s_w, &gtot);
    grank += gtot;
    const bool keep = valid && pv > 0.0 && (s_all || key > tau || (isg && gr < t_cut));
    int ktot;
    const int pos = out + block_scan_flag(keep, s_w, &ktot);
    if (keep) {
      ids[pos] = id;
      probs[pos] = pv;
    }
    out += ktot;
  }
  __syncthreads();
  if (out == 0) {   // empty filter -> argmax one-hot (mtplx/sampling.py:197-199)
    if (tid == 0) {
      ids[0] = s_argmax;
      probs[0] = 1.0;
      hdr->n = 1;
      hdr->nonfinite = 0;
    }
    return;
  }
  // filtered / total, then the SparseDistribution renormalisation.
  const double t1 = block_sum_f64(probs, out, s_d);
  for (int i = tid; i < out; i += kWideThreads) probs[i] = probs[i] / t1;
  __syncthreads();
  const double t2 = block_sum_f64(probs, out, s_d);
  for (int i = tid; i < out; i += kWideThreads) probs[i] = probs[i] / t2;
  if (tid == 0) {
    hdr->n = out;
    hdr->nonfinite = 0;
  }
}

// The accept loop of one request over wide laws: target rows b*(K+1)+d,
// draft rows B*(K+1) + b*K + d; scratch: this request's residual ids/probs.
__global__ __launch_bounds__(kWideThreads) void wide_accept_kernel(
    const unsigned char* __restrict__ lawbuf, size_t row_bytes, int V, int B, int K,
    const int32_t* __restrict__ draft_ids, const double* __restrict__ uniforms, int32_t* __restrict__ out_tokens,
    int32_t* __restrict__ n_accepted, double* __restrict__ accept_probs, int32_t* __restrict__ status,
    unsigned char* __restrict__ scratch, AcceptRows rr) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int Kb = req_k(rr, b, K), tb = req_t(rr, b, K), db = req_d(rr, b, K);
  if (!req_in_bounds(rr, Kb, tb, db, K)) {   // uniform over the block
    if (tid == 0) req_reject(b, K, out_tokens, n_accepted, accept_probs, status);
    return;
  }
  const int nt = rr.t_off ? rr.nt : B * (K + 1);
  __shared__ double s_d[kWideWaves];
  __shared__ double s_last, s_p, s_q;
  __shared__ uint32_t s_w[kWideWaves + 1];
  int* rid = reinterpret_cast<int*>(scratch + (size_t)b * wide_row_bytes(V) + wide_ids_off());
  double* rp = reinterpret_cast<double*>(scratch + (size_t)b * wide_row_bytes(V) + wide_probs_off(V));
  int32_t* ot = out_tokens + (size_t)b * (K + 1);
  for (int d = tid; d <= K; d += kWideThreads) ot[d] = -1;
  for (int d = tid; d < K; d += kWideThreads) accept_probs[(size_t)b * K + d] = -1.0;
  const double* u = uniforms + (size_t)b * (K + 1);
  int ui = 0, nacc = 0, bad = 0;
  for (int d = 0; d <= Kb; ++d) {
    const WideLaw P = wide_law(lawbuf, row_bytes, V, tb + d);
    const WideLaw Q = d < Kb ? wide_law(lawbuf, row_bytes, V, nt + db + d) : P;
    if (P.nonfinite || Q.nonfinite) {
      bad = 1;
      break;
    }
    if (d == Kb) {   // all drafts accepted: bonus from row K_b
      const int tok = block_choice(P.ids, P.probs, P.n, u[ui++], s_d, &s_last, s_w);
      if (tid == 0) ot[Kb] = tok;
      nacc = Kb;
      break;
    }
    const int tok = draft_ids[(size_t)db + d];
    if (tid == 0) {
      s_p = wide_prob(P, tok);
      s_q = wide_prob(Q, tok);
    }
    __syncthreads();
    const double p = s_p, q = s_q;
    __syncthreads();
    const double a = (q <= 0.0) ? (p > 0.0 ? 1.0 : 0.0) : fmin(1.0, p / q);
    const bool acc = u[ui++] <= a;
    if (tid == 0) accept_probs[(size_t)b * K + d] = a;
    if (acc) {
      if (tid == 0) ot[d] = tok;
      continue;
    }
    // Residual max(p - q, 0) over the union of supports, ids ascending: only
    // P's ids can be positive, in P's order.
    int n = 0;
    for (int base = 0; base < P.n; base += kWideThreads) {
      const int i = base + tid;
      double r = 0.0;
      int id = 0;
      if (i < P.n) {
        id = P.ids[i];
        r = fmax(P.probs[i] - wide_prob(Q, id), 0.0);
      }
      const bool keep = i < P.n && r > 0.0 && isfinite(r);
      int tot;
      const int pos = n + block_scan_flag(keep, s_w, &tot);
      if (keep) {
        rid[pos] = id;
        rp[pos] = r;
      }
      n += tot;
    }
    __syncthreads();
    int corr;
    const double t1 = n ? block_sum_f64(rp, n, s_d) : 0.0;
    if (n == 0 || !(isfinite(t1) && t1 > 0.0)) {
      corr = block_choice(P.ids, P.probs, P.n, u[ui++], s_d, &s_last, s_w);
    } else {
      for (int i = tid; i < n; i += kWideThreads) rp[i] = rp[i] / t1;
      __syncthreads();
      const double t2 = block_sum_f64(rp, n, s_d);
      for (int i = tid; i < n; i += kWideThreads) rp[i] = rp[i] / t2;
      __syncthreads();
      corr = block_choice(rid, rp, n, u[ui++], s_d, &s_last, s_w);
    }
    if (tid == 0) ot[d] = corr;
    nacc = d;
    break;
  }
  if (tid == 0) {
    status[b] = bad;
    n_accepted[b] = nacc;
  }
}

// Per-row output of wide laws (and one draw per row).
__global__ __launch_bounds__(kWideThreads) void wide_rows_kernel(const unsigned char* __restrict__ lawbuf,
                                                                 size_t row_bytes, int V,
                                                                 const double* __restrict__ uniforms,
                                                                 int32_t* __restrict__ out_ids,
                                                                 double* __restrict__ out_probs, int ld_out,
                                                                 int32_t* __restrict__ out_count,
                                                                 int32_t* __restrict__ sampled,
                                                                 int32_t* __restrict__ status) {
  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  __shared__ double s_d[kWideWaves];
  __shared__ double s_last;
  __shared__ uint32_t s_w[kWideWaves + 1];
  const WideLaw L = wide_law(lawbuf, row_bytes, V, r);
  if (tid == 0) {
    status[r] = L.nonfinite ? 1 : 0;
    if (out_count) out_count[r] = L.n;
  }
  if (out_ids)
    for (int i = tid; i < ld_out; i += kWideThreads) {
      out_ids[(size_t)r * ld_out + i] = i < L.n ? L.ids[i] : -1;
      out_probs[(size_t)r * ld_out + i] = i < L.n ? L.probs[i] : 0.0;
    }
  if (sampled) {
    const int tok = L.nonfinite ? -1 : block_choice(L.ids, L.probs, L.n, uniforms[r], s_d, &s_last, s_w);
    if (tid == 0) sampled[r] = tok;
  }
}

// logits[rows[i] * ld + ids[i]] += -deltas[i] in fp32 ((row, id) pairs unique).
__global__ void logit_deltas_kernel(float* logits, long long ld, const int32_t* rows, const int32_t* ids,
                                    const float* deltas, int n, int R, int V, int32_t* status) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int r = rows[i], id = ids[i];
  if (r < 0 || r >= R || id < 0 || id >= V) {
    if (status) atomicOr(status, 1);
    return;
  }
  float* x = logits + (size_t)r * ld + id;
  *x = *x + (-deltas[i]);
}

}  // namespace mtp

using namespace mtp;

// Workspace: chunk partials [rows][n_chunks]; on the wide path followed (at
// a 256-byte boundary) by rows wide laws and rows residual scratch areas.
static size_t parts_bytes(int rows, int V) {
  return ((size_t)rows * cdiv(V, kChunk) * sizeof(ChunkPart) + 255) & ~(size_t)255;
}

MTP_API size_t mtp_sampler_workspace_bytes(int rows, int V, int top_k) {
  if (rows < 1 || V < 1 || top_k < 0) return 0;
  const int k_eff = (top_k > 0 && top_k < V) ? top_k : V;
  size_t n = parts_bytes(rows, V);
  if (k_eff > kMaxTopK) n += 2 * (size_t)rows * wide_row_bytes(V);
  return n;
}

// The accept step over nt target and nd draft rows (the uniform batch has
// nt = B (K + 1), nd = B K and null offsets).
static int spec_accept_run(const float* target_logits, const float* draft_logits, const int32_t* draft_ids,
                           const double* uniforms, int B, int K, int V, double temperature, int top_k, double top_p,
                           int32_t* out_tokens, int32_t* n_accepted, double* accept_probs, int32_t* status, void* ws,
                           size_t ws_bytes, void* stream, AcceptRows rr, int nt, int nd, const char* who) {
  SamplerPlan pl;
  int rc = sampler_plan(V, top_k, temperature, &pl, who);
  if (rc) return rc;
  if (B < 1 || K < 1 || nt < B || nd < 0 || !target_logits || (nd > 0 && !draft_logits) || !draft_ids || !uniforms ||
      !out_tokens || !n_accepted || !accept_probs || !status) {
    set_error("%s: need B>=1, K>=1 and non-null buffers", who);
    return MTP_ERR_ARG;
  }
  const int rows = nt + nd;
  const size_t need = mtp_sampler_workspace_bytes(rows, V, pl.greedy ? 1 : top_k);
  if (!ws || ws_bytes < need) {
    set_error("%s: workspace %zu B < required %zu B", who, ws_bytes, need);
    return MTP_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  const int n_chunks = pl.n_chunks;
  ChunkPart* tparts = reinterpret_cast<ChunkPart*>(ws);
  ChunkPart* dparts = tparts + (size_t)nt * n_chunks;
  const double temp = pl.greedy ? 1.0 : temperature;
  rr.nt = nt;
  rr.nd = nd;
  // target rows then draft rows, one launch (dparts follows tparts)
  hipLaunchKernelGGL(vocab_partials, dim3(n_chunks, rows), dim3(kSampThreads), 0, st, target_logits,
                     draft_logits ? draft_logits : target_logits, nt, (long long)V, V, n_chunks, temp, pl.ksel,
                     pl.greedy, tparts);
  if ((rc = launch_check(who))) return rc;
  if (pl.wide) {
    unsigned char* lawbuf = reinterpret_cast<unsigned char*>(ws) + parts_bytes(rows, V);
    const size_t rb = wide_row_bytes(V);
    hipLaunchKernelGGL(wide_law_kernel, dim3(rows), dim3(kWideThreads), 0, st, target_logits,
                       draft_logits ? draft_logits : target_logits, nt, (long long)V, V, tparts, n_chunks, temp,
                       pl.k_eff, top_p, lawbuf, rb);
    if ((rc = launch_check(who))) return rc;
    hipLaunchKernelGGL(wide_accept_kernel, dim3(B), dim3(kWideThreads), 0, st, lawbuf, rb, V, B, K, draft_ids,
                       uniforms, out_tokens, n_accepted, accept_probs, status, lawbuf + (size_t)rows * rb, rr);
  } else if (n_chunks <= 64) {
    const int nwv = 2 * K + 1 < 16 ? 2 * K + 1 : 16;
    const size_t lds = accept_laws_lds(K, nwv);
    if (lds > 160 * 1024 || K + 1 > 64) {   // (the LDS bound alone keeps K <= 41)
      set_error("%s: K=%d needs %zu B of LDS", who, K, lds);
      return MTP_ERR_UNSUPPORTED;
    }
    // A failure here surfaces as a launch error, checked below.
    if (lds > 65536) (void)hipFuncSetAttribute((const void*)accept_laws, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds);
    hipLaunchKernelGGL(accept_laws, dim3(B), dim3(nwv * 64), lds, st, tparts, n_chunks, dparts, n_chunks, draft_ids,
                       uniforms,
                       K, pl.ksel, pl.greedy, temp, top_p, out_tokens, n_accepted, accept_probs, status, rr);
  } else {
    hipLaunchKernelGGL(accept_finish, dim3(B), dim3(64), 0, st, tparts, dparts, n_chunks, draft_ids, uniforms, K,
                       pl.ksel, pl.greedy, temp, top_p, out_tokens, n_accepted, accept_probs, status, rr);
  }
  return launch_check(who);
}

MTP_API int mtp_spec_accept(const float* target_logits, const float* draft_logits, const int32_t* draft_ids,
                            const double* uniforms, int B, int K, int V, double temperature, int top_k,
                            double top_p, int32_t* out_tokens, int32_t* n_accepted, double* accept_probs, int32_t* status,
                            void* ws, size_t ws_bytes, void* stream) {
  if (B < 1 || K < 1) {
    set_error("mtp_spec_accept: need B>=1, K>=1");
    return MTP_ERR_ARG;
  }
  return spec_accept_run(target_logits, draft_logits, draft_ids, uniforms, B, K, V, temperature, top_k, top_p,
                         out_tokens, n_accepted, accept_probs, status, ws, ws_bytes, stream, AcceptRows{}, B * (K + 1),
                         B * K, "mtp_spec_accept");
}

MTP_API int mtp_spec_accept_ragged(const float* target_logits, int n_target, const float* draft_logits, int n_draft,
                                   const int32_t* t_off, const int32_t* d_off, const int32_t* k_lens,
                                   const int32_t* draft_ids, const double* uniforms, int B, int K_max, int V,
                                   double temperature, int top_k, double top_p, int32_t* out_tokens,
                                   int32_t* n_accepted, double* accept_probs, int32_t* status, void* ws,
                                   size_t ws_bytes, void* stream) {
  if (!t_off || !d_off || !k_lens) {
    set_error("mtp_spec_accept_ragged: t_off, d_off and k_lens are required");
    return MTP_ERR_ARG;
  }
  AcceptRows rr{t_off, d_off, k_lens, n_target, n_draft};
  return spec_accept_run(target_logits, draft_logits, draft_ids, uniforms, B, K_max, V, temperature, top_k, top_p,
                         out_tokens, n_accepted, accept_probs, status, ws, ws_bytes, stream, rr, n_target, n_draft,
                         "mtp_spec_accept_ragged");
}

// ---- No-allocation variant --------------------------------------------------
// For callers that cannot allocate (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc): mtp_spec_accept with its
// workspace in a file-scope device array. Each GPU holds its own copy for the
// life of the process; its address is looked up once per device
// (hipGetSymbolAddress, with that device current) and cached. Nothing in the
// sampler's workspace has to start at zero: every chunk partial, law and
// residual area is written before it is read. Calls that overlap on one GPU
// share the array and race; calls must be stream-ordered.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int noalloc_scratch(void** out, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("%s: hipGetDevice failed: %s", who, hipGetErrorString(e));
    return MTP_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("%s: device %d outside the %d the scratch table covers", who, dev, kMaxDevices);
    return MTP_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev, hipGetErrorString(e));
      return MTP_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MTP_OK;
}

MTP_API int mtp_spec_accept_noalloc(const float* target_logits, const float* draft_logits, const int32_t* draft_ids,
                                    const double* uniforms, int B, int K, int V, double temperature, int top_k,
                                    double top_p, int32_t* out_tokens, int32_t* n_accepted, double* accept_probs,
                                    int32_t* status, void* stream) {
  const char* who = "mtp_spec_accept_noalloc";
  if (B < 1 || K < 1 || V < 1 || top_k < 0) {
    set_error("%s: need B>=1, K>=1, V>=1, top_k>=0", who);
    return MTP_ERR_ARG;
  }
  const int greedy = !(temperature > 0.0);
  const size_t need = mtp_sampler_workspace_bytes(B * (2 * K + 1), V, greedy ? 1 : top_k);
  if (need > kNoAllocScratchBytes) {
    set_error("%s: B=%d K=%d V=%d top_k=%d needs %zu B of scratch; the no-allocation entry point has %zu B "
              "(use mtp_spec_accept with a workspace)", who, B, K, V, top_k, need, kNoAllocScratchBytes);
    return MTP_ERR_UNSUPPORTED;
  }
  void* ws = nullptr;
  const int rc = noalloc_scratch(&ws, who);
  if (rc) return rc;
  return mtp_spec_accept(target_logits, draft_logits, draft_ids, uniforms, B, K, V, temperature, top_k, top_p,
                         out_tokens, n_accepted, accept_probs, status, ws, kNoAllocScratchBytes, stream);
}

MTP_API int mtp_sample_rows(const float* logits, int rows, int V, double temperature, int top_k, double top_p,
                            const double* uniforms, int32_t* out_ids, double* out_probs, int ld_out,
                            int32_t* out_count, int32_t* sampled, int32_t* status, void* ws, size_t ws_bytes,
                            void* stream) {
  const char* who = "mtp_sample_rows";
  SamplerPlan pl;
  int rc = sampler_plan(V, top_k, temperature, &pl, who);
  if (rc) return rc;
  if (rows < 1 || !logits || !status || (sampled && !uniforms) || (out_ids && !out_probs)) {
    set_error("%s: need rows>=1, logits, status, and uniforms when sampling", who);
    return MTP_ERR_ARG;
  }
  const int bound = pl.greedy ? 1 : pl.k_eff;   // the support never exceeds this
  if (out_ids && ld_out < bound) {
    set_error("%s: ld_out %d < the support bound %d", who, ld_out, bound);
    return MTP_ERR_ARG;
  }
  const size_t need = mtp_sampler_workspace_bytes(rows, V, pl.greedy ? 1 : top_k);
  if (!ws || ws_bytes < need) {
    set_error("%s: workspace %zu B < required %zu B", who, ws_bytes, need);
    return MTP_ERR_WORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  ChunkPart* parts = reinterpret_cast<ChunkPart*>(ws);
  const double temp = pl.greedy ? 1.0 : temperature;
  hipLaunchKernelGGL(vocab_partials, dim3(pl.n_chunks, rows), dim3(kSampThreads), 0, st, logits, logits, rows,
                     (long long)V, V, pl.n_chunks, temp, pl.ksel, pl.greedy, parts);
  if ((rc = launch_check(who))) return rc;
  if (pl.wide) {
    unsigned char* lawbuf = reinterpret_cast<unsigned char*>(ws) + parts_bytes(rows, V);
    const size_t rb = wide_row_bytes(V);
    hipLaunchKernelGGL(wide_law_kernel, dim3(rows), dim3(kWideThreads), 0, st, logits, logits, rows, (long long)V,
                       V, parts, pl.n_chunks, temp, pl.k_eff, top_p, lawbuf, rb);
    if ((rc = launch_check(who))) return rc;
    hipLaunchKernelGGL(wide_rows_kernel, dim3(rows), dim3(kWideThreads), 0, st, lawbuf, rb, V, uniforms, out_ids,
                       out_probs, ld_out, out_count, sampled, status);
  } else {
    hipLaunchKernelGGL(row_laws, dim3(rows), dim3(64), 0, st, parts, pl.n_chunks, pl.ksel, pl.greedy, temp, top_p,
                       uniforms, out_ids, out_probs, ld_out, out_count, sampled, status);
  }
  return launch_check(who);
}

MTP_API int mtp_apply_logit_deltas(float* logits, long long ld, int rows, int V, const int32_t* row_ids,
                                   const int32_t* token_ids, const float* deltas, int n, int32_t* status,
                                   void* stream) {
  const char* who = "mtp_apply_logit_deltas";
  if (n == 0) return MTP_OK;
  if (!logits || !row_ids || !token_ids || !deltas || n < 0 || rows < 1 || V < 1 || ld < V) {
    set_error("%s: bad arguments", who);
    return MTP_ERR_ARG;
  }
  hipLaunchKernelGGL(logit_deltas_kernel, dim3(cdiv(n, 256)), dim3(256), 0, (hipStream_t)stream, logits, ld, row_ids,
                     token_ids, deltas, n, rows, V, status);
  return launch_check(who);
}
