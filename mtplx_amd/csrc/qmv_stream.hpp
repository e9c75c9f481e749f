// The resident streaming matmul body for the verify shapes (packed weights,
// all of x in LDS), run by the standalone kernel (qmv.hip); written as a body
// with a pre-read hook so a persistent kernel can run it as one phase.
#pragma once

#include "qmv_common.hpp"

#include <type_traits>

namespace mtp {

// ---------------------------------------------------------------------------
// Resident streaming kernel (the fast path): all of x is staged into LDS once
// per workgroup, then every wave walks its flat (tile, quad) item list with a
// register ring of NR quads advanced by unrolling — no register copies and
// no data-dependent branches between a load and its use, so the compiler's
// wait for quad i only covers loads issued before i (the NR-1 quads behind it
// stay in flight). Lanes whose A-operand row is past M read a zero block in
// LDS instead of branching.
//
// MF (packed layout 2, M <= 4 with R = 4, M <= 16 with R = 8): the quads run
// on v_mfma_f32_16x16x32_bf16 (quad_mma16 / quad_mma16x16): half the MFMA
// cycles of the 32x32x16 form, whose 32 A rows these row counts half fill,
// and at 4 rows a quarter of the group-finish FMAs. Staging and epilogues are
// shared.
//
// The body takes its block index vb and grid size vg as arguments so a
// persistent kernel can run it as one phase of several. ``pre`` is called
// once by every thread after the weight ring's first loads are issued and
// before anything produced by an earlier phase is read (x, its norm
// statistics and sums): a grid barrier there overlaps the weights' first
// round trip with the previous phase's tail. With it the epilogue's global
// stores are device-coherent (WT), so the next phase may read them from
// another XCD after the barrier.
struct NoHook {
  __device__ void operator()() const {}
};

// Adds the S parts of one tile's fp32 sums [S][M*64] (device-coherent loads)
// into fin, in part order. A thread's elements (at most 8: M*64 <= 8 *
// threads) of up to 8 parts are loaded together, so the sum costs
// ceil(S / 8) round trips (a tile split 16 ways, 2).
// MAXN: the largest n the caller has (M <= 2R rows of 64 values).
template <int NT, int MAXN>
__device__ __forceinline__ void sum_parts(const float* p0, int S, int n, float* fin, int tid) {
  static_assert(NT * 8 >= MAXN, "at most 8 elements per thread");
  constexpr int kE = (MAXN + NT - 1) / NT;   // elements per thread at n = MAXN
  float a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) a[k] = 0.f;
  for (int q0 = 0; q0 < S; q0 += 8) {
    float l[8][kE];
#pragma unroll
    for (int qq = 0; qq < 8; ++qq)
#pragma unroll
      for (int k = 0; k < kE; ++k) {
        const int idx = tid + k * NT;
        l[qq][k] = (q0 + qq < S && idx < n)
                       ? __hip_atomic_load(p0 + (size_t)(q0 + qq) * n + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                       : 0.f;
      }
#pragma unroll
    for (int qq = 0; qq < 8; ++qq)
      if (q0 + qq < S)
#pragma unroll
        for (int k = 0; k < kE; ++k) a[k] += l[qq][k];
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int idx = tid + k * NT;
    if (idx < n) fin[idx] = a[k];
  }
}

//
// NRT: depth of the weight ring. Its first fill is a burst of every wave's
// loads at once, which x staging waits behind, so the best depth follows the
// quads a wave takes per tile: 1 for <= 3 (q|k|v, o at K = 5120), 2 beyond.
template <int NW, int R, int XM, int EM, int GSH, bool PK, bool MF = false, int NRT = 3, typename Hook = NoHook>
__device__ __forceinline__ void qmv_stream_body(const QmmParams& p, const int vb, const int vg, Hook&& pre) {
  constexpr bool kPhase = !std::is_same<std::decay_t<Hook>, NoHook>::value;
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NT = NW * 64;
  constexpr bool dual = (EM == E_DUAL || EM == E_DUAL_SWIGLU);
  constexpr int KS = dual ? NW / 2 : NW;
  constexpr int XSW = 2 * R;
  constexpr int NR = NRT;
  constexpr bool MF16 = MF && R == 8;   // up to 16 rows on the 16x16x32 form
  static_assert(!MF || R == 4 || R == 8, "the 16x16x32 form takes R = 4 (4 rows) or 8 (16 rows)");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: scalar loop control
  const int kw = wave % KS;
  const int which = dual ? (wave / KS) : 0;
  const int M = p.M;
  const int Q = p.K >> 8;
  const NibConsts nc = nib_consts();
  // Tail split (packed weights only): workgroups from p.tail_first on each
  // take quads [q_lo, q_lo + q_n) of a leftover tile, one of tail_split
  // parts; the part that arrives last sums the parts in order and finishes.
  const bool tail = PK && p.tail_split > 1 && vb >= p.tail_first;
  const bool full = tail && p.full_split;
  // Tile stride between a workgroup's tiles: the grid, or the number of tile
  // groups in the full split.
  const int G = full ? vg / p.tail_split : vg;
  int tile0 = vb, part = 0, q_lo = 0, q_n = Q;
  if (tail) {
    const int e = vb - p.tail_first;
    tile0 = p.tail_first + e / p.tail_split;
    part = e - (e / p.tail_split) * p.tail_split;
    q_lo = (part * Q) / p.tail_split;
    q_n = ((part + 1) * Q) / p.tail_split - q_lo;
  }
  // A phase's grid can exceed its work (a persistent kernel keeps every CU):
  // workgroups without a tile only meet the barrier.
  if (tail ? vb - p.tail_first >= (p.n_blocks - p.tail_first) * p.tail_split : tile0 >= p.n_blocks) {
    if constexpr (kPhase) pre();
    return;
  }

  // LDS holds QX quads of x: all of K, or one part's share (full split).
  const int QX = p.xq > 0 ? p.xq : Q;
  uint4* xa = reinterpret_cast<uint4*>(smem);                                  // staged x, xa_index()
  const int rstride = xa_row_stride(4 * QX);
  float* xs = reinterpret_cast<float*>(smem + xa_bytes(4 * QX, M));            // [QX*4][XSW]
  float* red = xs + QX * 4 * XSW;                                              // [NW][M][32]
  float* fin = red + NW * M * 32;                                              // [M][64]
  __shared__ float s_inv_rms[32];
  __shared__ int s_last;

  const int c32 = lane & 31;
  const int kq = lane >> 5;
  const uint32_t* W = which ? p.w1 : p.w0;
  const uint16_t* Sc = which ? p.s1 : p.s0;
  const uint16_t* Bi = which ? p.b1 : p.b0;
  const int sgroups = p.K >> (6 + GSH);
  const int qw = (q_n > kw) ? cdiv(q_n - kw, KS) : 0;
  const int ntiles = full ? cdiv(p.n_blocks - tile0, G) : ((PK && p.tail_split > 1) ? 1 : cdiv(p.n_blocks - vb, G));
  const int nitems = ntiles * qw;

  // A operands: lanes of rows >= M repeat row c32 % M (their output rows
  // are never stored), so every lane reads its quad at immediate offsets.
  const uint32_t a_lane = (uint32_t)xa_index(kq, c32 % M, M, rstride, 0, 0) * 16;
  const uint32_t x_lane = (uint32_t)((unsigned char*)xs - smem) + 16 * kq;

  struct QuadRegs {
    uint4 w[4];
    uint32_t s[2], b[2];
    uint32_t s1[MF ? 2 : 1], b1[MF ? 2 : 1];   // MF: the lane's second column (16 + l%16)
  };
  // Prefetch iterator: tile j_pf, quad counter t_pf (q = kw + t_pf*KS); the
  // per-lane row pointers are recomputed only when the tile changes.
  int j_pf = 0, t_pf = 0, left_pf = nitems;
  const uint32_t* wrow = nullptr;
  const uint16_t* srow = nullptr;
  const uint16_t* brow = nullptr;
  auto set_rows = [&](int j) {
    const int nb = tile0 + j * G;
    if (PK) {
      // Tile-major packed weights: per (tile, quad) 1152 words — 4 x 256
      // words of nibbles in load order, then 32 rows x (4 s, 4 b) bf16.
      wrow = W + (size_t)nb * Q * kPackQuadWords + lane * 4;
      srow = reinterpret_cast<const uint16_t*>(W + (size_t)nb * Q * kPackQuadWords + 1024 + (MF ? (lane & 15) : c32) * 4);
      brow = nullptr;
    } else {
      const int n = nb * 32 + c32;
      const int nrow = n < p.N ? n : 0;
      const int kw0 = qw > 0 ? kw : 0;   // waves without quads read a valid block
      wrow = W + (size_t)nrow * (p.K >> 3) + kq * 4 + 32 * kw0;
      srow = Sc + (size_t)nrow * sgroups + (GSH == 0 ? 4 : 2) * kw0;
      brow = Bi + (size_t)nrow * sgroups + (GSH == 0 ? 4 : 2) * kw0;
    }
  };
  set_rows(0);
  // Loads the iterator's current item, then advances it (past the end it
  // keeps re-reading the last item, whose registers are never used).
  auto load_next = [&](QuadRegs& qr) {
    if (PK) {
      const size_t qoff = (size_t)(q_lo + (qw > 0 ? kw + KS * t_pf : 0)) * kPackQuadWords;
      const uint32_t* wp = wrow + qoff;
#pragma unroll
      for (int u = 0; u < 4; ++u) qr.w[u] = *reinterpret_cast<const uint4*>(wp + 256 * u);
      const uint4 sb = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint32_t*>(srow) + qoff);
      qr.s[0] = sb.x; qr.s[1] = sb.y;
      qr.b[0] = sb.z; qr.b[1] = sb.w;
      if (MF) {
        const uint4 sb1 = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint32_t*>(srow) + qoff + 64);
        qr.s1[0] = sb1.x; qr.s1[MF ? 1 : 0] = sb1.y;
        qr.b1[0] = sb1.z; qr.b1[MF ? 1 : 0] = sb1.w;
      }
    } else {
      const uint32_t* wp = wrow + 32 * KS * t_pf;
#pragma unroll
      for (int u = 0; u < 4; ++u) qr.w[u] = *reinterpret_cast<const uint4*>(wp + 8 * u);
      if (GSH == 0) {
        const uint2 sv = *reinterpret_cast<const uint2*>(srow + 4 * KS * t_pf);
        const uint2 bv = *reinterpret_cast<const uint2*>(brow + 4 * KS * t_pf);
        qr.s[0] = sv.x; qr.s[1] = sv.y;
        qr.b[0] = bv.x; qr.b[1] = bv.y;
      } else {
        qr.s[0] = *reinterpret_cast<const uint32_t*>(srow + 2 * KS * t_pf);
        qr.b[0] = *reinterpret_cast<const uint32_t*>(brow + 2 * KS * t_pf);
        qr.s[1] = qr.s[0];
        qr.b[1] = qr.b[0];
      }
    }
    if (left_pf > 1) {
      --left_pf;
      if (++t_pf == qw) {
        t_pf = 0;
        set_rows(++j_pf);
      }
    }
  };

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  // MF: A row 4m holds x row m, read by lanes with (l%16) = 4m (the other
  // lanes of each four read a valid row too; their outputs are unused).
  // MF16: A row m holds x row m (rows past M read row 0, outputs unused), and
  // lane l's group sums are those of rows 4(l/16) .. + 3 (zero past M).
  const int mf_arow = MF16 ? ((lane & 15) < M ? (lane & 15) : 0) : (((lane & 15) >> 2) < M ? ((lane & 15) >> 2) : 0);
  const uint32_t mf_a0 = (uint32_t)xa_index(0, mf_arow, M, rstride, 0, lane >> 4) * 16;
  const uint32_t mf_a1 = (uint32_t)xa_index(1, mf_arow, M, rstride, 0, lane >> 4) * 16;
  const uint32_t mf_x = (uint32_t)((unsigned char*)xs - smem) +
                        (MF16 ? 16 * (lane >> 4) : 4 * ((lane >> 4) < M ? (lane >> 4) : 0));

  auto compute = [&](const QuadRegs& cr, int t) {
    const int gq = 4 * (kw + t * KS);
    float sv[4], cb[4];
    quad_scales<GSH>(cr.s, cr.b, sv, cb);
    if constexpr (MF) {
      float sv1[4], cb1[4];
      const uint32_t s1w[2] = {cr.s1[0], cr.s1[MF ? 1 : 0]}, b1w[2] = {cr.b1[0], cr.b1[MF ? 1 : 0]};
      quad_scales<0>(s1w, b1w, sv1, cb1);
      if constexpr (MF16) {
        float (&t0)[4] = *reinterpret_cast<float (*)[4]>(&acc[0]);
        float (&t1)[4] = *reinterpret_cast<float (*)[4]>(&acc[MF16 ? 4 : 0]);
        quad_mma16x16(smem, mf_a0 + (uint32_t)gq * 128, mf_a1 + (uint32_t)gq * 128,
                      mf_x + (uint32_t)gq * (XSW * 4), XSW, cr.w, sv, cb, sv1, cb1, nc, t0, t1);
      } else {
        quad_mma16(smem, mf_a0 + (uint32_t)gq * 128, mf_a1 + (uint32_t)gq * 128, mf_x + (uint32_t)gq * (XSW * 4),
                   XSW, cr.w, sv, cb, sv1, cb1, nc, acc[0], acc[1]);
      }
    } else {
      quad_mma<R>(smem, a_lane + (uint32_t)gq * 128, x_lane + (uint32_t)gq * (XSW * 4), cr.w, sv, cb, nc, acc);
    }
  };

  // Residual of this thread's first epilogue element, fetched now so the
  // epilogue does not wait for it.
  float pre_resid = 0.f;
  const bool use_pre = (EM == E_RESID) && (R == 4) && ntiles > 0;
  if (use_pre && tid < M * 32) {
    const int col = tile0 * 32 + (tid & 31);
    if (col < p.N) pre_resid = bf2f(p.resid[(size_t)(tid >> 5) * p.ldy + col]);
  }
  // E_ROPE_QKV: the request offsets of this thread's first epilogue element
  // are fetched now; its rotation is computed after staging.
  RopeRow rope_pre = {};
  const bool use_rpre = (EM == E_ROPE_QKV) && ntiles > 0 && tid < M * 16;
  int rq_start = 0, rq_len = 0;
  if (use_rpre) {
    const int b = (tid >> 4) / p.rope_L;
    rq_start = p.q_start[b];
    rq_len = p.q_lens ? p.q_lens[b] : p.rope_L;
  }

  // End of tile j: reduce the K-split waves in LDS (wave order), epilogue.
  auto finish = [&](int j) {
    const int nb = tile0 + j * G;
    const bool valid = nb * 32 + c32 < p.N;
    lds_barrier();
    if constexpr (MF16) {   // lane l: rows 4(l/16) + i, columns l%16 (acc[i]) and 16 + l%16 (acc[4 + i])
      const int c = lane & 15;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 4 * (lane >> 4) + i;
        if (m < M) {
          red[(wave * M + m) * 32 + c] = (nb * 32 + c < p.N) ? acc[i] : 0.f;
          red[(wave * M + m) * 32 + 16 + c] = (nb * 32 + 16 + c < p.N) ? acc[4 + i] : 0.f;
        }
      }
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.f;
    } else if constexpr (MF) {   // lane l: row l/16, columns l%16 and 16 + l%16
      const int m = lane >> 4, c = lane & 15;
      if (m < M) {
        red[(wave * M + m) * 32 + c] = (nb * 32 + c < p.N) ? acc[0] : 0.f;
        red[(wave * M + m) * 32 + 16 + c] = (nb * 32 + 16 + c < p.N) ? acc[1] : 0.f;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] = 0.f;
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int m = 8 * (r >> 2) + 4 * kq + (r & 3);
        if (m < M) red[(wave * M + m) * 32 + c32] = valid ? acc[r] : 0.f;
        acc[r] = 0.f;
      }
    }
    lds_barrier();
    for (int idx = tid; idx < M * 64; idx += NT) {
      const int m = idx >> 6;
      const int cc = idx & 63;
      const int mat = cc >> 5;
      float v = 0.f;
      if (!dual && mat == 0) {
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[(w * M + m) * 32 + cc];
      } else if (dual) {
#pragma unroll
        for (int w = 0; w < KS; ++w) v += red[((mat * KS + w) * M + m) * 32 + (cc & 31)];
      }
      fin[idx] = v;
    }
    lds_barrier();
    if (tail) {
      // This part's sums to the workspace (device-coherent stores), then
      // arrive; the last arrival adds the parts in part order and finishes.
      const int e = (nb - p.tail_first) * p.tail_split + part;   // this tile's part slot
      for (int idx = tid; idx < M * 64; idx += NT)
        __hip_atomic_store(p.partial + (size_t)e * (M * 64) + idx, fin[idx], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      if (full) return;   // arrives for all its tiles at the end (arrive_all)
      __builtin_amdgcn_s_waitcnt(0);
      lds_barrier();
      const int ti = nb - p.tail_first;
      if (tid == 0) {
        const unsigned old =
            __hip_atomic_fetch_add(p.counters + ti, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old == (unsigned)(p.tail_split - 1)) ? 1 : 0;
      }
      lds_barrier();
      if (!s_last) return;
      sum_parts<NT, 2 * R * 64>(p.partial + (size_t)ti * p.tail_split * (M * 64), p.tail_split, M * 64, fin, tid);
      lds_barrier();
      qmm_epilogue<NW, EM, kPhase>(p, fin, nb, M, 0);
      if (tid == 0) __hip_atomic_store(p.counters + ti, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    qmm_epilogue<NW, EM, kPhase>(p, fin, nb, M, 0, (use_pre && j == 0) ? &pre_resid : nullptr,
                         (use_rpre && j == 0) ? &rope_pre : nullptr);
  };

  // Full split: after the last tile, wait once for all the part stores, then
  // arrive at every tile's counter; for the tiles where this part came last,
  // add the parts in part order and run the epilogue.
  __shared__ unsigned char s_lastv[64];
  auto arrive_all = [&]() {
    if (!full) return;
    __builtin_amdgcn_s_waitcnt(0);
    lds_barrier();
    for (int j0 = 0; j0 < ntiles; j0 += 64) {
      const int jn = ntiles - j0 < 64 ? ntiles - j0 : 64;
      if (tid < jn) {
        const int nb = tile0 + (j0 + tid) * G;
        const unsigned old =
            __hip_atomic_fetch_add(p.counters + nb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_lastv[tid] = (old == (unsigned)(p.tail_split - 1)) ? 1 : 0;
      }
      lds_barrier();
      for (int jj = 0; jj < jn; ++jj) {
        if (!s_lastv[jj]) continue;   // the same LDS value for every thread
        const int nb = tile0 + (j0 + jj) * G;
        sum_parts<NT, 2 * R * 64>(p.partial + (size_t)nb * p.tail_split * (M * 64), p.tail_split, M * 64, fin, tid);
        lds_barrier();
        qmm_epilogue<NW, EM, kPhase>(p, fin, nb, M, 0);
        if (tid == 0) __hip_atomic_store(p.counters + nb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lds_barrier();   // fin is reused by the next tile
      }
      lds_barrier();   // s_lastv is rewritten by the next round
    }
  };

  // Prologue: the norm statistics, x straight into LDS, the norm weights
  // into registers, then all three ring slots, issued back to back. The
  // wait below is for everything but the ring loads (they are the newest),
  // so staging x overlaps the weights' first round trip.
  // As a phase (kPhase), the ring loads come first and ``pre`` runs before
  // the staging loads, which then wait with everything else.
  QuadRegs ring[NR];
  if constexpr (kPhase) {
#pragma unroll
    for (int u = 0; u < NR; ++u) load_next(ring[u]);
    asm volatile("" ::: "memory");
    pre();
  }
  float ssv[kMaxSsLoads];
  if (XM == X_RMSNORM && p.ss_in && wave < M) ss_prefetch(p, wave, lane, ssv);
  stage_x_issue<NW>(p, xa, rstride, M, Q, q_lo, q_n, wave, lane);
  uint4 wpre[kNormPre];
  if (XM == X_RMSNORM) norm_w_prefetch<NW>(p, wpre, Q, q_lo, q_n, tid);
  float2 xsv[kSumPre];
  if (XM == X_PRE) xsum_prefetch<NW, XSW>(p, xsv, M, Q, q_lo, q_n, tid);
  asm volatile("" ::: "memory");
  if constexpr (kPhase) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
  } else {
#pragma unroll
    for (int u = 0; u < NR; ++u) load_next(ring[u]);   // waves without items reload a valid block; never used
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(NR * ((PK && !MF) ? 5 : 6)));   // loads per ring slot
  }
  if (XM == X_RMSNORM) {
    for (int m = wave; m < M; m += NW) {
      const float v = (p.ss_in && m == wave) ? ss_reduce(p, ssv, lane) : row_inv_rms(p, m, lane);
      if (lane == 0) s_inv_rms[m] = v;
    }
  }
  lds_barrier();
  if (XM == X_PRE)
    xsum_finish<NW, XSW>(p, xs, xsv, M, Q, q_lo, q_n, tid);
  else
    stage_x_finish<XM, NW, XSW, PK>(p, xa, rstride, xs, wpre, s_inv_rms, M, Q, q_lo, q_n, tid);
  lds_barrier();  // staged x visible to every wave
  if (use_rpre) {
    const int head = tile0 / (p.rope_D >> 5);
    const int d = 16 * (tile0 - head * (p.rope_D >> 5)) + (tid & 15);
    rope_pre = rope_row(p, tid >> 4, d, rq_start, rq_len);
  }

  // Every wave of the workgroup must reach each tile's barriers: waves with
  // fewer quads per tile (qw smaller) still finish every tile.
  if (qw == 0) {
    for (int j = 0; j < ntiles; ++j) finish(j);
    arrive_all();
    return;
  }
  // One exit, at the bottom: a break after each step would be merged by the
  // control-flow structurizer into the latch, and the waitcnt analysis would
  // then see the ring's newest loads as pending at the loop head and drain
  // the whole ring there (vmcnt(0)) every iteration. Steps past the end are
  // skipped by a uniform branch instead.
  int i = 0, t = 0, j = 0;
  auto step = [&](const QuadRegs& cur) {
    if (i < nitems) {
      compute(cur, t);
      if (++t == qw) {
        finish(j);
        t = 0;
        ++j;
      }
      ++i;
    }
  };
  do {
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      step(ring[u]);
      load_next(ring[u]);
    }
  } while (i < nitems);
  arrive_all();
}

}  // namespace mtp
