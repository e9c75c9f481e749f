// 4-bit affine quantized matmul for 9..64 verify rows (continuous-batched
// ragged verify: M = sum of the requests' K_b + 1), gfx950.
//
//   y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/gs] + b[n, k/gs])
//
// At these M all of x no longer fits in one workgroup's LDS (64 rows x 5120
// k is 640 KB), so x streams through LDS quad by quad (256 k per step, a
// double buffer of at most 32 KB each) while every weight quad is read from
// HBM exactly once and applied to all M rows:
//  * a workgroup of 4 waves owns a column group: 4 tiles of 32 columns (one
//    per wave), or 2 column tiles x {gate, up} for the fused SwiGLU pair, so
//    each staged x quad serves 128 weight columns;
//  * x rows land in LDS with direct-to-LDS loads (no registers); each 16-byte
//    chunk kc of row m sits at slot 32m + (kc ^ (m & 15)), so one wave load
//    writes 1 KB contiguous and the A-operand reads of 16 consecutive rows
//    hit 16 different 16-byte bank groups;
//  * the weights stream from the tile-major packed layout (mtp_pack_affine4)
//    through a two-deep register ring, exactly as the skinny kernel reads
//    them; nibbles become exact bf16 operands 128 + q with one AND-OR each;
//  * v_mfma_f32_32x32x16_bf16 with A = x rows (one or two 32-row blocks), B =
//    the lane's weight column; each 64-k group is finished as acc += s * G
//    on the VALU, and the bias term (b - 128 s) * sum(x_group) of a quad's
//    four groups as an fp32 MFMA over (group sums from LDS) x (b - 128 s), so
//    the dequantised weights are never rounded (the numerics of the skinny
//    path);
//  * groups left over after the last full round of workgroups are split by K
//    over the idle CUs; their parts store fp32 sums, and the last part to
//    arrive adds them in part order (deterministic) and runs the epilogue.
// Epilogues: bf16 store (or fp32 of the bf16-rounded value), + residual,
// and silu(gate) * up for the fused pair.
#include "qmv_args.hpp"

namespace mtp {

constexpr int kQmWaves = 4;
constexpr int kQmThreads = kQmWaves * 64;
constexpr int kQmSlotsPerRow = 32;   // 16-byte chunks of one x row per quad (256 bf16)

struct QmmRowsParams {
  const uint16_t* x;
  const uint32_t* w0;
  const uint32_t* w1;      // up matrix of the fused pair
  uint16_t* y;
  float* yf;
  const uint16_t* resid;
  int M, N, K, ldx, ldy;
  int Q;                   // quads (K / 256)
  int ntiles;              // 32-column tiles
  int full_groups;         // groups that run over all of K
  int split;               // parts of each leftover group (1: none)
  float* partial;          // [leftover groups][split][waves][R2*16][64]
  uint32_t* counters;      // [leftover groups]
};

__device__ __forceinline__ int xslot(int m, int kc) { return m * kQmSlotsPerRow + (kc ^ (m & 15)); }

// Direct-to-LDS loads of x[0:M, 256q : 256q + 256): wave instruction t
// covers rows 2t and 2t + 1, instructions spread over nw waves. A row past M
// (odd M) loads row M - 1 into a slot row that is never an output.
__device__ __forceinline__ void qm_stage(const QmmRowsParams& p, unsigned char* buf, int q, int wave, int nw,
                                         int lane) {
  const int ninst = (p.M + 1) >> 1;
  for (int t = wave; t < ninst; t += nw) {
    const int m = 2 * t + (lane >> 5);
    const int mr = m < p.M ? m : p.M - 1;
    const int kc = (lane & 31) ^ (m & 15);
    __builtin_amdgcn_global_load_lds((gptr_t)(p.x + (size_t)mr * p.ldx + 256 * q + 8 * kc),
                                     (lptr_t)(buf + (size_t)t * 1024), 16, 0, 0);
  }
}

static bool rows_aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

static int env_int_rows(const char* name, int dflt) {
  const char* v = getenv(name);
  return (v && *v) ? atoi(v) : dflt;
}

struct QmQuad {
  uint4 w[4];
  uint4 sb;
};

// KH = 2: 8-wave workgroups whose two 4-wave halves take the two halves of
// the unit's quads in the same steps (both quads staged behind the same
// barriers), then add their sums in LDS in half order; two waves per SIMD
// instead of one, with the same grid.
// RGL: 8-row register groups of the last 32-row block that are finished
// (rows past M need no group finish): 4, or 2 when M <= 32 (R2 - 1) + 16.
// RS = 2 (with R2 = 2): twice the waves, each computing one of the two
// 32-row blocks of its tile (both read the tile's weights; the second read
// hits L2). Every output element sees the same operations in the same
// order as with RS = 1; the waves per SIMD double, which hides more of each
// wave's waits.
template <int R2, int EM, int KH, int RGL = 4, int RS = 1>
__global__ __launch_bounds__(kQmThreads * KH * RS, RS == 2 ? 4 : 1) void qmm_rows_kernel(QmmRowsParams p) {
  static_assert(RS == 1 || (RS == 2 && R2 == 2), "row split: two 32-row blocks");
  constexpr bool dual = EM == E_DUAL_SWIGLU;
  constexpr int ROWS = 32 * R2;
  constexpr int NR2 = R2 / RS;   // row blocks per wave
  constexpr int XBUF = ROWS * kQmSlotsPerRow * 16;   // bytes of one staged quad
  // Dynamic LDS: staged x quads [2][KH], then their group sums [2][KH][4][ROWS].
  extern __shared__ __align__(16) unsigned char qm_lds[];
  auto xbuf = [&](int b, int h) { return qm_lds + (size_t)(b * KH + h) * XBUF; };
  float (*xs)[KH][4][ROWS] = reinterpret_cast<float (*)[KH][4][ROWS]>(qm_lds + 2 * KH * XBUF);
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rs = wave / (kQmWaves * KH);         // row-block share of this wave
  const int wk = wave - rs * (kQmWaves * KH);
  const int kh = wk / kQmWaves;                  // K half of this wave
  const int wt = wk % kQmWaves;                  // the wave's tile slot in the group
  const int rb0 = rs * NR2;                      // first 32-row block of this wave
  const int c32 = lane & 31, kq = lane >> 5;
  const int M = p.M, Q = p.Q;

  // Unit: a column group over all of K, or one K part of a leftover group.
  int g, part = 0, q_lo = 0, q_n = Q;
  const bool split = (int)blockIdx.x >= p.full_groups;
  if (!split) {
    g = blockIdx.x;
  } else {
    const int e = blockIdx.x - p.full_groups;
    g = p.full_groups + e / p.split;
    part = e % p.split;
    q_lo = (part * Q) / p.split;
    q_n = ((part + 1) * Q) / p.split - q_lo;
  }
  // This half's quads [h_lo, h_lo + h_n); the steps run over the first half's count.
  const int h0 = KH == 2 ? (q_n + 1) >> 1 : q_n;
  const int h_lo = q_lo + (kh ? h0 : 0);
  const int h_n = kh ? q_n - h0 : h0;
  const int steps = h0;
  // This wave's tile (column tile ct of matrix mat).
  const int ct = dual ? 2 * g + (wt & 1) : 4 * g + wt;
  const int mat = dual ? (wt >> 1) : 0;
  const bool has_tile = ct < p.ntiles;
  const uint32_t* W = (mat ? p.w1 : p.w0) + (size_t)(has_tile ? ct : 0) * Q * kPackQuadWords;
  const uint32_t* wl = W + lane * 4;
  const uint32_t* sl = W + 1024 + c32 * 4;
  const NibConsts nc = nib_consts();

  auto load_quad = [&](QmQuad& r, int c) {
    // past the half's end (or an empty half): a valid block, never used
    const int q = h_n > 0 ? h_lo + (c < h_n ? c : h_n - 1) : q_lo;
    const size_t off = (size_t)q * kPackQuadWords;
#pragma unroll
    for (int u = 0; u < 4; ++u) r.w[u] = *reinterpret_cast<const uint4*>(wl + off + 256 * u);
    r.sb = *reinterpret_cast<const uint4*>(sl + off);
  };

  // acc[r2]: row block rb0 + r2.
  f32x16 acc[NR2];
#pragma unroll
  for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r2][r] = 0.f;

  // A-operand rows of this lane, per row block: row 32 (rb0 + r2) + c32
  // (chunk kc = 8u + 4 kq + ii of the quad).
  int arow[NR2];
#pragma unroll
  for (int r2 = 0; r2 < NR2; ++r2) {
    const int m = 32 * (rb0 + r2) + c32;
    arow[r2] = m < M ? m : (M - 1);
  }

  auto compute = [&](const QmQuad& r, int buf) {
    float sv[4], cb[4];
    const uint32_t sw[2] = {r.sb.x, r.sb.y}, bw[2] = {r.sb.z, r.sb.w};
    quad_scales<0>(sw, bw, sv, cb);   // the pack stores scales per 64-group for either group size
    const unsigned char* xb = xbuf(buf, kh);
    // The bias term of the quad's four groups, sum_u (b_u - 128 s_u) * sum(x_u),
    // is a (rows x 4) . (4 x 32 columns) product in fp32: two
    // v_mfma_f32_32x32x2_f32 per row block, whose A operand of lane l is the
    // group sum of row l % 32 for group 2p + l / 32, and B operand the lane's
    // column's (b - 128 s) of the same group; same output layout as the
    // bf16 MFMA, so it accumulates into acc directly.
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const float cbk = kq ? cb[2 * pp + 1] : cb[2 * pp];
#pragma unroll
      for (int r2 = 0; r2 < NR2; ++r2)
        acc[r2] = __builtin_amdgcn_mfma_f32_32x32x2f32(xs[buf][kh][2 * pp + kq][32 * (rb0 + r2) + c32], cbk, acc[r2],
                                                       0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t wv[4] = {r.w[u].x, r.w[u].y, r.w[u].z, r.w[u].w};
      f32x16 G[NR2];
#pragma unroll
      for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
        for (int i = 0; i < 16; ++i) G[r2][i] = 0.f;
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const bf16x8 b = nibbles_to_bf16(wv[ii], nc);
        const int kc = 8 * u + 4 * kq + ii;
#pragma unroll
        for (int r2 = 0; r2 < NR2; ++r2) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(xb + 16 * xslot(arow[r2], kc));
          G[r2] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, G[r2], 0, 0, 0);
        }
      }
#pragma unroll
      for (int r2 = 0; r2 < NR2; ++r2) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // Rows 32 (rb0 + r2) + 8 j .. + 7 of register group j: groups past
          // the last RGL of the last row block hold no output row (M <= 32 (R2 - 1) + 8 RGL).
          if (rb0 + r2 == R2 - 1 && j >= RGL) continue;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int r = 4 * j + i;
            acc[r2][r] = fmaf(sv[u], G[r2][r], acc[r2][r]);
          }
        }
      }
    }
  };

  // Group sums of staged quad `buf` of each half: thread t < 4M of half h
  // (among the waves of row share 0) sums row t % M, group t / M (4M <= the
  // half's threads: one sum at most, its row and group fixed for the whole
  // launch).
  const int gs_t = tid % kQmThreads;
  const int gs_u = gs_t / M, gs_m = gs_t - (gs_t / M) * M;
  auto group_sums = [&](int buf, int c) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t one2 = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);
    const int h = kh;
    if (rs != 0) return;
    if (c >= (h ? q_n - h0 : h0)) return;   // this half has no quad c
    if (gs_t < 4 * M) {
      const int u = gs_u, m = gs_m;
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint4 cc = *reinterpret_cast<const uint4*>(xbuf(buf, h) + 16 * xslot(m, 8 * u + j));
        s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, cc.x), one2, s, false);
        s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, cc.y), one2, s, false);
        s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, cc.z), one2, s, false);
        s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, cc.w), one2, s, false);
      }
      xs[buf][h][u][m] = s;
    }
  };

  // Prologue: each half's quad 0 of x, then its first two weight quads.
  QmQuad ring0, ring1;
  const int sw = rs * kQmWaves + wt;   // this wave's index among its half's RS * 4 staging waves
  if (h_n > 0) qm_stage(p, xbuf(0, kh), h_lo, sw, kQmWaves * RS, lane);
  load_quad(ring0, 0);
  load_quad(ring1, 1);
  // One step: quad c of each half from ring slot `cur` and x buffer c & 1;
  // refills `cur` with quad c + 2. At the wait only the newest ring slot (5
  // loads) may be outstanding: this wave's x loads of quad c and its weights
  // have landed.
  auto step = [&](QmQuad& cur, int c) {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(5));
    lds_barrier();   // every wave's x loads of quad c are in LDS
    group_sums(c & 1, c);
    if (c + 1 < h_n) qm_stage(p, xbuf((c + 1) & 1, kh), h_lo + c + 1, sw, kQmWaves * RS, lane);
    lds_barrier();   // group sums visible; buffer (c+1)&1 was last read before the first barrier
    if (c < h_n) compute(cur, c & 1);
    load_quad(cur, c + 2);
  };
  int c = 0;
  do {
    step(ring0, c);
    if (c + 1 < steps) step(ring1, c + 1);
    c += 2;
  } while (c < steps);
  __builtin_amdgcn_s_waitcnt(0);

  if constexpr (KH == 2) {
    // The second half's sums join the first half's, in half order.
    float* red = reinterpret_cast<float*>(qm_lds);   // [4 tile waves][R2*16][64]
    __syncthreads();   // every wave is done with the staged x
    if (kh == 1) {
#pragma unroll
      for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[(wt * R2 * 16 + (rb0 + r2) * 16 + r) * 64 + lane] = acc[r2][r];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r2][r] += red[(wt * R2 * 16 + (rb0 + r2) * 16 + r) * 64 + lane];
    }
  }
  const bool owner = kh == 0;   // the waves that hold the finished sums

  // Output element of acc[r2][r]: row 32 (rb0 + r2) + 8 (r / 4) + 4 kq + r % 4,
  // column 32 ct + c32.
  auto row_of = [&](int r2, int r) { return 32 * (rb0 + r2) + 8 * (r >> 2) + 4 * kq + (r & 3); };

  if (split) {
    // This part's sums, device-coherent, in register order; the last part to
    // arrive adds the parts in part order.
    const int eg = g - p.full_groups;
    float* mine = p.partial + (((size_t)eg * p.split + part) * kQmWaves + wt) * (R2 * 16 * 64);
    if (owner) {
#pragma unroll
      for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          __hip_atomic_store(mine + ((rb0 + r2) * 16 + r) * 64 + lane, acc[r2][r], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const unsigned old = __hip_atomic_fetch_add(p.counters + eg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = old == (unsigned)(p.split - 1);
    }
    __syncthreads();
    if (!s_last) return;
    if (owner) {
#pragma unroll
      for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r2][r] = 0.f;
      for (int pp = 0; pp < p.split; ++pp) {
        const float* src = p.partial + (((size_t)eg * p.split + pp) * kQmWaves + wt) * (R2 * 16 * 64);
        float v[NR2][16];
#pragma unroll
        for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            v[r2][r] = __hip_atomic_load(src + ((rb0 + r2) * 16 + r) * 64 + lane, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[r2][r] += v[r2][r];
      }
    }
    if (tid == 0) __hip_atomic_store(p.counters + eg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  const int col = 32 * ct + c32;
  if constexpr (dual) {
    // The up waves hand their sums to the gate waves of the same columns.
    float* ex = reinterpret_cast<float*>(qm_lds);   // [2 column tiles][R2*16][64]
    __syncthreads();
    if (owner && mat == 1) {
#pragma unroll
      for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
        for (int r = 0; r < 16; ++r) ex[((wt & 1) * R2 * 16 + (rb0 + r2) * 16 + r) * 64 + lane] = acc[r2][r];
    }
    __syncthreads();
    if (owner && mat == 0 && has_tile && col < p.N) {
#pragma unroll
      for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = row_of(r2, r);
          if (m < M) {
            const float up = ex[((wt & 1) * R2 * 16 + (rb0 + r2) * 16 + r) * 64 + lane];
            const float gsl = round_bf(silu_f(round_bf(acc[r2][r])));
            p.y[(size_t)m * p.ldy + col] = f2bf(gsl * round_bf(up));
          }
        }
    }
    return;
  }
  if (!owner || !has_tile || col >= p.N) return;
#pragma unroll
  for (int r2 = 0; r2 < NR2; ++r2)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = row_of(r2, r);
      if (m >= M) continue;
      const size_t o = (size_t)m * p.ldy + col;
      if (EM == E_RESID) {
        p.y[o] = f2bf(round_bf(acc[r2][r]) + bf2f(p.resid[o]));
      } else if (p.yf) {
        p.yf[o] = round_bf(acc[r2][r]);
      } else {
        p.y[o] = f2bf(acc[r2][r]);
      }
    }
}

static size_t rows_lds_bytes(int R2, int KH) {
  const size_t xbuf = (size_t)32 * R2 * kQmSlotsPerRow * 16;
  const size_t stage = 2 * KH * xbuf + (size_t)2 * KH * 4 * 32 * R2 * sizeof(float);
  const size_t red = (size_t)kQmWaves * R2 * 16 * 64 * sizeof(float);   // the halves' reduction / the pair's exchange
  return stage > red ? stage : red;
}

// One launch of qmm_rows_kernel: KH K halves per workgroup, and with two row
// blocks (R2 = 2) optionally one row block per wave (RS = 2). A failure of
// the attribute call surfaces as a launch error, checked by the caller.
template <int R2, int EM, int RGL>
static void launch_rows(const QmmRowsParams& p, int grid, int kh, int rsplit, hipStream_t st) {
  const size_t lds = rows_lds_bytes(R2, kh);
  auto go = [&](auto kern, int threads) {
    if (lds > 65536) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(threads), lds, st, p);
  };
  if constexpr (R2 == 2) {
    if (rsplit) {
      if (kh == 2)
        go(qmm_rows_kernel<2, EM, 2, RGL, 2>, 4 * kQmThreads);
      else
        go(qmm_rows_kernel<2, EM, 1, RGL, 2>, 2 * kQmThreads);
      return;
    }
  }
  if (kh == 2)
    go(qmm_rows_kernel<R2, EM, 2, RGL>, 2 * kQmThreads);
  else
    go(qmm_rows_kernel<R2, EM, 1, RGL>, kQmThreads);
}

struct RowsPlan {
  int groups, full, split, leftover;
};

static RowsPlan rows_plan(int M, int N, int K, int dual) {
  RowsPlan pl;
  const int ntiles = cdiv(N, 32);
  pl.groups = dual ? cdiv(ntiles, 2) : cdiv(ntiles, 4);
  const int cus = device_cus();
  const int Q = K >> 8;
  // The plan depends on N, K and the CU count only, never on M: a row's
  // sums then run in the same order (same K parts, same part sums) at any M,
  // so a request's outputs are bit-identical alone and inside a batch. The
  // partial-sum cap below is sized for the 64-row partials.
  (void)M;
  const int R2 = 2;
  const int E = pl.groups % cus;
  pl.full = pl.groups - E;
  pl.split = 1;
  pl.leftover = 0;
  if (E > 0) {
    int S = cus / E;
    if (S > Q) S = Q;
    // Partial sums cost 4 waves x R2 x 4 KB per part of each leftover group
    // (written, then read once); keep them under half the group's weights.
    const double wbytes = (double)E * 4 * Q * kPackQuadWords * 4;
    const double per_part = (double)E * kQmWaves * R2 * 4096;
    const int cap = (int)(0.5 * wbytes / per_part);
    if (S > cap) S = cap;
    if (S >= 2) {
      pl.split = S;
      pl.leftover = E;
    } else {
      pl.full = pl.groups;
    }
  }
  return pl;
}

static size_t rows_partial_bytes(const RowsPlan& pl, int M) {
  const int R2 = M > 32 ? 2 : 1;
  return ((size_t)pl.leftover * pl.split * kQmWaves * R2 * 16 * 64 * sizeof(float) + 255) & ~(size_t)255;
}

}  // namespace mtp

using namespace mtp;

MTP_API size_t mtp_qmm_workspace_bytes(int M, int N, int K, int dual) {
  if (M < 1 || M > 64 || N < 1 || K < 256 || K % 256) return 0;
  const RowsPlan pl = rows_plan(M, N, K, dual);
  return pl.leftover ? kCounterBytes + rows_partial_bytes(pl, M) : 0;
}

MTP_API int mtp_qmm_affine4_mfma(const mtp_qmm_args* a, void* stream) {
  const char* who = "mtp_qmm_affine4_mfma";
  if (!a || !a->x || !a->w0 || (!a->y && !a->yf)) {
    set_error("%s: null argument block, x, w0 or output", who);
    return MTP_ERR_ARG;
  }
  const int M = a->M, N = a->N, K = a->K;
  const int em = a->emode;
  if (M < 1 || M > 64 || N < 1 || K < 256 || K % 256) {
    set_error("%s: need 1 <= M <= 64, N >= 1, K a multiple of 256 (got M=%d N=%d K=%d)", who, M, N, K);
    return MTP_ERR_ARG;
  }
  if (a->group_size != 64 && a->group_size != 128) {
    set_error("%s: group_size %d unsupported (64 or 128)", who, a->group_size);
    return MTP_ERR_UNSUPPORTED;
  }
  if (em != E_STORE && em != E_RESID && em != E_DUAL_SWIGLU) {
    set_error("%s: emode %d unsupported (0 store, 1 residual, 3 SwiGLU pair)", who, em);
    return MTP_ERR_UNSUPPORTED;
  }
  if ((em == E_DUAL_SWIGLU && (!a->w1 || !a->y)) || (em == E_RESID && (!a->resid || !a->y))) {
    set_error("%s: emode %d needs %s", who, em, em == E_RESID ? "resid and y" : "w1 and y");
    return MTP_ERR_ARG;
  }
  const int ldx = a->ldx > 0 ? a->ldx : K, ldy = a->ldy > 0 ? a->ldy : N;
  if (ldx < K || ldy < N || !rows_aligned16(a->x) || (ldx % 8) || !rows_aligned16(a->w0) || (a->w1 && !rows_aligned16(a->w1))) {
    set_error("%s: x rows must be 16-byte aligned (ldx %% 8 == 0), weights 16-byte aligned", who);
    return MTP_ERR_ARG;
  }
  const int dual = em == E_DUAL_SWIGLU;
  const RowsPlan pl = rows_plan(M, N, K, dual);
  QmmRowsParams p = {};
  p.x = (const uint16_t*)a->x;
  p.w0 = (const uint32_t*)a->w0;
  p.w1 = (const uint32_t*)a->w1;
  p.y = (uint16_t*)a->y;
  p.yf = a->yf;
  p.resid = (const uint16_t*)a->resid;
  p.M = M;
  p.N = N;
  p.K = K;
  p.ldx = ldx;
  p.ldy = ldy;
  p.Q = K >> 8;
  p.ntiles = cdiv(N, 32);
  p.full_groups = pl.full;
  p.split = pl.split;
  if (pl.split > 1) {
    const size_t need = mtp_qmm_workspace_bytes(M, N, K, dual);
    if (!a->ws || a->ws_bytes < need || ((uintptr_t)a->ws & 255)) {
      set_error("%s: a 256-byte aligned workspace of %zu B is needed (mtp_qmm_workspace_bytes), got %zu B", who, need,
                a->ws_bytes);
      return MTP_ERR_WORKSPACE;
    }
    p.counters = reinterpret_cast<uint32_t*>(a->ws);   // the fixed counter area every shape shares
    p.partial = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(a->ws) + kCounterBytes);
  }
  const int grid = pl.full + pl.leftover * pl.split;
  hipStream_t st = (hipStream_t)stream;
  // (the pack repeats a group-128 scale over its two 64-groups, so the kernel
  // is the same for both group sizes). A failure of the attribute call
  // surfaces as a launch error, checked below.
  // Two K halves per workgroup (8 waves, one workgroup per CU by LDS at 64
  // rows) when the grid fits on the CUs at once (q|k|v, o, down at cfg4:
  // 20.8 -> 20.3, 27.6 -> 26.8, 41.1 -> 36.4 us); one (4 waves, two
  // workgroups per CU) when it does not (gate|up 51 vs 57 us, lm_head 168
  // vs 193 us with two halves).
  const int kh_env = env_int_rows("MTPLX_AMD_QMM_HALVES", 0);
  const int kh = kh_env == 1 || kh_env == 2 ? kh_env : (grid <= device_cus() ? 2 : 1);
  // Past 32 rows each wave takes one 32-row block (MTPLX_AMD_QMM_ROWSPLIT=0:
  // both blocks per wave).
  const int rsplit = env_int_rows("MTPLX_AMD_QMM_ROWSPLIT", 1) != 0;
  if (M > 48) {
    if (em == E_STORE) launch_rows<2, E_STORE, 4>(p, grid, kh, rsplit, st);
    else if (em == E_RESID) launch_rows<2, E_RESID, 4>(p, grid, kh, rsplit, st);
    else launch_rows<2, E_DUAL_SWIGLU, 4>(p, grid, kh, rsplit, st);
  } else if (M > 32) {
    if (em == E_STORE) launch_rows<2, E_STORE, 2>(p, grid, kh, rsplit, st);
    else if (em == E_RESID) launch_rows<2, E_RESID, 2>(p, grid, kh, rsplit, st);
    else launch_rows<2, E_DUAL_SWIGLU, 2>(p, grid, kh, rsplit, st);
  } else {
    if (em == E_STORE) launch_rows<1, E_STORE, 4>(p, grid, kh, 0, st);
    else if (em == E_RESID) launch_rows<1, E_RESID, 4>(p, grid, kh, 0, st);
    else launch_rows<1, E_DUAL_SWIGLU, 4>(p, grid, kh, 0, st);
  }
  return launch_check(who);
}
