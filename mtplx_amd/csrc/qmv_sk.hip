// Stream-K 4-bit verify matmul over tile-major packed weights, gfx950.
//
// Work item = (tile unit, k-quad): a tile unit is 32 output columns (both
// matrices of a dual gate/up pair, i.e. 2Q items, in the dual modes), a
// k-quad is 256 input columns. The T = n_tiles * Q(T) items are cut into G
// equal contiguous ranges, one per workgroup and one workgroup per CU, so
// every CU streams the same number of bytes whatever N is (the per-tile
// kernel leaves 96 CUs idle when N = 5120 gives 160 tiles).
//
// Inside a workgroup the range splits into segments, one per tile unit; the
// waves take a segment's items round-robin, stream their packed weights
// through a three-deep register ring and meet in LDS at the end of the
// segment (wave order, deterministic). A segment that is a whole unit goes
// straight to the epilogue. A unit shared with neighbouring workgroups is
// fixed up without waiting: each contributor stores its fp32 partial with
// device-coherent stores, waits for them, then bumps the unit's arrival
// counter; the contributor that arrives last sums all partials in workgroup
// (= K) order, runs the epilogue and resets the counter for the next launch.
// No workgroup ever spins on another.
//
// x is staged once per workgroup, for just the k-quads its range touches
// (at most Q of them), with the same fused producers and A-operand order as
// the per-tile kernel.
#include "qmv_common.hpp"

namespace mtp {

namespace {

constexpr int kSkWaves = 12;   // 768 threads: 3 waves per SIMD, one workgroup per CU

__host__ __device__ __forceinline__ int sk_begin(int T, int G, int g) {
  return (int)((long long)T * g / G);
}
// Workgroup whose range holds item i: the largest g with sk_begin(g) <= i.
__host__ __device__ __forceinline__ int sk_owner(int T, int G, int i) {
  return (int)(((long long)(i + 1) * G - 1) / T);
}

size_t sk_lds_bytes(int nslot, int nseg, int M, int R, int nmat) {
  return xa_bytes(4 * nslot, M) + (size_t)nslot * 4 * 2 * R * 4 + (size_t)nseg * kSkWaves * nmat * M * 32 * 4 +
         (size_t)M * 64 * 4;
}

// Most segments (tile units met) in any workgroup's range of <= per items.
int sk_max_segments(int per, int QT) { return (per + QT - 2) / QT + 1; }

// Workspace layout, the same for every call so that calls of different
// shapes can share one buffer: fp32 partials [2 G][8 rows][64] first, then
// one arrival counter per 32-column tile.
constexpr int kSkMaxRows = 8;

}  // namespace

// Shared with the per-tile kernel's tail split (qmv.hip).
size_t sk_counter_offset(int G) { return (size_t)2 * G * kSkMaxRows * 64 * sizeof(float); }

template <int NW, int R, int XM, int EM>
__global__ __launch_bounds__(NW * 64) void qmv_sk_kernel(QmmParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NT = NW * 64;
  constexpr bool dual = (EM == E_DUAL || EM == E_DUAL_SWIGLU);
  constexpr int NMAT = dual ? 2 : 1;
  constexpr int XSW = 2 * R;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = p.M;
  const int Q = p.K >> 8;
  const int QT = NMAT * Q;
  const int T = p.n_blocks * QT;
  const int G = gridDim.x;
  const int g = blockIdx.x;
  const int r0 = sk_begin(T, G, g);
  const int r1 = sk_begin(T, G, g + 1);
  const int kq0 = r0 % Q;
  const int nslot = (r1 - r0) < Q ? (r1 - r0) : Q;
  const NibConsts nc = nib_consts();

  uint4* xa = reinterpret_cast<uint4*>(smem);                                   // staged x, xa_index()
  const int rstride = xa_row_stride(4 * nslot);
  float* xs = reinterpret_cast<float*>(smem + xa_bytes(4 * nslot, M));          // [nslot*4][XSW]
  float* red = xs + nslot * 4 * XSW;                                            // [nseg][NW][NMAT][M][32]
  float* fin = red + p.chunk * NW * NMAT * M * 32;                              // [M][64]
  __shared__ float s_inv_rms[32];
  __shared__ int s_last;

  const int c32 = lane & 31;
  const int kq = lane >> 5;

  // ---- items of this wave: segment walk (wave-uniform) ----
  auto seg_end = [&](int a) {
    const int e = (a / QT + 1) * QT;
    return e < r1 ? e : r1;
  };
  auto wave_items = [&](int a, int b) { return (a + wave < b) ? (b - a - wave + NW - 1) / NW : 0; };
  int wave_total = 0;
  for (int a = r0; a < r1;) {
    const int b = seg_end(a);
    wave_total += wave_items(a, b);
    a = b;
  }

  struct Item {
    uint4 w[4];
    uint32_t s[2], b[2];
    int mat, slot;
  };
  // Prefetch iterator: item it_r (global index) of unit it_u at position
  // it_w inside the unit; it_b = end of its segment.
  int it_r = 0, it_u = 0, it_w = 0, it_b = 0, pf_left = wave_total;
  auto seek = [&](int a) {   // first item of this wave at or after segment start a
    while (a < r1) {
      const int b = seg_end(a);
      if (a + wave < b) {
        it_r = a + wave;
        it_u = a / QT;
        it_w = it_r - it_u * QT;
        it_b = b;
        return;
      }
      a = b;
    }
  };
  if (wave_total > 0) seek(r0);
  auto load_next = [&](Item& it) {
    const int mat = dual ? (it_w >= Q ? 1 : 0) : 0;
    const int q = it_w - mat * Q;
    const uint32_t* W = mat ? p.w1 : p.w0;
    const uint32_t* base = W + ((size_t)it_u * Q + q) * kPackQuadWords;
#pragma unroll
    for (int u = 0; u < 4; ++u) it.w[u] = *reinterpret_cast<const uint4*>(base + lane * 4 + 256 * u);
    const uint4 sb = *reinterpret_cast<const uint4*>(base + 1024 + c32 * 4);
    it.s[0] = sb.x;
    it.s[1] = sb.y;
    it.b[0] = sb.z;
    it.b[1] = sb.w;
    it.mat = mat;
    it.slot = (q >= kq0) ? q - kq0 : q - kq0 + Q;
    if (pf_left > 1) {   // past the last item the iterator stays put (reloads are never used)
      --pf_left;
      it_r += NW;
      it_w += NW;
      if (it_r >= it_b) seek(it_b);
    }
  };

  // Prologue: the norm statistics, x (and the norm weights) straight into
  // LDS, then all three ring slots, issued back to back; the wait is for
  // everything but the ring loads, so staging overlaps their round trip.
  float ssv[kMaxSsLoads];
  if (XM == X_RMSNORM && p.ss_in && wave < M) ss_prefetch(p, wave, lane, ssv);
  stage_x_issue<NW>(p, xa, rstride, M, Q, kq0, nslot, wave, lane);
  uint4 wpre[kNormPre];
  if (XM == X_RMSNORM) norm_w_prefetch<NW>(p, wpre, Q, kq0, nslot, tid);
  asm volatile("" ::: "memory");
  Item A, B, C;
  load_next(A);   // waves without items reload a valid block; never used
  load_next(B);
  load_next(C);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(15));
  if (XM == X_RMSNORM && wave < M) {   // M <= 8 < NW
    const float v = p.ss_in ? ss_reduce(p, ssv, lane) : row_inv_rms(p, wave, lane);
    if (lane == 0) s_inv_rms[wave] = v;
  }
  __syncthreads();
  stage_x_finish<XM, NW, XSW, true>(p, xa, rstride, xs, wpre, s_inv_rms, M, Q, kq0, nslot, tid);
  __syncthreads();

  // A operands: lanes of rows >= M repeat row c32 % M (their output rows
  // are never stored), so every lane reads its quad at immediate offsets.
  const uint32_t a_lane = (uint32_t)xa_index(kq, c32 % M, M, rstride, 0, 0) * 16;
  const uint32_t x_lane = (uint32_t)((unsigned char*)xs - smem) + 16 * kq;

  float acc0[R], acc1[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc0[r] = acc1[r] = 0.f;

  auto compute = [&](const Item& cr) {
    const int gq = 4 * cr.slot;
    float sv[4], cb[4];
    quad_scales<0>(cr.s, cr.b, sv, cb);
    float t[R];
#pragma unroll
    for (int r = 0; r < R; ++r) t[r] = 0.f;
    quad_mma<R>(smem, a_lane + (uint32_t)gq * 128, x_lane + (uint32_t)gq * (XSW * 4), cr.w, sv, cb, nc, t);
    if (dual && cr.mat) {
#pragma unroll
      for (int r = 0; r < R; ++r) acc1[r] += t[r];
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) acc0[r] += t[r];
    }
  };

  int pend_first = -1, pend_last = -1;   // shared units awaiting their arrival (wave-uniform)

  // End of this wave's part of segment si: its accumulators go to LDS slot
  // [si][wave] - no barrier, the other waves keep streaming.
  auto park = [&](int si) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int m = 8 * (r >> 2) + 4 * kq + (r & 3);
      if (m < M) {
        red[(((si * NW + wave) * NMAT + 0) * M + m) * 32 + c32] = acc0[r];
        if (dual) red[(((si * NW + wave) * NMAT + 1) * M + m) * 32 + c32] = acc1[r];
      }
      acc0[r] = 0.f;
      acc1[r] = 0.f;
    }
  };

  // After the range: segment si = [a, b) of unit u, summed over the waves
  // that had items in it (wave order); a whole unit goes to the epilogue, a
  // shared one stores this workgroup's partial (its arrival comes last).
  auto finalize = [&](int si, int a, int b) {
    const int u = a / QT;
    const bool whole = (a == u * QT) && (b == (u + 1) * QT);
    const int nwv = (b - a) < NW ? (b - a) : NW;
    for (int idx = tid; idx < M * 64; idx += NT) {
      const int m = idx >> 6;
      const int cc = idx & 63;
      const int mat = cc >> 5;
      float v = 0.f;
      if (mat < NMAT)
        for (int w = 0; w < nwv; ++w) v += red[(((si * NW + w) * NMAT + mat) * M + m) * 32 + (cc & 31)];
      fin[idx] = v;
    }
    __syncthreads();
    if (whole) {
      qmm_epilogue<NW, EM>(p, fin, u, M, 0);
    } else {
      const int first_unit = r0 / QT;
      float* part = p.partial + (size_t)(2 * g + (u == first_unit ? 0 : 1)) * (M * 64);
      for (int idx = tid; idx < M * 64; idx += NT)
        __hip_atomic_store(part + idx, fin[idx], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (u == first_unit)
        pend_first = u;
      else
        pend_last = u;
    }
    __syncthreads();   // fin is reused by the next segment
  };

  // Arrival at shared unit u: the contributor that arrives last sums every
  // partial in workgroup (K) order and runs the epilogue.
  auto fixup = [&](int u) {
    if (tid == 0) {
      const int gf = sk_owner(T, G, u * QT);
      const int gl = sk_owner(T, G, (u + 1) * QT - 1);
      const unsigned old = __hip_atomic_fetch_add(p.counters + u, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = (old == (unsigned)(gl - gf)) ? 1 : 0;
    }
    __syncthreads();
    if (s_last) {
      const int gf = sk_owner(T, G, u * QT);
      const int gl = sk_owner(T, G, (u + 1) * QT - 1);
      for (int idx = tid; idx < M * 64; idx += NT) {
        float v = 0.f;
        for (int gg = gf; gg <= gl; ++gg) {
          const int slot = 2 * gg + (sk_begin(T, G, gg) / QT == u ? 0 : 1);
          v += __hip_atomic_load(p.partial + (size_t)slot * (M * 64) + idx, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
        }
        fin[idx] = v;
      }
      __syncthreads();
      qmm_epilogue<NW, EM>(p, fin, u, M, 0);
      if (tid == 0) __hip_atomic_store(p.counters + u, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();   // s_last and fin are reused by the next fix-up
  };

  // Consumer walk over the segments: a wave parks its sums at the end of each
  // segment it has items in and moves on; nothing synchronises the waves
  // until the whole range is done.
  int si = 0, cs_a = r0, cs_b = seg_end(r0);
  int c_left = wave_items(cs_a, cs_b);
  auto skip_empty = [&]() {   // to the next segment holding one of this wave's items
    while (cs_a < r1 && c_left == 0) {
      ++si;
      cs_a = cs_b;
      if (cs_a < r1) {
        cs_b = seg_end(cs_a);
        c_left = wave_items(cs_a, cs_b);
      }
    }
  };
  skip_empty();

  // Single exit at the bottom so the compiler's wait for an item covers only
  // the loads issued before it (the two items behind it stay in flight).
  int done = 0;
  auto step = [&](const Item& cur) {
    if (done < wave_total) {
      compute(cur);
      ++done;
      if (--c_left == 0) {
        park(si);
        skip_empty();
      }
    }
  };
  if (wave_total > 0) {
    do {
      step(A);
      load_next(A);
      step(B);
      load_next(B);
      step(C);
      load_next(C);
    } while (done < wave_total);
  }
  __syncthreads();
  {
    int sj = 0;
    for (int a = r0; a < r1; ++sj) {
      const int b = seg_end(a);
      finalize(sj, a, b);
      a = b;
    }
  }
  // Shared units: make this workgroup's partial stores complete, then arrive.
  if (pend_first >= 0 || pend_last >= 0) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (pend_first >= 0) fixup(pend_first);
    if (pend_last >= 0) fixup(pend_last);
  }
}

// ---------------------------------------------------------------------------
// Host side.

static int sk_grid(int T) {
  const int cus = device_cus();
  return T < cus ? T : cus;
}

size_t qmv_sk_workspace_bytes(int M, int N, int K, int dual) {
  (void)K;
  (void)dual;
  if (M < 1 || N < 1) return 0;
  return sk_counter_offset(device_cus()) + ((size_t)cdiv(N, 32) * 4 + 255) / 256 * 256;
}

template <int R, int XM, int EM>
static void sk_launch_one(const QmmParams& q, int G, size_t lds, hipStream_t st) {
  auto k = qmv_sk_kernel<kSkWaves, R, XM, EM>;
  // A failure here surfaces as a launch error, which the caller checks.
  if (lds > 65536) (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(k, dim3(G), dim3(kSkWaves * 64), lds, st, q);
}

template <int XM, int EM>
static void sk_launch_r(const QmmParams& q, int G, size_t lds, hipStream_t st) {
  sk_launch_one<4, XM, EM>(q, G, lds, st);   // M <= 8 (checked by the caller)
}

template <int XM>
static void sk_launch_e(int em, const QmmParams& q, int G, size_t lds, hipStream_t st) {
  switch (em) {
    case E_STORE: sk_launch_r<XM, E_STORE>(q, G, lds, st); break;
    case E_RESID: sk_launch_r<XM, E_RESID>(q, G, lds, st); break;
    case E_DUAL: sk_launch_r<XM, E_DUAL>(q, G, lds, st); break;
    default: sk_launch_r<XM, E_DUAL_SWIGLU>(q, G, lds, st); break;
  }
}

int qmv_sk_launch(int xm, int em, const QmmParams& p, void* ws, size_t ws_bytes, hipStream_t st) {
  const bool dual = (em == E_DUAL || em == E_DUAL_SWIGLU);
  const int n_blocks = cdiv(p.N, 32);
  const int Q = p.K / 256;
  const int T = n_blocks * Q * (dual ? 2 : 1);
  const int G = sk_grid(T);
  const int per = cdiv(T, G);
  const int nslot = per < Q ? per : Q;
  // Verify widths (M <= 8 rows: one 4-register accumulator row block); wider
  // M keeps the per-tile kernel, whose staged x is shared by fewer items.
  if (p.M > 8 || !p.packed || xm == X_PRE) return MTP_ERR_UNSUPPORTED;
  const int nseg = sk_max_segments(per, Q * (dual ? 2 : 1));
  const size_t lds = sk_lds_bytes(nslot, nseg, p.M, 4, dual ? 2 : 1);
  if (lds > 160 * 1024 - 256) return MTP_ERR_UNSUPPORTED;
  const size_t coff = sk_counter_offset(device_cus());   // G <= CUs
  if (!ws || ws_bytes < coff + (size_t)n_blocks * 4 || ((uintptr_t)ws & 255)) return MTP_ERR_WORKSPACE;
  QmmParams q = p;
  q.n_blocks = n_blocks;
  q.chunk = nseg;   // LDS segment slots
  q.partial = reinterpret_cast<float*>(ws);
  q.counters = reinterpret_cast<uint32_t*>(reinterpret_cast<unsigned char*>(ws) + coff);
  switch (xm) {
    case X_PLAIN: sk_launch_e<X_PLAIN>(em, q, G, lds, st); break;
    case X_SWIGLU: sk_launch_e<X_SWIGLU>(em, q, G, lds, st); break;
    default: sk_launch_e<X_RMSNORM>(em, q, G, lds, st); break;
  }
  return MTP_OK;
}

}  // namespace mtp
