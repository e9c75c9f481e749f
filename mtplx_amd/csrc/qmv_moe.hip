// Expert-gathered streaming matmul over tile-major packed expert weights:
// the routed experts of the MoE sorted chain (mtplx/moe_sorted_gather.py:241
// gather_qmm_rows, :288 swiglu_rows; mtplx/models/qwen4_exp.py:1544-1577) at
// verify-step sizes, where each active expert holds a few sorted rows.
//
// A work unit is (expert, row tile, tile residue r): it stages the
// row tile's x once (gathered through rowmap for the token rows of gate|up,
// contiguous sorted rows for down) and streams the expert's column tiles
// r, r + S, r + 2S, ... through the resident streaming body (qmv_stream.hpp)
// - 1 KB contiguous weight loads, a register ring across the unit's tiles,
// the MFMA quad and the same epilogues as the dense verify matmuls. The
// per-unit cost of staging and ramp is paid once per S-th of an expert
// instead of once per 32-column tile.
//
// Experts are split into two launches by their row count, because LDS (all
// of a row tile's x) sets the occupancy: rows <= 4 run with R = 4 and LDS
// for four rows (four 4-wave workgroups per CU at K = 4096); rows >= 5 run
// 16-row tiles with R = 8 and 8-wave workgroups. The stack is packed in
// layout 1 (32x32x16 quads) or layout 2 (16x16x32 quads: the 4-row form for
// the first class, the 16-row form for the second). Each workgroup first lists
// its class's experts in LDS from the device's active list (one parallel
// pass), sizes the units so that about one round of them covers the grid,
// then takes units grid-stride.
#include "qmv_kernels.hpp"

#include <climits>

namespace mtp {

struct MoeUnits {
  int tpu;               // tiles per unit; 0: from the class's expert count (about one unit per CU)
  int cus;               // compute units of the device
  int rows_tile;         // rows per row tile
  int row_tiles;         // row tiles per expert (of the largest possible)
  int m_lo, m_hi;        // this launch's experts: m_lo <= rows <= m_hi
  long long w_estride;   // uint32 words between consecutive experts' packed tiles
  long long w1_off;      // E_DUAL_SWIGLU: words from an expert's gate tiles to its up tiles
};

constexpr int kMoeList = 512;   // experts of a class listed in LDS (more: read from memory per unit)

// The pack holds each 64-k group's scale and bias (group 128 repeats them),
// so the body runs with GSH = 0 for either group size.
template <int NW, int R, int EM, int NRT, bool MF>
__global__ __launch_bounds__(NW * 64) void moe_stream_kernel(QmmParams p, MoeUnits mu) {
  constexpr int NT = NW * 64;
  // This class's experts, in active-list order: (e | rows << 16, first row).
  __shared__ int s_er[kMoeList], s_e0[kMoeList];
  __shared__ int s_wcnt[NW];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n_active = p.active[0];
  const bool listed = n_active <= kMoeList;
  int n_class = 0;
  if (listed) {
    for (int c0 = 0; c0 < n_active; c0 += NT) {
      const int t = c0 + tid;
      int e = 0, e0 = 0, rows = 0;
      if (t < n_active) {
        e = p.active[1 + t];
        e0 = p.expert_off[e];
        rows = p.expert_off[e + 1] - e0;
      }
      const bool member = t < n_active && rows >= mu.m_lo && rows <= mu.m_hi;
      const unsigned long long bal = __ballot(member);
      if (lane == 0) s_wcnt[wave] = __popcll(bal);
      __syncthreads();
      int base = n_class, total = 0;
      for (int w = 0; w < NW; ++w) {
        if (w < wave) base += s_wcnt[w];
        total += s_wcnt[w];
      }
      if (member) {
        const int at = base + __popcll(bal & ((1ull << lane) - 1ull));
        s_er[at] = e | (rows << 16);
        s_e0[at] = e0;
      }
      n_class += total;
      __syncthreads();
    }
  }
  const int n_exp = listed ? n_class : n_active;
  // Tiles per unit, unless fixed: about one unit per CU. Long units pay the
  // staging and ramp once for many tiles; measured at the cfg5 shape, one
  // long unit per CU streams faster than several short ones per CU.
  int tpu = mu.tpu;
  if (tpu <= 0) {
    const long long streams = (long long)n_exp * mu.row_tiles * p.n_blocks;
    tpu = (int)((streams + mu.cus - 1) / mu.cus);
    if (tpu < 1) tpu = 1;
  }
  const int S = (p.n_blocks + tpu - 1) / tpu;
  const int per_expert = mu.row_tiles * S;
  const int units = n_exp * per_expert;
  for (int u = blockIdx.x; u < units; u += gridDim.x) {
    const int slot = u / per_expert;
    const int rem = u - slot * per_expert;
    const int rt = rem / S;
    const int r = rem - rt * S;
    int e, e0, rows;
    if (listed) {
      e = s_er[slot] & 0xffff;
      rows = s_er[slot] >> 16;
      e0 = s_e0[slot];
    } else {
      e = p.active[1 + slot];
      e0 = p.expert_off[e];
      rows = p.expert_off[e + 1] - e0;
      if (rows < mu.m_lo || rows > mu.m_hi) continue;   // uniform over the workgroup
    }
    // uniform over the workgroup: keep the unit's scalars in SGPRs
    e = __builtin_amdgcn_readfirstlane(e);
    e0 = __builtin_amdgcn_readfirstlane(e0);
    rows = __builtin_amdgcn_readfirstlane(rows);
    const int t0 = rt * mu.rows_tile;
    if (t0 >= rows) continue;
    QmmParams q = p;
    q.M = min(mu.rows_tile, rows - t0);
    if (p.rowmap)
      q.rowmap = p.rowmap + e0 + t0;
    else
      q.x = p.x + (size_t)(e0 + t0) * p.ldx;
    q.w0 = p.w0 + e * mu.w_estride;
    if (EM == E_DUAL_SWIGLU) q.w1 = q.w0 + mu.w1_off;
    q.y0 = p.y0 + (size_t)(e0 + t0) * p.ldy;
    qmv_stream_body<NW, R, X_PLAIN, EM, 0, true, MF, NRT>(q, r, S, NoHook{});
    __syncthreads();   // the next unit restages LDS
  }
}

template <int NW, int R, int EM, bool MF>
static int moe_launch(const QmmParams& p, const MoeUnits& mu, int rows_lds, hipStream_t st) {
  auto k = moe_stream_kernel<NW, R, EM, 2, MF>;
  const size_t lds = stream_lds(p.K >> 8, rows_lds, NW);
  if (lds + 2 * kMoeList * sizeof(int) + 512 > kLdsMax) return MTP_ERR_UNSUPPORTED;   // + the static expert list
  if (lds > 65536) (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k, NW * 64, lds) != hipSuccess || occ < 1) occ = 1;
  hipLaunchKernelGGL(k, dim3((unsigned)(occ * device_cus())), dim3(NW * 64), lds, st, p, mu);
  return MTP_OK;
}

// row_class: 0 both launches, 1 only the experts with 1-4 rows, 2 only those
// with more (two streams can then run the classes side by side).
template <int EM, bool MF>
static int moe_launch_classes(const QmmParams& p, MoeUnits mu, int max_rows, hipStream_t st, int row_class) {
  // rows <= 4: one row tile, LDS for four rows
  mu.rows_tile = 4;
  mu.row_tiles = 1;
  mu.m_lo = 1;
  mu.m_hi = 4;
  // gate|up: six tiles per unit (graph-free cfg5 steps measured 14.3 ms at
  // 4-6, 14.7 at 8, 15.0 at 10 and 16.0 with one unit per CU). down, whose
  // tiles are 4x smaller at K = 1536: twelve (cfg5 graph steps with the side
  // stream 12.67-12.69 ms against 12.73-12.76 at six, 12.93-12.96 at nine,
  // 12.99 at eighteen).
  mu.tpu = EM == E_STORE ? env_int("MTPLX_AMD_MOE_TILES_SMALL_DOWN", 12) : env_int("MTPLX_AMD_MOE_TILES_SMALL", 6);
  if (row_class != 2) {
    const int rc = moe_launch<4, 4, EM, MF>(p, mu, 4, st);
    if (rc != MTP_OK) return rc;
  }
  if (max_rows <= 4 || row_class == 1) return MTP_OK;
  // rows >= 5: 16-row tiles (the rows of an expert past 16 in further
  // tiles). 8-row tiles on 4-wave workgroups measured the same at cfg5.
  mu.rows_tile = 16;
  mu.row_tiles = cdiv(max_rows, 16);
  mu.m_lo = 5;
  mu.m_hi = INT_MAX;
  // three tiles per unit (cfg5 graph steps with the side stream: 12.42-12.43
  // ms at three, 12.43-12.47 at four, 12.59 at five, 12.67-12.69 with about
  // one unit per CU, 13.0 at eight)
  mu.tpu = env_int("MTPLX_AMD_MOE_TILES_LARGE", 3);
  return moe_launch<8, 8, EM, MF>(p, mu, 16, st);
}

}  // namespace mtp

using namespace mtp;

// Packed form of mtp_gather_qmv_affine4: wp is mtp_pack_affine4 (layout 1)
// or mtp_pack_affine4_mf16 (layout 2) of the [E * rows_per_expert, K] matrix
// (expert e's rows at e * rows_per_expert; for the fused pair its N gate rows
// then its N up rows).
static int gather_packed_run(const void* x, const uint32_t* rowmap, const int32_t* expert_off, const int32_t* active,
                             const void* wp, void* y, int max_rows_per_expert, int E, int N, int K, int group_size,
                             int emode, int rows_per_expert, int row_class, int layout, void* stream,
                             const char* who) {
  if (row_class < 0 || row_class > 2) {
    set_error("%s: row_class %d (0 all experts, 1 those with 1-4 rows, 2 those with more)", who, row_class);
    return MTP_ERR_ARG;
  }
  if (!x || !expert_off || !active || !wp || !y || max_rows_per_expert < 1 || max_rows_per_expert > 32767 || E < 1 ||
      E > 65535 || N < 32 || K < 256) {
    set_error("%s: bad arguments", who);
    return MTP_ERR_ARG;
  }
  if (K % 256 || N % 32 || rows_per_expert % 32 ||
      rows_per_expert < (emode == E_DUAL_SWIGLU ? 2 * N : N)) {
    set_error("%s: need K %% 256 == 0, N and rows_per_expert multiples of 32, rows_per_expert >= %s (got N=%d "
              "K=%d rows_per_expert=%d)", who, emode == E_DUAL_SWIGLU ? "2N" : "N", N, K, rows_per_expert);
    return MTP_ERR_ARG;
  }
  if (group_size != 64 && group_size != 128) {
    set_error("%s: group_size %d unsupported", who, group_size);
    return MTP_ERR_UNSUPPORTED;
  }
  if (emode != E_STORE && emode != E_DUAL_SWIGLU) {
    set_error("%s: epilogue %d unsupported (store or dual-swiglu)", who, emode);
    return MTP_ERR_UNSUPPORTED;
  }
  if (((uintptr_t)x & 15) || ((uintptr_t)wp & 15) || ((uintptr_t)y & 3)) {
    set_error("%s: x and the packed weights must be 16-byte aligned", who);
    return MTP_ERR_ARG;
  }
  QmmParams p = {};
  p.x = (const uint16_t*)x;
  p.w0 = (const uint32_t*)wp;
  p.y0 = (uint16_t*)y;
  p.rowmap = rowmap;
  p.expert_off = expert_off;
  p.active = active;
  p.M = 1;
  p.N = N;
  p.K = K;
  p.gs = group_size;
  p.ldx = K;
  p.ldy = N;
  p.eps = 1e-6f;
  p.packed = layout;
  p.n_blocks = N / 32;
  p.tail_split = 1;
  MoeUnits mu = {};
  mu.cus = device_cus();
  const long long tile_words = (long long)(K / 256) * kPackQuadWords;
  mu.w_estride = (long long)(rows_per_expert / 32) * tile_words;
  mu.w1_off = (long long)(N / 32) * tile_words;
  hipStream_t st = (hipStream_t)stream;
  int rc;
  if (emode == E_DUAL_SWIGLU)
    rc = layout == 2 ? moe_launch_classes<E_DUAL_SWIGLU, true>(p, mu, max_rows_per_expert, st, row_class)
                     : moe_launch_classes<E_DUAL_SWIGLU, false>(p, mu, max_rows_per_expert, st, row_class);
  else
    rc = layout == 2 ? moe_launch_classes<E_STORE, true>(p, mu, max_rows_per_expert, st, row_class)
                     : moe_launch_classes<E_STORE, false>(p, mu, max_rows_per_expert, st, row_class);
  if (rc != MTP_OK) {
    set_error("%s: K=%d needs more LDS than a workgroup has", who, K);
    return rc;
  }
  return launch_check(who);
}

MTP_API int mtp_gather_qmv_affine4_packed(const void* x, const uint32_t* rowmap, const int32_t* expert_off,
                                          const int32_t* active, const void* wp, void* y, int max_rows_per_expert,
                                          int E, int N, int K, int group_size, int emode, int rows_per_expert,
                                          void* stream) {
  return gather_packed_run(x, rowmap, expert_off, active, wp, y, max_rows_per_expert, E, N, K, group_size, emode,
                           rows_per_expert, 0, 1, stream, "mtp_gather_qmv_affine4_packed");
}

MTP_API int mtp_gather_qmv_affine4_packed_rows(const void* x, const uint32_t* rowmap, const int32_t* expert_off,
                                               const int32_t* active, const void* wp, void* y,
                                               int max_rows_per_expert, int E, int N, int K, int group_size, int emode,
                                               int rows_per_expert, int row_class, void* stream) {
  return gather_packed_run(x, rowmap, expert_off, active, wp, y, max_rows_per_expert, E, N, K, group_size, emode,
                           rows_per_expert, row_class, 1, stream, "mtp_gather_qmv_affine4_packed_rows");
}

MTP_API int mtp_gather_qmv_affine4_packed_mf16(const void* x, const uint32_t* rowmap, const int32_t* expert_off,
                                               const int32_t* active, const void* wp, void* y,
                                               int max_rows_per_expert, int E, int N, int K, int group_size, int emode,
                                               int rows_per_expert, int row_class, void* stream) {
  return gather_packed_run(x, rowmap, expert_off, active, wp, y, max_rows_per_expert, E, N, K, group_size, emode,
                           rows_per_expert, row_class, 2, stream, "mtp_gather_qmv_affine4_packed_mf16");
}
