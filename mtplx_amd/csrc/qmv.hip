// 4-bit affine (group 64/128) quantized skinny GEMM for verify rows, gfx950.
//
//   y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/gs] + b[n, k/gs])
//
// Weight format is the reference's (mtplx/verify_kernels.py:69-88, :372):
// uint32 [N, K/8] with little-endian nibbles, bf16 scales/biases [N, K/gs].
//
// Design (MI355X-first, not a translation of the Metal kernels):
//  * At M <= 32 a VALU dot product cannot keep up with 8 TB/s of nibbles, so
//    the contraction runs on the matrix cores even for skinny M:
//    v_mfma_f32_32x32x16_bf16 with A = activations (rows m, zero-padded to 32)
//    and B = nibbles.
//  * Nibbles become bf16 operands with one AND-OR each: (w & 0x000F000F) |
//    0x43004300 is the bf16 pair (128 + q_lo, 128 + q_hi), exact. The MFMA
//    therefore yields G = sum x*(128+q) per 64-wide group, and the group is
//    finished on the VALU as s*G + (b - 128*s)*sum(x) with sum(x) per group
//    precomputed while staging x. Dequantised weights are never rounded.
//  * A workgroup owns one 32-column tile; its waves split K by quads (256 k)
//    and meet in LDS in wave order (deterministic). Weights stream either in
//    the reference layout or in the tile-major packed layout (1 KB contiguous
//    per wave load).
//  * Activations are staged once per workgroup into LDS in the MFMA A-operand
//    order, with optional fused producers: SwiGLU (silu(gate)*up) or RMSNorm.
#include "qmv_kernels.hpp"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

namespace mtp {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

// Expert-gathered matmul: work items (active expert slot, row tile, column
// tile) in slot-major order, taken grid-stride by a bounded grid. The number
// of active experts is known only on the device; a grid over every expert
// slot would dispatch mostly empty workgroups (e.g. 63 of 256 experts
// active), while this one stops at the active items.
template <int R, int XM, int EM, int GSH>
__global__ __launch_bounds__(kThreads) void gather_qmm4_kernel(QmmParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int per_slot = p.n_blocks * p.row_tiles;
  const int items = p.active[0] * per_slot;
  for (int w = blockIdx.x; w < items; w += gridDim.x) {
    const int slot = w / per_slot;
    const int rem = w - slot * per_slot;
    const int rt = rem / p.n_blocks;
    const int nb = rem - rt * p.n_blocks;
    const int e = p.active[1 + slot];
    const int r0 = p.expert_off[e] + 32 * rt;
    const int r1 = p.expert_off[e + 1];
    if (r0 < r1) {
      const int M = min(32, r1 - r0);
      qmm_body<4, R, XM, EM, GSH>(p, smem, nb, M, r0, (long long)e * p.w_estride, (long long)e * p.s_estride);
      qmm_epilogue<4, EM>(p, fin_of(smem, 4), nb, M, r0);
    }
    __syncthreads();   // the next item restages LDS
  }
}

int device_cus() {
  static thread_local int dev_cached = -1, cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev != dev_cached) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    dev_cached = dev;
  }
  return cus;
}

static void launch_x(int xm, int em, int gsh, const QmmParams& p, const Plan& pl, hipStream_t st) {
  switch (xm) {
    case X_PLAIN: qmv_launch_plain(em, gsh, p, pl, st); break;
    case X_SWIGLU: qmv_launch_swiglu(em, gsh, p, pl, st); break;
    case X_PRE: qmv_launch_pre(em, gsh, p, pl, st); break;
    default: qmv_launch_rmsnorm(em, gsh, p, pl, st); break;
  }
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

// Shared validation + dispatch for every qmm entry point.
// Argument checks shared by every streaming-matmul entry point.
static int qmm_check(int xm, int em, const QmmParams& p, const char* who) {
  if (p.M < 1 || p.M > 32 || p.N < 1 || p.K < 256) {
    set_error("%s: need 1<=M<=32, N>=1, K>=256 (got M=%d N=%d K=%d)", who, p.M, p.N, p.K);
    return MTP_ERR_ARG;
  }
  if (p.K % 256) {
    set_error("%s: K=%d must be a multiple of 256", who, p.K);
    return MTP_ERR_ARG;
  }
  if (p.gs != 64 && p.gs != 128) {
    set_error("%s: group_size %d unsupported (64 or 128)", who, p.gs);
    return MTP_ERR_UNSUPPORTED;
  }
  if (!p.x || !p.w0 || (!p.packed && (!p.s0 || !p.b0)) || (!p.y0 && !p.yf && em != E_ROPE_QKV)) {
    set_error("%s: null pointer argument", who);
    return MTP_ERR_ARG;
  }
  if (p.ldx < p.K || p.ldx % 8 || !aligned16(p.x) || !aligned16(p.w0) ||
      (!p.packed && (((uintptr_t)p.s0 & 7) || ((uintptr_t)p.b0 & 7))) ||
      (p.x2 && xm == X_SWIGLU && !aligned16(p.x2))) {
    set_error("%s: x rows/weights must be 16-byte and scales/biases 8-byte aligned, ldx %% 8 == 0 (ldx=%d)", who,
              p.ldx);
    return MTP_ERR_ARG;
  }
  const bool dual = (em == E_DUAL || em == E_DUAL_SWIGLU);
  if (dual && (!p.w1 || !aligned16(p.w1) ||
               (!p.packed && (!p.s1 || !p.b1 || ((uintptr_t)p.s1 & 7) || ((uintptr_t)p.b1 & 7))))) {
    set_error("%s: dual mode needs a second aligned weight triple", who);
    return MTP_ERR_ARG;
  }
  if (em == E_DUAL && !p.y1) {
    set_error("%s: dual mode needs a second output", who);
    return MTP_ERR_ARG;
  }
  if (em == E_RESID && !p.resid) {
    set_error("%s: residual mode needs a residual input", who);
    return MTP_ERR_ARG;
  }
  if ((xm == X_SWIGLU || xm == X_RMSNORM) && !p.x2) {
    set_error("%s: fused producer needs its second input", who);
    return MTP_ERR_ARG;
  }
  if (xm == X_PRE && (!p.x_sums || !p.packed)) {
    set_error("%s: xmode 3 needs the input's 32-column sums and packed weights", who);
    return MTP_ERR_ARG;
  }
  if (p.ldy < p.N) {
    set_error("%s: ldy=%d < N=%d", who, p.ldy, p.N);
    return MTP_ERR_ARG;
  }
  if (p.packed < 0 || p.packed > 2) {
    set_error("%s: packed=%d (0 = MLX layout, 1, 2 = packed layouts)", who, p.packed);
    return MTP_ERR_ARG;
  }
  if (p.packed == 2 && p.M > 16) {
    set_error("%s: packed layout 2 (16x16x32) serves M <= 16 only (M=%d)", who, p.M);
    return MTP_ERR_UNSUPPORTED;
  }
  if (em == E_ROPE_QKV) {
    const int D = p.rope_D;
    if (!p.packed || p.M > 16 || (xm != X_PLAIN && xm != X_RMSNORM) || !p.q_start || !p.q_out || !p.k_cache ||
        !p.v_cache || D < 32 || D % 32 || p.rope_L < 1 || p.M % p.rope_L || p.rope_Hq < 1 || p.rope_Hkv < 1 ||
        p.N != (p.rope_Hq + 2 * p.rope_Hkv) * D || p.rope_cap < 1 || !(p.rope_log2_base > 0.f) ||
        (p.rope_blocked && (p.rope_cap % 32 || D != 128))) {
      set_error("%s: RoPE epilogue needs packed weights in RoPE tile order, M<=16 (a multiple of L), plain or "
                "RMSNorm x, N=(Hq+2Hkv)*D with D%%32==0, base>1, non-null q_start/q_out/caches "
                "(blocked caches: D=128, cap%%32==0)", who);
      return MTP_ERR_ARG;
    }
  }
  return MTP_OK;
}

static int qmm_dispatch(int xm, int em, QmmParams p, void* ws, size_t ws_bytes, hipStream_t st,
                        const char* who, int schedule = 0) {
  const int rc = qmm_check(xm, em, p, who);
  if (rc != MTP_OK) return rc;
  if (em == E_ROPE_QKV) {
    Plan pl = make_plan(p.M, p.N, p.K);
    if (!pl.resident) {
      set_error("%s: packed weights need all of x in LDS (M=%d, K=%d too large)", who, p.M, p.K);
      return MTP_ERR_UNSUPPORTED;
    }
    p.chunk = pl.chunk;
    p.n_blocks = pl.n_blocks;
    qmv_launch_rope_qkv(xm, p, pl, st);
    return launch_check(who);
  }
  if (schedule != 0) {
    set_error("%s: schedule %d unsupported (0 = the per-tile kernel)", who, schedule);
    return MTP_ERR_UNSUPPORTED;
  }
  if (p.packed && ws) {
    const size_t need = tail_workspace_bytes(p.M, p.N);
    if (ws_bytes < need || ((uintptr_t)ws & 255)) {
      set_error("%s: workspace of %zu B (256-B aligned) needed, got %zu B", who, need, ws_bytes);
      return MTP_ERR_WORKSPACE;
    }
    // Per-tile kernel with its leftover tiles split over all CUs (counters:
    // one per leftover tile, fewer than the CUs).
    p.tail_ok = 1;
    p.counters = reinterpret_cast<uint32_t*>(ws);
    p.partial = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(ws) + kCounterBytes);
  }
  Plan pl = make_plan(p.M, p.N, p.K);
  if (p.packed && !pl.resident) {
    // All of x does not fit in LDS (M >= 16 at large K): split K into parts
    // whose share of x does, one part per workgroup over a group of tiles;
    // the parts meet through the workspace.
    const int S = full_split_parts(p.M, p.K, pl.nw);
    const size_t need = full_split_ws_bytes(p.M, p.N, p.K, pl.nw);
    if (S < 2 || !ws || ws_bytes < need || ((uintptr_t)ws & 255) || pl.n_blocks > kMaxCounters) {
      set_error("%s: packed weights with x too large for LDS (M=%d, K=%d) need a 256-B aligned workspace of %zu B "
                "(mtp_qmv_workspace_bytes) and N <= %d", who, p.M, p.K, need, 32 * kMaxCounters);
      return ws ? MTP_ERR_WORKSPACE : MTP_ERR_UNSUPPORTED;
    }
    pl.split = S;
    pl.xq = cdiv(p.K >> 8, S);
    pl.lds = stream_lds(pl.xq, p.M, pl.nw);
    p.tail_ok = 1;
    p.counters = reinterpret_cast<uint32_t*>(ws);   // one per tile
    p.partial = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(ws) + kCounterBytes);
  }
  p.chunk = pl.chunk;
  launch_x(xm, em, p.gs == 64 ? 0 : 1, p, pl, st);
  return launch_check(who);
}

int qmm_check_args(int xm, int em, const QmmParams& p, const char* who) { return qmm_check(xm, em, p, who); }
size_t stream_lds_bytes(int chunk_q, int M, int nw) { return stream_lds(chunk_q, M, nw); }

static QmmParams base_params(const void* x, const void* w, const void* s, const void* b, void* y, int M,
                             int N, int K, int gs) {
  QmmParams p = {};
  p.x = (const uint16_t*)x;
  p.w0 = (const uint32_t*)w;
  p.s0 = (const uint16_t*)s;
  p.b0 = (const uint16_t*)b;
  p.y0 = (uint16_t*)y;
  p.M = M;
  p.N = N;
  p.K = K;
  p.gs = gs;
  p.ldx = K;
  p.ldy = N;
  p.eps = 1e-6f;
  return p;
}

}  // namespace mtp

using namespace mtp;

MTP_API const char* mtp_last_error(void) { return g_err; }

MTP_API int mtp_qmv_rope_fusable(int M, int N, int K) {
  // The RoPE epilogue (emode 4) takes up to 16 rows with all of x in LDS.
  if (M < 1 || M > 16 || N < 1 || K < 256 || K % 256) return 0;
  return make_plan(M, N, K).resident ? 1 : 0;
}

MTP_API size_t mtp_qmv_workspace_bytes(int M, int N, int K, int dual) {
  // Packed weights only: the tail split (fp32 partials of the tiles shared by
  // several workgroups, then arrival counters) and, when all of x does not
  // fit in LDS, the full K split.
  (void)dual;
  size_t b = tail_workspace_bytes(M, N);
  if (M >= 1 && N >= 1 && K >= 256 && K % 256 == 0 && M <= 32) {
    const Plan pl = make_plan(M, N, K);
    if (!pl.resident && full_split_parts(M, K, pl.nw) >= 2) {
      const size_t f = full_split_ws_bytes(M, N, K, pl.nw);
      if (f > b) b = f;
    }
  }
  return b;
}

MTP_API int mtp_qmv_affine4(const void* x, const void* w, const void* scales, const void* biases, void* y,
                            int M, int N, int K, int group_size, void* ws, size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w, scales, biases, y, M, N, K, group_size);
  return qmm_dispatch(X_PLAIN, E_STORE, p, ws, ws_bytes, (hipStream_t)stream, "mtp_qmv_affine4");
}

MTP_API int mtp_qmv_affine4_residual(const void* x, const void* w, const void* scales, const void* biases,
                                     const void* resid, void* y, float* ss_out, int M, int N, int K, int group_size,
                                     void* ws, size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w, scales, biases, y, M, N, K, group_size);
  p.resid = (const uint16_t*)resid;
  p.ss_out = ss_out;
  return qmm_dispatch(X_PLAIN, E_RESID, p, ws, ws_bytes, (hipStream_t)stream, "mtp_qmv_affine4_residual");
}

MTP_API int mtp_qmv_affine4_dual(const void* x, const void* w0, const void* s0, const void* b0, const void* w1,
                                 const void* s1, const void* b1, void* y0, void* y1, int M, int N, int K,
                                 int group_size, int swiglu, void* ws, size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w0, s0, b0, y0, M, N, K, group_size);
  p.w1 = (const uint32_t*)w1;
  p.s1 = (const uint16_t*)s1;
  p.b1 = (const uint16_t*)b1;
  p.y1 = (uint16_t*)y1;
  return qmm_dispatch(X_PLAIN, swiglu ? E_DUAL_SWIGLU : E_DUAL, p, ws, ws_bytes, (hipStream_t)stream,
                      "mtp_qmv_affine4_dual");
}

MTP_API int mtp_qmv_affine4_swiglu_in(const void* gate, const void* up, const void* w, const void* scales,
                                      const void* biases, const void* resid, void* y, int M, int N, int K,
                                      int group_size, void* ws, size_t ws_bytes, void* stream) {
  QmmParams p = base_params(gate, w, scales, biases, y, M, N, K, group_size);
  p.x2 = (const uint16_t*)up;
  p.resid = (const uint16_t*)resid;
  return qmm_dispatch(X_SWIGLU, resid ? E_RESID : E_STORE, p, ws, ws_bytes, (hipStream_t)stream,
                      "mtp_qmv_affine4_swiglu_in");
}

MTP_API int mtp_qmv_affine4_rmsnorm_in(const void* x, const void* norm_w, const float* ss_in, float eps, const void* w,
                                       const void* scales, const void* biases, void* y, int M, int N, int K,
                                       int group_size, void* ws, size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w, scales, biases, y, M, N, K, group_size);
  p.x2 = (const uint16_t*)norm_w;
  p.eps = eps;
  p.ss_in = ss_in;
  p.ss_parts = cdiv(K, 32);
  return qmm_dispatch(X_RMSNORM, E_STORE, p, ws, ws_bytes, (hipStream_t)stream, "mtp_qmv_affine4_rmsnorm_in");
}

MTP_API int mtp_qmv_affine4_rmsnorm_f32(const void* x, const void* norm_w, const float* ss_in, float eps, const void* w,
                                        const void* scales, const void* biases, float* y, int M, int N, int K,
                                        int group_size, void* ws, size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w, scales, biases, nullptr, M, N, K, group_size);
  p.x2 = (const uint16_t*)norm_w;
  p.eps = eps;
  p.ss_in = ss_in;
  p.ss_parts = cdiv(K, 32);
  p.yf = y;
  return qmm_dispatch(norm_w ? X_RMSNORM : X_PLAIN, E_STORE, p, ws, ws_bytes, (hipStream_t)stream,
                      "mtp_qmv_affine4_rmsnorm_f32");
}

MTP_API int mtp_qmv_affine4_rmsnorm_dual(const void* x, const void* norm_w, const float* ss_in, float eps, const void* w0,
                                         const void* s0, const void* b0, const void* w1, const void* s1,
                                         const void* b1, void* y, int M, int N, int K, int group_size, void* ws,
                                         size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w0, s0, b0, y, M, N, K, group_size);
  p.x2 = (const uint16_t*)norm_w;
  p.eps = eps;
  p.ss_in = ss_in;
  p.ss_parts = cdiv(K, 32);
  p.w1 = (const uint32_t*)w1;
  p.s1 = (const uint16_t*)s1;
  p.b1 = (const uint16_t*)b1;
  return qmm_dispatch(X_RMSNORM, E_DUAL_SWIGLU, p, ws, ws_bytes, (hipStream_t)stream,
                      "mtp_qmv_affine4_rmsnorm_dual");
}

// ---------------------------------------------------------------------------
// Diagnostic: lane layout of v_mfma_f32_32x32x16_bf16. A[i][k] = i+1 on the
// diagonal block (k == i % 16), B[k][j] = 1 for k == j % 16 gives
// D[i][j] = (i+1) * [i%16 == j%16]. out[lane*16 + r] = D register r of lane.
__global__ void mfma_layout_probe(float* out) {
  const int l = threadIdx.x;
  bf16x8 a = {}, b = {};
  // Lane l supplies A row (l%32), k slots 8*(l/32)+e; B column (l%32), same k slots.
  uint16_t av[8], bv[8];
  for (int e = 0; e < 8; ++e) {
    const int k = 8 * (l >> 5) + e;
    av[e] = (k == (l & 31) % 16) ? f2bf((float)((l & 31) + 1)) : 0;
    bv[e] = (k == (l & 31) % 16) ? f2bf(1.f) : 0;
  }
  a = __builtin_bit_cast(bf16x8, av);
  b = __builtin_bit_cast(bf16x8, bv);
  f32x16 d = {};
  d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, d, 0, 0, 0);
  for (int r = 0; r < 16; ++r) out[l * 16 + r] = d[r];
}

MTP_API int mtp_probe_mfma_layout(float* out, void* stream) {
  if (!out) {
    set_error("mtp_probe_mfma_layout: null output");
    return MTP_ERR_ARG;
  }
  hipLaunchKernelGGL(mfma_layout_probe, dim3(1), dim3(64), 0, (hipStream_t)stream, out);
  return launch_check("mtp_probe_mfma_layout");
}

// ---------------------------------------------------------------------------
// Expert-gathered quantized matmul for the expert-sorted MoE chain
// (mtplx/moe_sorted_gather.py:241 gather_qmm_rows, :288 swiglu_rows,
// :339 switch_linear). Sorted row i multiplies x[rowmap[i]] (rowmap NULL:
// x[i]) by expert e's weights, where i lies in [expert_off[e], expert_off[e+1]).
// active = [count, expert ids...] from mtp_moe_sort. xmode 1 = silu(x)*x2 input;
// emode 3 = silu(x@W0^T)*(x@W1^T) output. rows_per_expert: weight rows between
// consecutive experts (N for separate gate/up tensors, 2N for a fused [gate|up]).
MTP_API int mtp_gather_qmv_affine4(const void* x, const void* x2, const uint32_t* rowmap, const int32_t* expert_off,
                                   const int32_t* active, const void* w0, const void* s0, const void* b0,
                                   const void* w1, const void* s1, const void* b1, void* y, int max_rows_per_expert,
                                   int E, int N, int K, int group_size, int xmode, int emode, int rows_per_expert,
                                   void* ws, size_t ws_bytes, void* stream) {
  (void)ws;
  (void)ws_bytes;
  const char* who = "mtp_gather_qmv_affine4";
  if (!x || !expert_off || !active || !w0 || !s0 || !b0 || !y || max_rows_per_expert < 1 || E < 1 || N < 1 ||
      K < 256 || K % 256 || rows_per_expert < N) {
    set_error("%s: bad arguments", who);
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
  if ((emode == E_DUAL_SWIGLU && (!w1 || !s1 || !b1)) || (xmode == X_SWIGLU && !x2) ||
      (xmode != X_PLAIN && xmode != X_SWIGLU)) {
    set_error("%s: mode/pointer mismatch", who);
    return MTP_ERR_ARG;
  }
  if (!aligned16(x) || !aligned16(w0) || (w1 && !aligned16(w1)) || (x2 && !aligned16(x2)) ||
      ((uintptr_t)s0 & 7) || ((uintptr_t)b0 & 7)) {
    set_error("%s: x and weights must be 16-byte aligned", who);
    return MTP_ERR_ARG;
  }
  QmmParams p = base_params(x, w0, s0, b0, y, 32, N, K, group_size);
  p.x2 = (const uint16_t*)x2;
  p.w1 = (const uint32_t*)w1;
  p.s1 = (const uint16_t*)s1;
  p.b1 = (const uint16_t*)b1;
  p.rowmap = rowmap;
  p.expert_off = expert_off;
  p.active = active;
  p.w_estride = (long long)rows_per_expert * (K / 8);
  p.s_estride = (long long)rows_per_expert * (K / group_size);
  const int mrows = max_rows_per_expert < 32 ? max_rows_per_expert : 32;
  p.row_tiles = cdiv(max_rows_per_expert, 32);
  Plan pl;
  pl.n_blocks = cdiv(N, 32);
  {
    const int Q = K / 256;
    const int ch = max_chunk_quads(mrows);
    pl.chunk = ch < Q ? ch : Q;
  }
  p.chunk = pl.chunk;
  pl.lds = lds_bytes(pl.chunk, mrows, 4);
  p.n_blocks = pl.n_blocks;
  const long long all_items = (long long)pl.n_blocks * p.row_tiles * E;
  const int cap = 4 * device_cus();   // a few resident workgroups per CU
  dim3 grid((unsigned)(all_items < cap ? all_items : cap));
  hipStream_t st = (hipStream_t)stream;
#define MTP_GATHER(RR, XMV, EMV)                                                                            \
  do {                                                                                                       \
    if (group_size == 64)                                                                                    \
      hipLaunchKernelGGL((gather_qmm4_kernel<RR, XMV, EMV, 0>), grid, dim3(kThreads), pl.lds, st, p);       \
    else                                                                                                     \
      hipLaunchKernelGGL((gather_qmm4_kernel<RR, XMV, EMV, 1>), grid, dim3(kThreads), pl.lds, st, p);       \
  } while (0)
  if (xmode == X_PLAIN && emode == E_STORE) {
    if (mrows <= 8) MTP_GATHER(4, X_PLAIN, E_STORE); else if (mrows <= 16) MTP_GATHER(8, X_PLAIN, E_STORE); else MTP_GATHER(16, X_PLAIN, E_STORE);
  } else if (xmode == X_PLAIN) {
    if (mrows <= 8) MTP_GATHER(4, X_PLAIN, E_DUAL_SWIGLU); else if (mrows <= 16) MTP_GATHER(8, X_PLAIN, E_DUAL_SWIGLU); else MTP_GATHER(16, X_PLAIN, E_DUAL_SWIGLU);
  } else if (emode == E_STORE) {
    if (mrows <= 8) MTP_GATHER(4, X_SWIGLU, E_STORE); else if (mrows <= 16) MTP_GATHER(8, X_SWIGLU, E_STORE); else MTP_GATHER(16, X_SWIGLU, E_STORE);
  } else {
    if (mrows <= 8) MTP_GATHER(4, X_SWIGLU, E_DUAL_SWIGLU); else if (mrows <= 16) MTP_GATHER(8, X_SWIGLU, E_DUAL_SWIGLU); else MTP_GATHER(16, X_SWIGLU, E_DUAL_SWIGLU);
  }
#undef MTP_GATHER
  return launch_check(who);
}

// ---------------------------------------------------------------------------
// Tile-major packing of a 4-bit affine matrix for the streaming kernel.
// Per (32-row tile nb, 256-k quad q), 1152 words:
//   words [256u + 4l, +4)  = row 32nb + l%32, words 32q + 8u + 4*(l/32) .. +3
//                            (u = 0..3, lane l = 0..63: the order one wave
//                            instruction reads, 1 KiB contiguous);
//   words [1024 + 4c, +4)  = row 32nb + c: scales of groups 4q..4q+3 then
//                            biases (bf16; group 128 repeats each value).
// Rows past N are zero (their outputs are never stored).
// Nibble k of a word moves to position (k >> 1) + 4 (k & 1): the operand
// conversion (w >> 4i) & 0x000F000F then yields bf16 pairs (k0,k1), (k2,k3),
// (k4,k5), (k6,k7) - natural k order, so packed weights take x as it is.
__device__ __forceinline__ uint32_t nibbles_natural(uint32_t w) {
  uint32_t o = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) o |= ((w >> (4 * k)) & 0xFu) << (4 * ((k >> 1) + 4 * (k & 1)));
  return o;
}

// layout 1: the 32x32x16 order - load u, lane l: words [32q + 8u + 4(l/32), +4)
// of row 32t + l%32. layout 2 (16x16x32, quad_mma16): load u = group u, lane l:
// word jj = 2 kk + h is word 8u + 4kk + l/16 of row 32t + 16h + l%16.
__global__ void pack_affine4_kernel(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint32_t* out, int N,
                                    int K, int gshift, int layout) {
  const int Q = K >> 8;
  const size_t units = (size_t)cdiv(N, 32) * Q * 288;   // 16 B units
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < units; t += (size_t)gridDim.x * blockDim.x) {
    const size_t tq = t / 288;
    const int u16 = (int)(t - tq * 288);
    const int nb = (int)(tq / Q);
    const int q = (int)(tq - (size_t)nb * Q);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (u16 < 256 && layout == 2) {
      const int u = u16 >> 6, l = u16 & 63;
      uint32_t wv[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int row = nb * 32 + 16 * (jj & 1) + (l & 15);
        wv[jj] = row < N ? nibbles_natural(w[(size_t)row * (K >> 3) + 32 * q + 8 * u + 4 * (jj >> 1) + (l >> 4)]) : 0u;
      }
      v = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    } else if (u16 < 256) {
      const int u = u16 >> 6, l = u16 & 63;
      const int row = nb * 32 + (l & 31);
      if (row < N) {
        v = *reinterpret_cast<const uint4*>(w + (size_t)row * (K >> 3) + 32 * q + 8 * u + 4 * (l >> 5));
        v = make_uint4(nibbles_natural(v.x), nibbles_natural(v.y), nibbles_natural(v.z), nibbles_natural(v.w));
      }
    } else {
      const int c = u16 - 256;
      const int row = nb * 32 + c;
      if (row < N) {
        const int sg = K >> (6 + gshift);
        const uint16_t* sr = s + (size_t)row * sg;
        const uint16_t* br = b + (size_t)row * sg;
        uint16_t e[8];
        for (int g = 0; g < 4; ++g) {
          const int gi = (4 * q + g) >> gshift;
          e[g] = sr[gi];
          e[4 + g] = br[gi];
        }
        v.x = e[0] | ((uint32_t)e[1] << 16);
        v.y = e[2] | ((uint32_t)e[3] << 16);
        v.z = e[4] | ((uint32_t)e[5] << 16);
        v.w = e[6] | ((uint32_t)e[7] << 16);
      }
    }
    *reinterpret_cast<uint4*>(out + tq * kPackQuadWords + 4 * (size_t)u16) = v;
  }
}

MTP_API size_t mtp_pack_affine4_bytes(int N, int K) {
  if (N < 1 || K < 256 || K % 256) return 0;
  return (size_t)cdiv(N, 32) * (K / 256) * kPackQuadWords * 4;
}

static int pack_run(const void* w, const void* scales, const void* biases, void* out, int N, int K, int group_size,
                    int layout, void* stream, const char* who) {
  if (!w || !scales || !biases || !out || N < 1 || K < 256 || K % 256 || !aligned16(w) || !aligned16(out)) {
    set_error("%s: bad arguments (K %% 256 == 0, 16-byte aligned w/out)", who);
    return MTP_ERR_ARG;
  }
  if (group_size != 64 && group_size != 128) {
    set_error("%s: group_size %d unsupported", who, group_size);
    return MTP_ERR_UNSUPPORTED;
  }
  const size_t units = (size_t)cdiv(N, 32) * (K / 256) * 288;
  size_t grid = (units + 255) / 256;
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(pack_affine4_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (const uint32_t*)w, (const uint16_t*)scales, (const uint16_t*)biases, (uint32_t*)out, N, K,
                     group_size == 128 ? 1 : 0, layout);
  return launch_check(who);
}

MTP_API int mtp_pack_affine4(const void* w, const void* scales, const void* biases, void* out, int N, int K,
                             int group_size, void* stream) {
  return pack_run(w, scales, biases, out, N, K, group_size, 1, stream, "mtp_pack_affine4");
}

MTP_API int mtp_pack_affine4_mf16(const void* w, const void* scales, const void* biases, void* out, int N, int K,
                                  int group_size, void* stream) {
  return pack_run(w, scales, biases, out, N, K, group_size, 2, stream, "mtp_pack_affine4_mf16");
}


namespace mtp {

// Argument block -> kernel parameters (no checks beyond the mode ranges).
int qmv_args_params(const mtp_qmv_args* a, QmmParams* out, const char* who) {
  if (!a) {
    set_error("%s: null argument block", who);
    return MTP_ERR_ARG;
  }
  if (a->xmode < 0 || a->xmode > 3 || a->emode < 0 || a->emode > 4 || (a->emode == E_ROPE_QKV && !a->rope)) {
    set_error("%s: xmode %d / emode %d out of range", who, a->xmode, a->emode);
    return MTP_ERR_ARG;
  }
  QmmParams p = base_params(a->x, a->w0, a->s0, a->b0, a->y0, a->M, a->N, a->K, a->group_size);
  p.x2 = (const uint16_t*)a->x2;
  p.ss_in = a->ss_in;
  p.ss_parts = cdiv(a->K, 32);
  p.w1 = (const uint32_t*)a->w1;
  p.s1 = (const uint16_t*)a->s1;
  p.b1 = (const uint16_t*)a->b1;
  p.y1 = (uint16_t*)a->y1;
  p.yf = a->yf;
  p.resid = (const uint16_t*)a->resid;
  p.ss_out = a->ss_out;
  p.eps = a->eps;
  p.packed = a->packed;
  if (a->ldx > 0) p.ldx = a->ldx;
  if (a->ldy > 0) p.ldy = a->ldy;
  p.x_sums = a->x_sums;
  p.y_sums = a->y_sums;
  if (a->emode == E_ROPE_QKV) {
    const mtp_rope_out* r = a->rope;
    p.q_start = r->q_start;
    p.q_lens = r->q_lens;
    p.q_out = (uint16_t*)r->q_out;
    p.k_cache = (uint16_t*)r->k_cache;
    p.v_cache = (uint16_t*)r->v_cache;
    p.status = r->status;
    p.rope_L = r->L;
    p.rope_Hq = r->Hq;
    p.rope_Hkv = r->Hkv;
    p.rope_D = r->D;
    p.rope_cap = r->cap;
    p.rope_blocked = r->blocked;
    p.rope_log2_base = r->rope_base > 1.f ? log2f(r->rope_base) : 0.f;
  }
  *out = p;
  return MTP_OK;
}

}  // namespace mtp

MTP_API int mtp_qmv_affine4_ex(const mtp_qmv_args* a, void* stream) {
  QmmParams p;
  const int rc = qmv_args_params(a, &p, "mtp_qmv_affine4_ex");
  if (rc != MTP_OK) return rc;
  return qmm_dispatch(a->xmode, a->emode, p, a->ws, a->ws_bytes, (hipStream_t)stream, "mtp_qmv_affine4_ex",
                      a->schedule);
}
