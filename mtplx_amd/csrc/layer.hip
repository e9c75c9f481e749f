// Fused dense decoder layer of the verify step: one persistent kernel per
// layer runs the six phases of mtplx/models' dense block (the reference's
// verify forward, mtplx/verify_qmv.py:1217 for the linears,
// mtplx/ragged_attention.py:42-85 for attention) that VerifyModel otherwise
// launches as six kernels:
//   1. RMSNorm + q|k|v + RoPE + K/V cache write   (qmv_stream_body, emode 4)
//   2. attention splits over the operand-major cache (attn_vt_body)
//   3. split merge                                   (attn_merge_body)
//   4. o_proj + residual                             (qmv_stream_body, emode 1)
//   5. RMSNorm + gate/up + SwiGLU (+ tail split)     (qmv_stream_body, emode 3)
//   6. down_proj + residual                          (qmv_stream_body, xmode 3)
//
// One 8-wave workgroup per CU, all resident (LDS sizes it to one per CU),
// with a grid barrier between phases. Each matmul phase issues its first
// weight loads before it waits at the barrier, so the weights' first round
// trip overlaps the previous phase's tail instead of following a kernel
// boundary. Phase outputs are written with device-coherent stores (through
// to memory) and no phase reads a buffer that an earlier phase of the same
// launch wrote on another XCD's copy: the caller's buffers are checked for
// that on the host (h, h1 = h + o(attn), act are distinct). The L2s start
// each launch clean, so plain loads then see the data, and the barrier needs
// no cache fences (a release + acquire pair would cost ~3 us per barrier).
#include "attn_vt.hpp"
#include "qmv_args.hpp"
#include "qmv_stream.hpp"

#include <stdlib.h>

namespace mtp {

constexpr int kLayerWaves = 8;
static_assert(kLayerWaves * 64 == kMergeThreads, "a merge item takes the whole workgroup");
constexpr unsigned kSpinLimit = 1u << 16;   // barrier polls before giving up (~0.1 s)

// Barrier state words, each on its own 256-byte line: [0] generation,
// [64] count of finished XCD groups, [128 + 64 g] arrivals of group g, and
// [128 + 64 * 8] the error flag.
constexpr int kBarGroups = 8;
constexpr int kBarErrWord = 128 + 64 * kBarGroups;
constexpr size_t kBarWords = kBarErrWord + 64;

struct LayerParams {
  QmmParams qkv, o, gu, gu_tail, down;
  AttnParams attn;
  int attn_units, merge_items, attn_tpw, has_tail;
  uint32_t* bar;
};

// Grid barrier, two levels (per XCD group of workgroups, then the groups),
// with self-resetting counters so consecutive launches need no reset. The
// caller's global stores must be complete (s_waitcnt) before it arrives;
// the last arrival of each level resets its counter before moving on. A wait
// that exceeds kSpinLimit polls sets the error flag and returns, so a
// workgroup that never arrives cannot hang the GPU (the results are then
// invalid and the host reports the flag).
__device__ __forceinline__ void grid_barrier(uint32_t* bar) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned G = gridDim.x;
    const unsigned g = blockIdx.x % kBarGroups;
    const unsigned ngroups = G < kBarGroups ? G : kBarGroups;
    const unsigned gsize = G / kBarGroups + (g < G % kBarGroups ? 1u : 0u);
    const unsigned gen = __hip_atomic_load(bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    uint32_t* grp = bar + 128 + 64 * g;
    if (__hip_atomic_fetch_add(grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gsize - 1) {
      __hip_atomic_store(grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      if (__hip_atomic_fetch_add(bar + 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ngroups - 1) {
        __hip_atomic_store(bar + 64, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        __hip_atomic_store(bar, gen + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    unsigned spins = 0;
    while (__hip_atomic_load(bar, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > kSpinLimit) {
        __hip_atomic_store(bar + kBarErrWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(kLayerWaves * 64) void verify_layer_kernel(LayerParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int vb = (int)blockIdx.x, vg = (int)gridDim.x;
  auto barrier = [&]() { grid_barrier(P.bar); };
  auto none = []() {};
  // 1. fused RMSNorm + q|k|v + RoPE, q to q_out, K/V into the cache.
  qmv_stream_body<kLayerWaves, 4, X_RMSNORM, E_ROPE_QKV, 0, true, true, 1>(P.qkv, vb, vg, none);
  // 2. attention splits, then 3. their merge.
  barrier();
  for (int u = vb; u < P.attn_units; u += vg) {
    if (P.attn_tpw == 1)
      attn_vt_body<1, true>(P.attn, u, smem);
    else
      attn_vt_body<2, true>(P.attn, u, smem);
    __syncthreads();   // the next unit rewrites the LDS merge area
  }
  barrier();
  for (int it = vb; it < P.merge_items; it += vg) {
    attn_merge_body<true>(P.attn, it, smem);
    __syncthreads();   // the next item's weights and l sum go to the same LDS
  }
  // 4. o_proj + residual; 5. gate/up (+ its leftover tiles split by K);
  // 6. down_proj + residual. Each issues its first weight loads, then waits.
  qmv_stream_body<kLayerWaves, 4, X_PLAIN, E_RESID, 0, true, true, 1>(P.o, vb, vg, barrier);
  qmv_stream_body<kLayerWaves, 4, X_RMSNORM, E_DUAL_SWIGLU, 0, true, true, 2>(P.gu, vb, vg, barrier);
  if (P.has_tail) qmv_stream_body<kLayerWaves, 4, X_RMSNORM, E_DUAL_SWIGLU, 0, true, true, 2>(P.gu_tail, vb, vg, none);
  qmv_stream_body<kLayerWaves, 4, X_PRE, E_RESID, 0, true, true, 2>(P.down, vb, vg, barrier);
}

static bool disjoint(const void* a, const void* b) { return a != b; }

}  // namespace mtp

using namespace mtp;

// Argument block of mtp_verify_layer (include/mtplx_amd.h).
struct mtp_verify_layer_args {
  mtp_qmv_args qkv;
  mtp_qmv_args o;
  mtp_qmv_args gate_up;
  mtp_qmv_args down;
  void* attn_out;
  float attn_scale;
  void* attn_ws;
  size_t attn_ws_bytes;
  void* sync;
  size_t sync_bytes;
};

// Sync buffer: the barrier words; 32-bit word 640 (kBarErrWord) is the error
// flag (1 after a barrier wait gave up), which the caller reads after the launch.
MTP_API size_t mtp_verify_layer_sync_bytes(void) { return kBarWords * sizeof(uint32_t); }

MTP_API int mtp_verify_layer(const mtp_verify_layer_args* a, void* stream) {
  const char* who = "mtp_verify_layer";
  if (!a || !a->qkv.rope || !a->attn_out || !a->attn_ws || !a->sync) {
    set_error("%s: null argument", who);
    return MTP_ERR_ARG;
  }
  LayerParams P{};
  int rc;
  if ((rc = qmv_args_params(&a->qkv, &P.qkv, who)) || (rc = qmv_args_params(&a->o, &P.o, who)) ||
      (rc = qmv_args_params(&a->gate_up, &P.gu, who)) || (rc = qmv_args_params(&a->down, &P.down, who)))
    return rc;
  const mtp_qmv_args &aq = a->qkv, &ao = a->o, &ag = a->gate_up, &ad = a->down;
  if (aq.xmode != X_RMSNORM || aq.emode != E_ROPE_QKV || ao.xmode != X_PLAIN || ao.emode != E_RESID ||
      ag.xmode != X_RMSNORM || ag.emode != E_DUAL_SWIGLU || ad.xmode != X_PRE || ad.emode != E_RESID) {
    set_error("%s: phases must be q|k|v (xmode 2, emode 4), o (0, 1), gate/up (2, 3), down (3, 1)", who);
    return MTP_ERR_ARG;
  }
  if ((rc = qmm_check_args(aq.xmode, aq.emode, P.qkv, who)) || (rc = qmm_check_args(ao.xmode, ao.emode, P.o, who)) ||
      (rc = qmm_check_args(ag.xmode, ag.emode, P.gu, who)) || (rc = qmm_check_args(ad.xmode, ad.emode, P.down, who)))
    return rc;
  const int M = P.qkv.M, H = P.qkv.K;
  const mtp_rope_out& r = *aq.rope;
  if (P.qkv.packed != 2 || P.o.packed != 2 || P.gu.packed != 2 || P.down.packed != 2 || M > 4 ||
      P.o.M != M || P.gu.M != M || P.down.M != M || P.qkv.gs != 64 || P.o.gs != 64 || P.gu.gs != 64 ||
      P.down.gs != 64 || !r.blocked || r.D != kHD || P.o.K != r.Hq * r.D || P.o.N != H || P.gu.K != H ||
      P.down.K != P.gu.N || P.down.N != H || (r.Hq / r.Hkv) * r.L > 32 || !ag.y_sums || !ag.ws) {
    set_error("%s: needs packed layout 2 (M <= 4, group 64) for all four matmuls, blocked K/V caches with "
              "head_dim 128, (Hq/Hkv)*L <= 32, gate/up row sums and a gate/up workspace, and matching shapes", who);
    return MTP_ERR_UNSUPPORTED;
  }
  // Dataflow: h -> q|k|v; attention -> attn_out -> o (+h) -> h1 -> gate/up
  // -> act (+ sums) -> down (+h1) -> y. Buffers written by a phase must not
  // be read before it in the same launch (no stale copies in another L2).
  if (ao.x != a->attn_out || ao.resid != aq.x || ag.x != ao.y0 || ag.ss_in != ao.ss_out || ad.x != ag.y0 ||
      ad.x_sums != ag.y_sums || ad.resid != ao.y0 || !ao.ss_out || !disjoint(ao.y0, aq.x) ||
      !disjoint(ao.ss_out, aq.ss_in) || !disjoint(ag.y0, aq.x) || !disjoint(ag.y0, ao.y0) ||
      !disjoint(ad.y0, ao.y0) || !disjoint(ad.y0, ag.y0)) {
    set_error("%s: buffers must chain h -> attn_out -> h1 -> act -> out, with h1 distinct from h, act distinct "
              "from h and h1, out distinct from h1 and act, and o's ss_out distinct from q|k|v's ss_in", who);
    return MTP_ERR_ARG;
  }
  if (a->sync_bytes < mtp_verify_layer_sync_bytes() || ((uintptr_t)a->sync & 255)) {
    set_error("%s: sync buffer of %zu B (256-B aligned, zeroed once) needed", who, mtp_verify_layer_sync_bytes());
    return MTP_ERR_WORKSPACE;
  }
  const int cus = device_cus();
  // q|k|v, o, down: one tile per workgroup, in order.
  P.qkv.n_blocks = cdiv(P.qkv.N, 32);
  P.o.n_blocks = cdiv(P.o.N, 32);
  P.down.n_blocks = cdiv(P.down.N, 32);
  // gate/up: T tiles; T - E run whole (several per workgroup), and when
  // E = T mod CUs divides the CUs, the E leftover tiles are split by K into
  // CUs / E parts (the standalone kernel's tail split, one part per CU).
  const int T = cdiv(P.gu.N, 32), Qg = P.gu.K >> 8;
  const int E = T % cus;
  P.gu.n_blocks = T;
  if (T > cus && E > 0 && cus % E == 0 && cus / E >= 2 && cus / E <= Qg) {
    const size_t need = qmv_sk_workspace_bytes(M, P.gu.N, P.gu.K, 1);
    if (ag.ws_bytes < need || ((uintptr_t)ag.ws & 255)) {
      set_error("%s: gate/up workspace of %zu B (256-B aligned) needed", who, need);
      return MTP_ERR_WORKSPACE;
    }
    P.has_tail = 1;
    P.gu.n_blocks = T - E;
    QmmParams& t = P.gu_tail;
    t = P.gu;
    const size_t tw = (size_t)(T - E) * Qg * kPackQuadWords;
    t.w0 += tw;
    t.w1 += tw;
    t.y0 += (size_t)(T - E) * 32;
    t.y_sums += (size_t)(T - E) * 32;
    t.N = P.gu.N - (T - E) * 32;
    t.n_blocks = E;
    t.tail_first = 0;
    t.tail_split = cus / E;
    t.partial = reinterpret_cast<float*>(ag.ws);
    t.counters = reinterpret_cast<uint32_t*>(reinterpret_cast<unsigned char*>(ag.ws) + sk_counter_offset(cus));
  }
  // Attention (rows layout out, the o projection's x).
  AttnParams& at = P.attn;
  at.q = (const uint16_t*)r.q_out;
  at.k = (const uint16_t*)r.k_cache;
  at.v = (const uint16_t*)r.v_cache;
  at.q_start = r.q_start;
  at.q_lens = r.q_lens;
  at.out = (uint16_t*)a->attn_out;
  at.B = M / r.L;
  at.Hq = r.Hq;
  at.Hkv = r.Hkv;
  at.L = r.L;
  at.cap = r.cap;
  at.out_rows = 1;
  at.scale_log2 = a->attn_scale * 1.4426950408889634f;
  int tpw = 1;
  if (attn_vt_plan(r.cap, &at.S, &tpw) != MTP_OK) {
    set_error("%s: capacity %d needs more than %d splits", who, r.cap, kMaxSplits);
    return MTP_ERR_UNSUPPORTED;
  }
  at.split_keys = kVtWaves * kTileKeys * tpw;
  const size_t units = (size_t)at.B * at.Hkv * at.S;
  if (a->attn_ws_bytes < units * 32 * kHD * sizeof(float) + units * 64 * sizeof(float)) {
    set_error("%s: attention workspace too small", who);
    return MTP_ERR_WORKSPACE;
  }
  at.part_o = (float*)a->attn_ws;
  at.part_ml = (float*)a->attn_ws + units * 32 * kHD;
  P.attn_units = (int)units;
  P.attn_tpw = tpw;
  P.merge_items = at.B * at.Hkv * (at.Hq / at.Hkv) * at.L;
  P.bar = (uint32_t*)a->sync;
  // LDS: the largest phase (all of x of each matmul, attention's merge area).
  size_t lds = attn_vt_lds_bytes();
  if (attn_merge_lds_bytes() > lds) lds = attn_merge_lds_bytes();
  const QmmParams* mm[4] = {&P.qkv, &P.o, &P.gu, &P.down};
  for (const QmmParams* q : mm) {
    const size_t l = stream_lds_bytes(q->K >> 8, M, kLayerWaves);
    if (l > lds) lds = l;
  }
  if (lds > 160 * 1024 - 256) {
    set_error("%s: staged x needs %zu B of LDS", who, lds);
    return MTP_ERR_UNSUPPORTED;
  }
  // Every workgroup must be resident: one per CU.
  if (hipFuncSetAttribute((const void*)verify_layer_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
      hipSuccess) {
    set_error("%s: cannot reserve %zu B of LDS", who, lds);
    return MTP_ERR_HIP;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, verify_layer_kernel, kLayerWaves * 64, lds) != hipSuccess ||
      occ < 1) {
    set_error("%s: the fused layer does not fit on a CU", who);
    return MTP_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(verify_layer_kernel, dim3(cus), dim3(kLayerWaves * 64), lds, (hipStream_t)stream, P);
  return launch_check(who);
}
