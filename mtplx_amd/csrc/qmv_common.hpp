// Shared pieces of the 4-bit verify matmul kernels (qmv.hip, qmm_mfma.hip):
// launch parameters, the nibble -> bf16 operand conversion, the fused x
// producers and the output epilogues.
#pragma once

#include "common.hpp"

namespace mtp {

// X_PRE: x comes with its per-32-column row sums (written by the producing
// epilogue), so staging is the copy alone.
enum XMode { X_PLAIN = 0, X_SWIGLU = 1, X_RMSNORM = 2, X_PRE = 3 };
enum EMode { E_STORE = 0, E_RESID = 1, E_DUAL = 2, E_DUAL_SWIGLU = 3, E_ROPE_QKV = 4 };

struct QmmParams {
  const uint16_t* x;       // activations [rows, ldx] (X_SWIGLU: gate)
  const uint16_t* x2;      // X_SWIGLU: up [rows, ldx]; X_RMSNORM: norm weight [K]
  const uint32_t* w0;
  const uint16_t* s0;
  const uint16_t* b0;
  const uint32_t* w1;      // second matrix (E_DUAL*), same shape
  const uint16_t* s1;
  const uint16_t* b1;
  uint16_t* y0;            // [rows, ldy]
  uint16_t* y1;            // E_DUAL: second output
  float* yf;               // E_STORE: optional fp32 output (bf16-rounded values)
  const uint16_t* resid;   // E_RESID: [rows, ldy]
  float* ss_out;           // E_RESID: per 32-column block, per row: sum of squares of y
  const float* ss_in;      // X_RMSNORM: producer's ss_out ([ss_parts][32]); null = compute
  int ss_parts;
  float* partial;          // [S, M, nvirt]
  uint32_t* counters;      // [n_blocks]
  // Expert-gathered mode (MoE): rows of expert e are [off[e], off[e+1]) of
  // the sorted row space; x row of sorted row i is rowmap[i] (null: i).
  const uint32_t* rowmap;
  const int32_t* expert_off;  // [E+1]
  const int32_t* active;      // [1 + E]: count, then active expert ids
  long long w_estride, s_estride;  // per-expert strides (uint32 words / bf16 elems)
  int row_tiles;              // 32-row tiles per expert in the grid
  int M, N, K, gs;
  int ldx, ldy;
  int S, gps, n_blocks, nvirt, chunk;
  int packed;              // w0/w1 in the tile-major layout (scales/biases inside)
  int tail_first, tail_split;   // tail split of the per-tile kernel (tail_split > 1)
  // Full K split (tail_first 0): workgroup vb takes part vb % tail_split of
  // the tiles vb / tail_split + j * (grid / tail_split), staging only that
  // part's xq quads of x (used when all of x does not fit in LDS).
  int full_split, xq;
  int tail_ok;                  // a workspace (partial, counters) is available for it
  // X_PRE input: per 32-column block, per row, sum of x ([K/32][32]).
  const float* x_sums;
  // Output for a following X_PRE matmul: the per-32-column row sums of the
  // stored y0 values, layout [N/32][32] (E_STORE, E_RESID, E_DUAL_SWIGLU).
  float* y_sums;
  float eps;
  // E_ROPE_QKV: the q|k|v rows go through RoPE straight to q_out [B, Hq, L, D]
  // and the K/V cache; row r is request r / rope_L, position q_start + r % rope_L.
  const int32_t* q_start;
  const int32_t* q_lens;
  uint16_t* q_out;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int32_t* status;
  int rope_L, rope_Hq, rope_Hkv, rope_D, rope_cap, rope_blocked;
  float rope_log2_base;
};

constexpr int kThreads = 256;
constexpr int kPackQuadWords = 1152;   // tile-major pack: words per (32-row tile, 256-k quad)

// Nibbles of one word -> bf16x8 operand (128+q exactly), element order
// (n0, n4, n1, n5, n2, n6, n3, n7). The mask and the exponent pattern are
// held in registers (gfx9 VOP3 encodings take no literal), so each output
// dword is one v_and_or_b32 (plus a shift): 7 VALU per word instead of 11.
struct NibConsts {
  uint32_t mask, bias;
};
__device__ __forceinline__ NibConsts nib_consts() {
  NibConsts c;
  asm volatile("s_mov_b32 %0, 0xf000f" : "=s"(c.mask));
  asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(c.bias));
  return c;
}
__device__ __forceinline__ bf16x8 nibbles_to_bf16(uint32_t w, NibConsts c) {
  uint32_t v[4];
  v[0] = (w & c.mask) | c.bias;
  v[1] = ((w >> 4) & c.mask) | c.bias;
  v[2] = ((w >> 8) & c.mask) | c.bias;
  v[3] = ((w >> 12) & c.mask) | c.bias;
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// x value as the consumer sees it (after the fused producer), rounded to bf16
// exactly as an unfused producer would have stored it. ``b`` is the up half
// (X_SWIGLU) or the norm weight (X_RMSNORM).
template <int XM>
__device__ __forceinline__ uint16_t produce(uint16_t a, uint16_t b, float inv_rms) {
  if (XM == X_PLAIN) return a;
  if (XM == X_SWIGLU) {
    float g = round_bf(silu_f(bf2f(a)));
    return f2bf(g * bf2f(b));
  }
  // X_RMSNORM: x * inv_rms * w in fp32, rounded once (a fused norm).
  return f2bf(bf2f(a) * inv_rms * bf2f(b));
}

// Sum over each aligned group of 8 lanes, result in all 8 (DPP, no LDS).
__device__ __forceinline__ float sum8_lanes(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
  return v;
}

// One 16 B chunk of x (8 consecutive k) through the producer, returned in
// the A-operand element order of the weights' nibble order: NAT = natural
// (tile-major packed weights), else bf16 pairs (t, t+4) (reference layout).
// Adds its 8 (bf16-rounded) values to ``sum``.
template <int XM, bool NAT>
__device__ __forceinline__ uint4 produce_chunk(uint4 raw, uint4 raw2, float inv_rms, float& sum) {
  uint4 o;
  if (XM == X_PLAIN) {
    if (NAT) {
      o = raw;
    } else {   // element t of the chunk is half (t & 1) of word t >> 1
      o.x = __builtin_amdgcn_perm(raw.z, raw.x, 0x05040100u);   // (e0, e4)
      o.y = __builtin_amdgcn_perm(raw.z, raw.x, 0x07060302u);   // (e1, e5)
      o.z = __builtin_amdgcn_perm(raw.w, raw.y, 0x05040100u);   // (e2, e6)
      o.w = __builtin_amdgcn_perm(raw.w, raw.y, 0x07060302u);   // (e3, e7)
    }
  } else {
    const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
    const uint32_t uv[4] = {raw2.x, raw2.y, raw2.z, raw2.w};
    float v[8];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float a0 = __uint_as_float(wv[t] << 16), a1 = __uint_as_float(wv[t] & 0xffff0000u);
      const float b0 = __uint_as_float(uv[t] << 16), b1 = __uint_as_float(uv[t] & 0xffff0000u);
      if (XM == X_SWIGLU) {
        v[2 * t] = round_bf(silu_f(a0)) * b0;
        v[2 * t + 1] = round_bf(silu_f(a1)) * b1;
      } else {   // X_RMSNORM: x * inv_rms * w in fp32, rounded once (a fused norm)
        v[2 * t] = a0 * inv_rms * b0;
        v[2 * t + 1] = a1 * inv_rms * b1;
      }
    }
    if (NAT) {
      o.x = f2bf2(v[0], v[1]);
      o.y = f2bf2(v[2], v[3]);
      o.z = f2bf2(v[4], v[5]);
      o.w = f2bf2(v[6], v[7]);
    } else {
      o.x = f2bf2(v[0], v[4]);
      o.y = f2bf2(v[1], v[5]);
      o.z = f2bf2(v[2], v[6]);
      o.w = f2bf2(v[3], v[7]);
    }
  }
  // Sum of the 8 bf16 values: one bf16 dot product with (1, 1) per pair.
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t one2 = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);
  sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o.x), one2, sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o.y), one2, sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o.z), one2, sum, false);
  sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, o.w), one2, sum, false);
  return o;
}

// Staged-x layout shared by the streaming kernels: row m holds the staged
// k range in natural order, 16-byte chunk c = k / 8 (group g = c / 8, half
// kq = (c / 4) % 2, MFMA step ii = c % 4), so staging copies 1 KB contiguous
// runs and a lane's A operands of a quad sit at immediate offsets (64-byte
// runs 128 bytes apart). Rows are padded by 16 B against LDS bank conflicts.
// Group sums: xs[g][2R] fp32.
__device__ __forceinline__ int xa_row_stride(int ngroups) { return ngroups * 8 + 1; }   // in uint4
__device__ __forceinline__ int xa_index(int kq, int m, int M, int rstride, int g, int ii) {
  (void)M;
  return m * rstride + g * 8 + kq * 4 + ii;
}
__host__ __device__ __forceinline__ size_t xa_bytes(int ngroups, int M) {
  return (size_t)M * (ngroups * 8 + 1) * 16;
}

typedef const __attribute__((address_space(1))) void* gptr_t;
typedef __attribute__((address_space(3))) void* lptr_t;

// Staging, phase 1: direct-to-LDS loads (no registers) of the raw x chunks of
// the k-quads kq0, kq0+1, ... (mod Q), nslot of them, into their staged
// positions. One wave instruction copies 64 consecutive chunks (1 KB) of one
// row of x.
template <int NW>
__device__ __forceinline__ void stage_x_issue(const QmmParams& p, uint4* xa, int rstride, int M, int Q, int kq0,
                                              int nslot, int wave, int lane) {
  const int rowchunks = 32 * nslot;
  const int nblk = (rowchunks + 63) >> 6;
  const int ntask = M * nblk;
  for (int task = wave; task < ntask; task += NW) {
    const int m = task / nblk;
    const int blk = task - m * nblk;
    const int c = blk * 64 + lane;
    if (c < rowchunks) {
      int qd = kq0 + (c >> 5);
      if (qd >= Q) qd -= Q;
      const int k = 256 * qd + 8 * (c & 31);
      const size_t xr = p.rowmap ? (size_t)p.rowmap[m] : (size_t)m;   // gathered rows (MoE)
      __builtin_amdgcn_global_load_lds((gptr_t)(p.x + xr * p.ldx + k),
                                       (lptr_t)(xa + (size_t)m * rstride + blk * 64), 16, 0, 0);
    }
  }
}

// X_RMSNORM staging works on items (staged 64-group gl, chunk cc), item it =
// 8 gl + cc, thread tid taking it = tid + j * NT. The norm-weight chunks of a
// thread's first kNormPre items are loaded into registers with the x loads;
// later items (K > 8 * kNormPre * NT) load theirs when used.
constexpr int kNormPre = 3;
__device__ __forceinline__ int norm_item_k(int it, int Q, int kq0) {
  const int gl = it >> 3;
  int qd = kq0 + (gl >> 2);
  if (qd >= Q) qd -= Q;
  return 64 * (4 * qd + (gl & 3)) + 8 * (it & 7);
}
template <int NW>
__device__ __forceinline__ void norm_w_prefetch(const QmmParams& p, uint4 (&wpre)[kNormPre], int Q, int kq0,
                                                int nslot, int tid) {
  const int nit = 32 * nslot;
#pragma unroll
  for (int j = 0; j < kNormPre; ++j) {
    const int it = tid + j * NW * 64;
    wpre[j] = make_uint4(0, 0, 0, 0);
    if (it < nit) wpre[j] = *reinterpret_cast<const uint4*>(p.x2 + norm_item_k(it, Q, kq0));
  }
}

// X_PRE: the group sums xs[gl][r] of the staged groups come from the
// producer's 32-column sums. Items are the (gl, r < M) pairs, it = gl * M + r;
// a thread's first kSumPre items are fetched with the x loads. Rows M..XSW-1
// are zeroed separately.
constexpr int kSumPre = 3;
__device__ __forceinline__ float2 xsum_item(const QmmParams& p, int it, int M, int Q, int kq0) {
  const int gl = it / M, r = it - gl * M;
  int qd = kq0 + (gl >> 2);
  if (qd >= Q) qd -= Q;
  const int g = 4 * qd + (gl & 3);
  return make_float2(p.x_sums[(size_t)(2 * g) * 32 + r], p.x_sums[(size_t)(2 * g + 1) * 32 + r]);
}
template <int NW, int XSW>
__device__ __forceinline__ void xsum_prefetch(const QmmParams& p, float2 (&sv)[kSumPre], int M, int Q, int kq0,
                                              int nslot, int tid) {
  const int nit = 4 * nslot * M;
#pragma unroll
  for (int j = 0; j < kSumPre; ++j) {
    const int it = tid + j * NW * 64;
    sv[j] = it < nit ? xsum_item(p, it, M, Q, kq0) : make_float2(0.f, 0.f);
  }
}
template <int NW, int XSW>
__device__ __forceinline__ void xsum_finish(const QmmParams& p, float* xs, const float2 (&sv)[kSumPre], int M, int Q,
                                            int kq0, int nslot, int tid) {
  const int nit = 4 * nslot * M;
  auto put = [&](int it, float2 v) {
    const int gl = it / M;
    xs[gl * XSW + (it - gl * M)] = v.x + v.y;
  };
#pragma unroll
  for (int j = 0; j < kSumPre; ++j) {
    const int it = tid + j * NW * 64;
    if (it < nit) put(it, sv[j]);
  }
  for (int it = tid + kSumPre * NW * 64; it < nit; it += NW * 64) put(it, xsum_item(p, it, M, Q, kq0));
  for (int idx = tid; idx < nslot * 4 * XSW; idx += NW * 64)
    if ((idx % XSW) >= M) xs[idx] = 0.f;
}

// Staging, phase 2 (after the loads have landed and a barrier): the fused
// producer, the A-operand element order and the per-group sums, in place.
// X_RMSNORM: one thread per (64-group, chunk) for all rows, so each norm
// weight chunk is loaded and unpacked once; the 8 threads of a group are 8
// consecutive lanes and add their row sums by DPP. Other modes: one thread
// per (row, 64-group), whose 8 chunks are independent LDS reads and whose sum
// needs no cross-lane step; X_SWIGLU reads its up half from global memory.
template <int XM, int NW, int XSW, bool NAT>
__device__ __forceinline__ void stage_x_finish(const QmmParams& p, uint4* xa, int rstride, float* xs,
                                               const uint4 (&wpre)[kNormPre], const float* inv_rms, int M, int Q,
                                               int kq0, int nslot, int tid) {
  constexpr int NT = NW * 64;
  const int ng = 4 * nslot;   // staged groups
  if (XM == X_RMSNORM) {
    const int nit = ng * 8;   // a multiple of 32: whole groups are in or out
    auto item = [&](int it, const uint4& wch) {
      const int gl = it >> 3, cc = it & 7;
      for (int m0 = 0; m0 < M; m0 += 4) {
        uint4 c[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (m0 + u < M) c[u] = xa[xa_index(cc >> 2, m0 + u, M, rstride, gl, cc & 3)];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (m0 + u < M) {
            float sum = 0.f;
            xa[xa_index(cc >> 2, m0 + u, M, rstride, gl, cc & 3)] =
                produce_chunk<XM, NAT>(c[u], wch, inv_rms[m0 + u], sum);
            sum = sum8_lanes(sum);
            if (cc == 0) xs[gl * XSW + m0 + u] = sum;
          }
        }
      }
    };
    // Trip counts are wave-uniform (base is a multiple of 64).
#pragma unroll
    for (int j = 0; j < kNormPre; ++j) {
      const int it = tid + j * NT;
      if ((it & ~63) < nit && it < nit) item(it, wpre[j]);
    }
    for (int it = tid + kNormPre * NT; (it & ~63) < nit; it += NT)
      if (it < nit) item(it, *reinterpret_cast<const uint4*>(p.x2 + norm_item_k(it, Q, kq0)));
  } else {
    for (int it = tid; it < M * ng; it += NT) {
      const int m = it / ng;
      const int gl = it - m * ng;
      int qd = kq0 + (gl >> 2);
      if (qd >= Q) qd -= Q;
      const int kb = 64 * (4 * qd + (gl & 3));
      float sum = 0.f;
      constexpr int B = (XM == X_PLAIN) ? 4 : 2;   // chunks read ahead (register budget)
#pragma unroll
      for (int cb = 0; cb < 8; cb += B) {   // chunk cc = 4 kq + ii covers k = kb + 8 cc
        uint4 c[B], aux[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int cc = cb + u;
          c[u] = xa[xa_index(cc >> 2, m, M, rstride, gl, cc & 3)];
          aux[u] = make_uint4(0, 0, 0, 0);
          if (XM == X_SWIGLU) aux[u] = *reinterpret_cast<const uint4*>(p.x2 + (size_t)m * p.ldx + kb + 8 * cc);
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int cc = cb + u;
          const uint4 o = produce_chunk<XM, NAT>(c[u], aux[u], 1.f, sum);
          if (!(XM == X_PLAIN && NAT)) xa[xa_index(cc >> 2, m, M, rstride, gl, cc & 3)] = o;
        }
      }
      xs[gl * XSW + m] = sum;
    }
  }
  for (int idx = tid; idx < nslot * 4 * XSW; idx += NT)
    if ((idx % XSW) >= M) xs[idx] = 0.f;
}

// Workgroup barrier for LDS data only. __syncthreads() also releases every
// global store, which compiles to s_waitcnt vmcnt(0): since loads and stores
// share that counter, it would drain a weight ring in flight at every tile
// boundary. This waits for the wave's LDS operations (lgkmcnt(0)) and meets;
// callers whose global stores must be visible wait for them explicitly.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0); vmcnt and expcnt left at their maxima
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt immediate for "at most vm vector-memory ops outstanding" (gfx9
// encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at 15:14).
__host__ __device__ constexpr int vmcnt_imm(int vm) { return (vm & 0xF) | (0x7 << 4) | (0xF << 8) | ((vm >> 4) << 14); }

// Row m's sum-of-squares partials, fetched into registers early (up to
// 64 * kMaxSsLoads partials, i.e. K <= 24576), reduced later.
constexpr int kMaxSsLoads = 12;
__device__ __forceinline__ void ss_prefetch(const QmmParams& p, int m, int lane, float (&v)[kMaxSsLoads]) {
#pragma unroll
  for (int i = 0; i < kMaxSsLoads; ++i) {
    const int j = lane + 64 * i;
    v[i] = (j < p.ss_parts) ? p.ss_in[(size_t)j * 32 + m] : 0.f;
  }
}
__device__ __forceinline__ float ss_reduce(const QmmParams& p, const float (&v)[kMaxSsLoads], int lane) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kMaxSsLoads; ++i) ss += v[i];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  (void)lane;
  return rsqrtf(ss / (float)p.K + p.eps);
}

// 1/rms of row m from the producer's sum-of-squares partials ([parts][32]),
// or from x itself when there are none; call with the whole wave.
__device__ __forceinline__ float row_inv_rms(const QmmParams& p, int m, int lane) {
  float ss = 0.f;
  if (p.ss_in) {
    for (int j = lane; j < p.ss_parts; j += 64) ss += p.ss_in[(size_t)j * 32 + m];
  } else {
    const uint16_t* xr = p.x + (size_t)m * p.ldx;
#pragma unroll 4
    for (int k = lane * 8; k < p.K; k += 64 * 8) {
      const uint4 raw = *reinterpret_cast<const uint4*>(xr + k);
      const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float a = __uint_as_float(wv[t] << 16), b = __uint_as_float(wv[t] & 0xffff0000u);
        ss += a * a + b * b;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  return rsqrtf(ss / (float)p.K + p.eps);
}

// Scales and bias corrections of the 4 groups of a quad from its packed
// bf16 words (GSH = 1: one scale per two groups, group size 128).
template <int GSH>
__device__ __forceinline__ void quad_scales(const uint32_t (&sw)[2], const uint32_t (&bw)[2], float (&s)[4],
                                            float (&cb)[4]) {
  float b[4];
  if (GSH == 0) {
    s[0] = __uint_as_float(sw[0] << 16), s[1] = __uint_as_float(sw[0] & 0xffff0000u);
    s[2] = __uint_as_float(sw[1] << 16), s[3] = __uint_as_float(sw[1] & 0xffff0000u);
    b[0] = __uint_as_float(bw[0] << 16), b[1] = __uint_as_float(bw[0] & 0xffff0000u);
    b[2] = __uint_as_float(bw[1] << 16), b[3] = __uint_as_float(bw[1] & 0xffff0000u);
  } else {
    s[0] = s[1] = __uint_as_float(sw[0] << 16);
    s[2] = s[3] = __uint_as_float(sw[0] & 0xffff0000u);
    b[0] = b[1] = __uint_as_float(bw[0] << 16);
    b[2] = b[3] = __uint_as_float(bw[0] & 0xffff0000u);
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) cb[g] = fmaf(-128.f, s[g], b[g]);
}

// One quad (4 groups of 64 k, 32 columns) into the R accumulator rows of
// this lane: t += s*G + (b - 128 s)*sum(x) per group, G = sum x*(128+q) on
// the MFMA. ``a_off``: byte offset of this lane's first A chunk of the quad;
// ``x_off``: byte offset of xs[g0][4*kq] (both relative to ``lds``).
template <int R>
__device__ __forceinline__ void quad_mma(const unsigned char* lds, uint32_t a_off, uint32_t x_off,
                                         const uint4 (&w)[4], const float (&s)[4], const float (&cb)[4],
                                         NibConsts nc, float (&t)[R]) {
  constexpr int XSW = 2 * R;
#pragma unroll
  for (int u = 0; u < 4; u += 2) {
    f32x16 G0 = {}, G1 = {};
    const uint32_t w0[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
    const uint32_t w1[4] = {w[u + 1].x, w[u + 1].y, w[u + 1].z, w[u + 1].w};
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(lds + a_off + (u * 8 + ii) * 16);
      const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(lds + a_off + ((u + 1) * 8 + ii) * 16);
      G0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, nibbles_to_bf16(w0[ii], nc), G0, 0, 0, 0);
      G1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, nibbles_to_bf16(w1[ii], nc), G1, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < R / 4; ++j) {
      const float4 x0 = *reinterpret_cast<const float4*>(lds + x_off + (u * XSW + 8 * j) * 4);
      const float4 x1 = *reinterpret_cast<const float4*>(lds + x_off + ((u + 1) * XSW + 8 * j) * 4);
      const float xv0[4] = {x0.x, x0.y, x0.z, x0.w};
      const float xv1[4] = {x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int r = 4 * j + r4;
        t[r] = fmaf(s[u], G0[r], fmaf(cb[u], xv0[r4], t[r]));
        t[r] = fmaf(s[u + 1], G1[r], fmaf(cb[u + 1], xv1[r4], t[r]));
      }
    }
  }
}

// One quad on v_mfma_f32_16x16x32_bf16 for M <= 4 (packed layout 2). x row m
// sits at A row 4m, so lane l's output register 0 is (row l/16, column
// l%16 [+16]): one accumulator per column half, two FMAs per group each.
// ``w[g]``: group g's words (2g, h=0), (2g, h=1), (2g+1, h=0), (2g+1, h=1);
// ``a0``/``a1``: byte offsets of the lane's A chunk of the group's first and
// second 32-k step; ``x_off``: byte offset of xs[g0][l/16].
__device__ __forceinline__ void quad_mma16(const unsigned char* lds, uint32_t a0, uint32_t a1, uint32_t x_off,
                                           int xsw, const uint4 (&w)[4], const float (&s0)[4], const float (&cb0)[4],
                                           const float (&s1)[4], const float (&cb1)[4], NibConsts nc, float& t0,
                                           float& t1) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const bf16x8 A0 = *reinterpret_cast<const bf16x8*>(lds + a0 + g * 128);
    const bf16x8 A1 = *reinterpret_cast<const bf16x8*>(lds + a1 + g * 128);
    f32x4_t G0 = {}, G1 = {};
    G0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, nibbles_to_bf16(w[g].x, nc), G0, 0, 0, 0);
    G1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, nibbles_to_bf16(w[g].y, nc), G1, 0, 0, 0);
    G0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, nibbles_to_bf16(w[g].z, nc), G0, 0, 0, 0);
    G1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, nibbles_to_bf16(w[g].w, nc), G1, 0, 0, 0);
    const float xv = *reinterpret_cast<const float*>(lds + x_off + g * xsw * 4);
    t0 = fmaf(s0[g], G0[0], fmaf(cb0[g], xv, t0));
    t1 = fmaf(s1[g], G1[0], fmaf(cb1[g], xv, t1));
  }
}

// The same quad on up to 16 rows (x row m at A row m): lane l's output
// register i is row 4(l/16) + i of columns l%16 (t0) and 16 + l%16 (t1), and
// its four rows' group sums are one float4 at x_off + g * xsw * 4.
__device__ __forceinline__ void quad_mma16x16(const unsigned char* lds, uint32_t a0, uint32_t a1, uint32_t x_off,
                                              int xsw, const uint4 (&w)[4], const float (&s0)[4],
                                              const float (&cb0)[4], const float (&s1)[4], const float (&cb1)[4],
                                              NibConsts nc, float (&t0)[4], float (&t1)[4]) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const bf16x8 A0 = *reinterpret_cast<const bf16x8*>(lds + a0 + g * 128);
    const bf16x8 A1 = *reinterpret_cast<const bf16x8*>(lds + a1 + g * 128);
    f32x4_t G0 = {}, G1 = {};
    G0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, nibbles_to_bf16(w[g].x, nc), G0, 0, 0, 0);
    G1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A0, nibbles_to_bf16(w[g].y, nc), G1, 0, 0, 0);
    G0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, nibbles_to_bf16(w[g].z, nc), G0, 0, 0, 0);
    G1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A1, nibbles_to_bf16(w[g].w, nc), G1, 0, 0, 0);
    const float4 xv = *reinterpret_cast<const float4*>(lds + x_off + g * xsw * 4);
    const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      t0[i] = fmaf(s0[g], G0[i], fmaf(cb0[g], xa[i], t0[i]));
      t1[i] = fmaf(s1[g], G1[i], fmaf(cb1[g], xa[i], t1[i]));
    }
  }
}

// Second producer input of the chunk at (row offset xo, column k): the up
// half for SwiGLU, the norm weight for RMSNorm, nothing otherwise.
template <int XM>
__device__ __forceinline__ uint4 producer_aux(const QmmParams& p, size_t xo, int k) {
  if (XM == X_SWIGLU) return *reinterpret_cast<const uint4*>(p.x2 + xo);
  if (XM == X_RMSNORM) return *reinterpret_cast<const uint4*>(p.x2 + k);
  return make_uint4(0, 0, 0, 0);
}

__device__ __forceinline__ size_t x_row(const QmmParams& p, int row0, int m) {
  const int r = row0 + m;
  return (size_t)(p.rowmap ? (int)p.rowmap[r] : r) * p.ldx;
}

// E_ROPE_QKV per-thread state of one epilogue element (row, pair): its
// position, the request's row count and the rotation.
struct RopeRow {
  int b, li, pos, len;
  float sn, cs;
};
// From the request's first position and row count (q_start[b], q_lens[b]).
__device__ __forceinline__ RopeRow rope_row(const QmmParams& p, int r, int d, int start, int len) {
  RopeRow q;
  q.b = r / p.rope_L;
  q.li = r - q.b * p.rope_L;
  q.pos = start + q.li;
  q.len = len;
  rope_angle(q.pos, d, p.rope_D, p.rope_log2_base, q.sn, q.cs);
  return q;
}
__device__ __forceinline__ RopeRow rope_row(const QmmParams& p, int r, int d) {
  const int b = r / p.rope_L;
  return rope_row(p, r, d, p.q_start[b], p.q_lens ? p.q_lens[b] : p.rope_L);
}

// ``pre``: this thread's residual value for its first output element, loaded
// at kernel start (E_RESID with M*32 <= threads), or null. ``rpre``: the same
// for E_ROPE_QKV (position and rotation of element idx == tid), or null.
template <int NW, int EM, bool WT = false>
__device__ __forceinline__ void qmm_epilogue(const QmmParams& p, float* fin, int nb, int M, int row0,
                                             const float* pre = nullptr, const RopeRow* rpre = nullptr) {
  constexpr int NT = NW * 64;
  const int tid = threadIdx.x;
  if (EM == E_ROPE_QKV) {
    // Packed column order: tile nb is head nb / (D/32), sub-block sb; local
    // column c < 16 holds d = 16 sb + c, c >= 16 holds d + D/2, so every
    // rotate-half pair sits in one tile. Values are rounded to bf16 first,
    // exactly as a stored q|k|v row would be.
    const int D = p.rope_D, half = D >> 1;
    const int head = nb / (D >> 5);
    const int d = 16 * (nb - head * (D >> 5));
    for (int idx = tid; idx < M * 16; idx += NT) {
      const int m = idx >> 4, i = idx & 15;
      const RopeRow rr = (rpre && idx == tid) ? *rpre : rope_row(p, row0 + m, d + i);
      const int b = rr.b, li = rr.li, pos = rr.pos, len = rr.len;
      const float x1 = round_bf(fin[m * 64 + i]), x2 = round_bf(fin[m * 64 + 16 + i]);
      uint16_t o1 = f2bf(x1), o2 = f2bf(x2);
      const bool kv = head >= p.rope_Hq;
      if (head < p.rope_Hq + p.rope_Hkv) rope_apply(x1, x2, rr.sn, rr.cs, o1, o2);
      if (!kv) {
        uint16_t* dst = p.q_out + (((size_t)b * p.rope_Hq + head) * p.rope_L + li) * D;
        st_u16<WT>(dst + d + i, o1);
        st_u16<WT>(dst + d + i + half, o2);
      } else if (li < len) {
        if (pos < 0 || pos >= p.rope_cap) {
          if (p.status) atomicOr(p.status, 1);
          continue;
        }
        const bool is_k = head < p.rope_Hq + p.rope_Hkv;
        const int kvh = head - p.rope_Hq - (is_k ? 0 : p.rope_Hkv);
        uint16_t* base = (is_k ? p.k_cache : p.v_cache) + ((size_t)b * p.rope_Hkv + kvh) * p.rope_cap * D;
        if (p.rope_blocked) {
          st_u16<WT>(base + (is_k ? kblk_index(pos, d + i) : vblk_index(pos, d + i)), o1);
          st_u16<WT>(base + (is_k ? kblk_index(pos, d + i + half) : vblk_index(pos, d + i + half)), o2);
        } else {
          st_u16<WT>(base + (size_t)pos * D + d + i, o1);
          st_u16<WT>(base + (size_t)pos * D + d + i + half, o2);
        }
      }
    }
    return;
  }
  for (int idx = tid; idx < M * 32; idx += NT) {
    const int m = idx >> 5;
    const int c = idx & 31;
    const int nn = nb * 32 + c;
    const bool in = nn < p.N;
    const size_t o = (size_t)(row0 + m) * p.ldy + nn;
    const float g = fin[m * 64 + c];
    if (EM == E_DUAL) {
      if (in) {
        st_u16<WT>(p.y0 + o, f2bf(g));
        st_u16<WT>(p.y1 + o, f2bf(fin[m * 64 + 32 + c]));
      }
    } else if (EM == E_DUAL_SWIGLU) {
      const float gs = round_bf(silu_f(round_bf(g)));
      const float a = in ? round_bf(gs * round_bf(fin[m * 64 + 32 + c])) : 0.f;
      if (in) st_u16<WT>(p.y0 + o, f2bf(a));
      fin[m * 64 + c] = a;   // this thread's own slot: the row sums below
    } else {
      float v = g;
      if (EM == E_RESID) {
        const float rv = (pre && idx == tid) ? *pre : (in ? bf2f(p.resid[o]) : 0.f);
        v = round_bf(in ? round_bf(v) + rv : 0.f);
        fin[m * 64 + 32 + c] = v * v;  // column 32+c is free in non-dual modes
        fin[m * 64 + c] = v;           // this thread's own slot: the row sums below
      } else {
        fin[m * 64 + c] = in ? round_bf(v) : 0.f;
      }
      if (in) {
        if (EM == E_STORE && p.yf)
          st_f32<WT>(p.yf + o, round_bf(v));
        else
          st_u16<WT>(p.y0 + o, f2bf(v));
      }
    }
  }
  const bool ss = EM == E_RESID && p.ss_out;
  const bool xsum = EM != E_DUAL && p.y_sums;
  if (ss || xsum) {
    lds_barrier();
    if (ss && tid < M) {
      float a = 0.f;
      for (int c = 0; c < 32; ++c) a += fin[tid * 64 + 32 + c];
      st_f32<WT>(p.ss_out + (size_t)nb * 32 + row0 + tid, a);
    }
    if (xsum && tid >= 64 && tid < 64 + M) {   // another wave, in parallel
      const int m = tid - 64;
      float a = 0.f;
      for (int c = 0; c < 32; ++c) a += fin[m * 64 + c];
      st_f32<WT>(p.y_sums + (size_t)nb * 32 + row0 + m, a);
    }
  }
}

int device_cus();

// Every split-K workspace starts with one fixed area of arrival counters
// (one per tile or tile group, each returned to zero by the call that used
// it), and its partials follow. With the counters at one place for every
// shape, one workspace serves calls of any shapes in turn: a call's partials
// never land where another shape keeps its counters.
constexpr size_t kCounterBytes = 65536;                 // 16384 counters
constexpr int kMaxCounters = (int)(kCounterBytes / 4);
// Tail split: fp32 partials of up to 16 rows x 64 values for two parts per CU.
constexpr int kTailMaxRows = 16;
inline size_t tail_workspace_bytes(int M, int N) {
  if (M < 1 || N < 1) return 0;
  return kCounterBytes + (size_t)2 * device_cus() * kTailMaxRows * 64 * sizeof(float);
}

}  // namespace mtp
