// 4-bit affine (group 64/128) quantized skinny GEMM for verify rows, gfx950.
//
//   y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/gs] + b[n, k/gs])
//
// Weight format is the reference's (mtplx/verify_kernels.py:69-88, :372):
// uint32 [N, K/8] with little-endian nibbles, bf16 scales/biases [N, K/gs].
//
// Design (MI355X-first, not a translation of the Metal split-K kernel):
//  * At M = 4 a VALU dot product cannot keep up with 8 TB/s of nibbles
//    (4 MACs + unpack per nibble exceeds the 64 lane-ops/clk/CU budget), so
//    the contraction runs on the matrix cores even for skinny M:
//    v_mfma_f32_32x32x16_bf16 with A = activations (rows m, zero-padded to 32)
//    and B = nibbles.
//  * Nibbles become bf16 operands with one AND-OR each: (w & 0x000F000F) |
//    0x43004300 is the bf16 pair (128 + q_lo, 128 + q_hi), exact. The MFMA
//    therefore yields G = sum x*(128+q) per 64-wide group, and the group is
//    finished on the VALU as s*G + (b - 128*s)*sum(x) with sum(x) per group
//    precomputed while staging x. Dequantised weights are never rounded.
//  * One lane streams 16 B of a weight row per 64-group (two lanes per row,
//    32 rows per wave, 128 rows per 256-thread workgroup): each wave load is
//    32 contiguous 32 B row segments.
//  * K is split across workgroups so every launch has ~1k workgroups; split
//    partials go to a fp32 workspace and the last workgroup of a column block
//    (an integer arrival counter, reset by that workgroup) sums them in split
//    order — deterministic, no float atomics. Splits of one column block are
//    mapped onto the same XCD so the partials meet in one L2.
//  * Activations are staged once per workgroup into LDS in the MFMA A-operand
//    order, with optional fused producers: SwiGLU (silu(gate)*up) or RMSNorm.
#include "common.hpp"

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

enum XMode { X_PLAIN = 0, X_SWIGLU = 1, X_RMSNORM = 2 };
enum EMode { E_STORE = 0, E_RESID = 1, E_DUAL = 2, E_DUAL_SWIGLU = 3 };

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
  float eps;
};

constexpr int kThreads = 256;

// Nibbles of one word -> bf16x8 operand (128+q exactly), element order
// (n0, n4, n1, n5, n2, n6, n3, n7).
__device__ __forceinline__ bf16x8 nibbles_to_bf16(uint32_t w) {
  uint32_t v[4];
  v[0] = (w & 0x000F000Fu) | 0x43004300u;
  v[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
  v[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
  v[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// x value as the consumer sees it (after the fused producer), rounded to bf16
// exactly as an unfused producer would have stored it.
template <int XM>
__device__ __forceinline__ uint16_t produce(const QmmParams& p, uint16_t a, uint16_t b, float inv_rms,
                                            int k) {
  if (XM == X_PLAIN) return a;
  if (XM == X_SWIGLU) {
    float g = round_bf(silu_f(bf2f(a)));
    return f2bf(g * bf2f(b));
  }
  // X_RMSNORM: x * inv_rms * w in fp32, rounded once (a fused norm).
  return f2bf(bf2f(a) * inv_rms * bf2f(p.x2[k]));
}

__device__ __forceinline__ size_t x_row(const QmmParams& p, int row0, int m) {
  const int r = row0 + m;
  return (size_t)(p.rowmap ? (int)p.rowmap[r] : r) * p.ldx;
}

// One workgroup = 4 waves over 32 output columns (one MFMA column tile) and
// the whole K range. K is split between the waves by "quads" (4 groups =
// 256 k = one 128 B line per weight row): plain modes give wave w the quads
// w, w+4, ...; dual modes give waves 0,1 matrix 0 and waves 2,3 matrix 1,
// each pair splitting the quads two ways. Partials meet in LDS and are summed
// in wave order — deterministic, no global atomics. x is staged in chunks of
// p.chunk quads shared by all waves; weight loads run one quad ahead of the
// MFMAs with no data-dependent branches, so the memory pipeline never drains.
// Leaves the final values in fin[M][64] (cols 0..31 matrix 0, 32..63 matrix 1).
template <int R, int XM, int EM, int GSH>
__device__ __forceinline__ void qmm_body(const QmmParams& p, unsigned char* smem, int nb, int M, int row0,
                                         long long woff, long long soff) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int Q = p.K >> 8;            // quads
  const int CHQ = p.chunk;           // quads per staging chunk
  constexpr bool dual = (EM == E_DUAL || EM == E_DUAL_SWIGLU);
  constexpr int KS = dual ? 2 : 4;   // waves sharing one column tile
  const int kw = dual ? (wave & 1) : wave;
  const int which = dual ? (wave >> 1) : 0;

  uint4* xa = reinterpret_cast<uint4*>(smem);                                 // [CHQ*4][4][2][M]
  float* xs = reinterpret_cast<float*>(smem + (size_t)CHQ * 4 * 8 * M * 16);  // [CHQ*4][32]
  float* red = reinterpret_cast<float*>(smem);  // [4][32 m][32 c], reuses the staging area
  __shared__ float s_inv_rms[32];

  // ---- RMSNorm statistics (full row, fp32, fixed order) ----
  if (XM == X_RMSNORM) {
    for (int m = wave; m < M; m += 4) {
      const uint16_t* xr = p.x + x_row(p, row0, m);
      float ss = 0.f;
      for (int k = lane * 8; k < p.K; k += 64 * 8) {
        uint4 raw = *reinterpret_cast<const uint4*>(xr + k);
        const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float a = bf2f((uint16_t)(wv[t] & 0xffff)), b = bf2f((uint16_t)(wv[t] >> 16));
          ss += a * a + b * b;
        }
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
      if (lane == 0) s_inv_rms[m] = rsqrtf(ss / (float)p.K + p.eps);
    }
    __syncthreads();
  }

  const int c32 = lane & 31;
  const int kq = lane >> 5;
  const int n = nb * 32 + c32;
  const bool valid = n < p.N;
  const int nrow = valid ? n : 0;
  const uint32_t* W = which ? p.w1 : p.w0;
  const uint16_t* Sc = which ? p.s1 : p.s0;
  const uint16_t* Bi = which ? p.b1 : p.b0;
  // Lane reads words [32*q + 8*u + 4*kq, +4) of its row for group u of quad q.
  const uint32_t* wrow = W + woff + (size_t)nrow * (p.K >> 3) + kq * 4;
  const int sgroups = p.K >> (6 + GSH);
  const uint16_t* srow = Sc + soff + (size_t)nrow * sgroups;
  const uint16_t* brow = Bi + soff + (size_t)nrow * sgroups;
  const bool arow = c32 < M;

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;

  // Per-quad operands: 4 x 16 B of nibbles, 4 scales, 4 biases.
  struct QuadRegs {
    uint4 w[4];
    uint32_t s[2], b[2];
  };
  auto load_quad = [&](int q, QuadRegs& qr) {
    const uint32_t* wp = wrow + 32 * q;
#pragma unroll
    for (int u = 0; u < 4; ++u) qr.w[u] = *reinterpret_cast<const uint4*>(wp + 8 * u);
    if (GSH == 0) {
      const uint2 sv = *reinterpret_cast<const uint2*>(srow + 4 * q);
      const uint2 bv = *reinterpret_cast<const uint2*>(brow + 4 * q);
      qr.s[0] = sv.x; qr.s[1] = sv.y;
      qr.b[0] = bv.x; qr.b[1] = bv.y;
    } else {
      qr.s[0] = *reinterpret_cast<const uint32_t*>(srow + 2 * q);
      qr.b[0] = *reinterpret_cast<const uint32_t*>(brow + 2 * q);
      qr.s[1] = qr.s[0];
      qr.b[1] = qr.b[0];
    }
  };
  auto scale_of = [&](const uint32_t* v, int u) -> float {
    // gs 64: group u -> element u; gs 128: groups (0,1)->elem 0, (2,3)->elem 1.
    const uint32_t word = (GSH == 0) ? v[u >> 1] : v[0];
    const int half = (GSH == 0) ? (u & 1) : (u >> 1);
    return bf2f((uint16_t)(half ? (word >> 16) : (word & 0xffff)));
  };

  const int nchunks = cdiv(Q, CHQ);
  int q = kw;
  QuadRegs cur;
  load_quad(q < Q ? q : Q - 1, cur);
  for (int c = 0; c < nchunks; ++c) {
    const int cq0 = c * CHQ;
    const int cq1 = min(Q, cq0 + CHQ);
    // ---- stage x for quads [cq0, cq1) in MFMA A order + group sums ----
    __syncthreads();
    const int ng = 4 * (cq1 - cq0);
    for (int pidx = tid; pidx < ng * M; pidx += kThreads) {
      const int gl = pidx / M;
      const int m = pidx - gl * M;
      const int kbase = 64 * (4 * cq0 + gl);
      const size_t xo = x_row(p, row0, m) + kbase;
      const uint16_t* xr = p.x + xo;
      const uint16_t* ur = (XM == X_SWIGLU) ? p.x2 + xo : nullptr;
      const float inv = (XM == X_RMSNORM) ? s_inv_rms[m] : 1.f;
      float sum = 0.f;
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        uint4 raw = *reinterpret_cast<const uint4*>(xr + 8 * cc);
        uint4 raw2 = make_uint4(0, 0, 0, 0);
        if (XM == X_SWIGLU) raw2 = *reinterpret_cast<const uint4*>(ur + 8 * cc);
        const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
        const uint32_t uv[4] = {raw2.x, raw2.y, raw2.z, raw2.w};
        uint16_t e[8];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          e[2 * t] = produce<XM>(p, (uint16_t)(wv[t] & 0xffff), (uint16_t)(uv[t] & 0xffff), inv,
                                 kbase + 8 * cc + 2 * t);
          e[2 * t + 1] = produce<XM>(p, (uint16_t)(wv[t] >> 16), (uint16_t)(uv[t] >> 16), inv,
                                     kbase + 8 * cc + 2 * t + 1);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) sum += bf2f(e[t]);
        uint4 o;
        o.x = (uint32_t)e[0] | ((uint32_t)e[4] << 16);
        o.y = (uint32_t)e[1] | ((uint32_t)e[5] << 16);
        o.z = (uint32_t)e[2] | ((uint32_t)e[6] << 16);
        o.w = (uint32_t)e[3] | ((uint32_t)e[7] << 16);
        // 8-element chunk cc covers k offset 8cc = 32*kq + 8*i within the group
        xa[((gl * 4 + (cc & 3)) * 2 + (cc >> 2)) * M + m] = o;
      }
      xs[gl * 32 + m] = sum;
    }
    for (int idx = tid; idx < ng * 32; idx += kThreads)
      if ((idx & 31) >= M) xs[idx] = 0.f;
    __syncthreads();

    // ---- this wave's quads inside the chunk ----
    for (; q < cq1; q += KS) {
      QuadRegs nxt;
      const int qn = q + KS;
      load_quad(qn < Q ? qn : Q - 1, nxt);
      const int gq = 4 * (q - cq0);
#pragma unroll
      for (int u = 0; u < 4; u += 2) {
        f32x16 G0 = {}, G1 = {};
        const uint32_t w0[4] = {cur.w[u].x, cur.w[u].y, cur.w[u].z, cur.w[u].w};
        const uint32_t w1[4] = {cur.w[u + 1].x, cur.w[u + 1].y, cur.w[u + 1].z, cur.w[u + 1].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bf16x8 a0 = {}, a1 = {};
          if (arow) {
            a0 = __builtin_bit_cast(bf16x8, xa[(((gq + u) * 4 + i) * 2 + kq) * M + c32]);
            a1 = __builtin_bit_cast(bf16x8, xa[(((gq + u + 1) * 4 + i) * 2 + kq) * M + c32]);
          }
          G0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, nibbles_to_bf16(w0[i]), G0, 0, 0, 0);
          G1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, nibbles_to_bf16(w1[i]), G1, 0, 0, 0);
        }
        const float s0 = scale_of(cur.s, u), s1 = scale_of(cur.s, u + 1);
        const float cb0 = scale_of(cur.b, u) - 128.f * s0;
        const float cb1 = scale_of(cur.b, u + 1) - 128.f * s1;
        const float4 xs0 = *reinterpret_cast<const float4*>(xs + (gq + u) * 32 + 4 * kq);
        const float4 xs1 = *reinterpret_cast<const float4*>(xs + (gq + u + 1) * 32 + 4 * kq);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int off = 8 * (r >> 2) + (r & 3);
          float x0, x1;
          if (off < 4) {
            x0 = (&xs0.x)[off];
            x1 = (&xs1.x)[off];
          } else {
            x0 = xs[(gq + u) * 32 + 4 * kq + off];
            x1 = xs[(gq + u + 1) * 32 + 4 * kq + off];
          }
          acc[r] = fmaf(s0, G0[r], fmaf(cb0, x0, acc[r]));
          acc[r] = fmaf(s1, G1[r], fmaf(cb1, x1, acc[r]));
        }
      }
      cur = nxt;
    }
  }

  // ---- reduce the K-split waves in LDS (wave order) ----
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int m = 8 * (r >> 2) + 4 * kq + (r & 3);
    if (m < M) red[(wave * 32 + m) * 32 + c32] = valid ? acc[r] : 0.f;
  }
  __syncthreads();
  float* fin = red + 4 * 32 * 32;  // [M][64]
  for (int idx = tid; idx < M * 64; idx += kThreads) {
    const int m = idx >> 6;
    const int c = idx & 63;
    const int mat = c >> 5;
    float v = 0.f;
    if (!dual && mat == 0) {
#pragma unroll
      for (int w = 0; w < 4; ++w) v += red[(w * 32 + m) * 32 + c];
    } else if (dual) {
      v = red[((2 * mat) * 32 + m) * 32 + (c & 31)] + red[((2 * mat + 1) * 32 + m) * 32 + (c & 31)];
    }
    fin[idx] = v;
  }
  __syncthreads();
}

// Epilogue from fin[m][64]: columns nb*32 + c, output rows row0 + m.
template <int EM>
__device__ __forceinline__ void qmm_epilogue(const QmmParams& p, const float* fin, int nb, int M, int row0) {
  const int tid = threadIdx.x;
  for (int idx = tid; idx < M * 32; idx += kThreads) {
    const int m = idx >> 5;
    const int c = idx & 31;
    const int nn = nb * 32 + c;
    if (nn >= p.N) continue;
    const size_t o = (size_t)(row0 + m) * p.ldy + nn;
    const float g = fin[m * 64 + c];
    if (EM == E_DUAL) {
      p.y0[o] = f2bf(g);
      p.y1[o] = f2bf(fin[m * 64 + 32 + c]);
    } else if (EM == E_DUAL_SWIGLU) {
      const float gs = round_bf(silu_f(round_bf(g)));
      p.y0[o] = f2bf(gs * round_bf(fin[m * 64 + 32 + c]));
    } else {
      float v = g;
      if (EM == E_RESID) v = round_bf(v) + bf2f(p.resid[o]);
      if (EM == E_STORE && p.yf)
        p.yf[o] = round_bf(v);
      else
        p.y0[o] = f2bf(v);
    }
  }
}

__device__ __forceinline__ float* fin_of(unsigned char* smem) {
  return reinterpret_cast<float*>(smem) + 4 * 32 * 32;
}

template <int R, int XM, int EM, int GSH>
__global__ __launch_bounds__(kThreads) void qmm4_kernel(QmmParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nb = blockIdx.x;
  qmm_body<R, XM, EM, GSH>(p, smem, nb, p.M, 0, 0, 0);
  qmm_epilogue<EM>(p, fin_of(smem), nb, p.M, 0);
}

// Expert-gathered launch: grid (column tiles, row tiles, expert slots).
template <int R, int XM, int EM, int GSH>
__global__ __launch_bounds__(kThreads) void gather_qmm4_kernel(QmmParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nb = blockIdx.x;
  const int rt = blockIdx.y;
  const int slot = blockIdx.z;
  if (slot >= p.active[0]) return;
  const int e = p.active[1 + slot];
  const int r0 = p.expert_off[e] + 32 * rt;
  const int r1 = p.expert_off[e + 1];
  if (r0 >= r1) return;
  const int M = min(32, r1 - r0);
  qmm_body<R, XM, EM, GSH>(p, smem, nb, M, r0, (long long)e * p.w_estride, (long long)e * p.s_estride);
  qmm_epilogue<EM>(p, fin_of(smem), nb, M, r0);
}

// ---------------------------------------------------------------------------
// Host side: split planning and dispatch.

struct Plan {
  int n_blocks, chunk;
  size_t lds;
};

static int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return (v && *v) ? atoi(v) : dflt;
}

// LDS: staged x per quad (4 groups x (8*M*16 B + 32 floats)); the K-split
// reduction (16 KiB + fin) reuses the same area afterwards.
static size_t lds_bytes(int chunk_q, int M) {
  size_t stage = (size_t)chunk_q * 4 * (8 * M * 16 + 32 * 4);
  size_t red = 4 * 32 * 32 * 4 + (size_t)M * 64 * 4;
  return stage > red ? stage : red;
}

static int max_chunk_quads(int M) {
  int ch = (60 * 1024) / (4 * (8 * M * 16 + 128));
  return ch < 1 ? 1 : ch;
}

static Plan make_plan(int M, int N, int K) {
  Plan pl;
  pl.n_blocks = cdiv(N, 32);
  const int Q = K / 256;
  int ch = max_chunk_quads(M);
  const int cap = env_int("MTPLX_AMD_QMV_CHUNK_QUADS", 0);
  if (cap > 0 && cap < ch) ch = cap;
  pl.chunk = ch < Q ? ch : Q;
  pl.lds = lds_bytes(pl.chunk, M);
  return pl;
}

template <int XM, int EM, int GSH>
static void launch_r(const QmmParams& p, const Plan& pl, hipStream_t st) {
  dim3 grid(pl.n_blocks), block(kThreads);
  if (p.M <= 8)
    hipLaunchKernelGGL((qmm4_kernel<4, XM, EM, GSH>), grid, block, pl.lds, st, p);
  else if (p.M <= 16)
    hipLaunchKernelGGL((qmm4_kernel<8, XM, EM, GSH>), grid, block, pl.lds, st, p);
  else
    hipLaunchKernelGGL((qmm4_kernel<16, XM, EM, GSH>), grid, block, pl.lds, st, p);
}

template <int XM, int GSH>
static void launch_e(int em, const QmmParams& p, const Plan& pl, hipStream_t st) {
  switch (em) {
    case E_STORE: launch_r<XM, E_STORE, GSH>(p, pl, st); break;
    case E_RESID: launch_r<XM, E_RESID, GSH>(p, pl, st); break;
    case E_DUAL: launch_r<XM, E_DUAL, GSH>(p, pl, st); break;
    default: launch_r<XM, E_DUAL_SWIGLU, GSH>(p, pl, st); break;
  }
}

template <int GSH>
static void launch_x(int xm, int em, const QmmParams& p, const Plan& pl, hipStream_t st) {
  switch (xm) {
    case X_PLAIN: launch_e<X_PLAIN, GSH>(em, p, pl, st); break;
    case X_SWIGLU: launch_e<X_SWIGLU, GSH>(em, p, pl, st); break;
    default: launch_e<X_RMSNORM, GSH>(em, p, pl, st); break;
  }
}

static bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

// Shared validation + dispatch for every qmm entry point.
static int qmm_dispatch(int xm, int em, QmmParams p, void* ws, size_t ws_bytes, hipStream_t st,
                        const char* who) {
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
  if (!p.x || !p.w0 || !p.s0 || !p.b0 || (!p.y0 && !p.yf)) {
    set_error("%s: null pointer argument", who);
    return MTP_ERR_ARG;
  }
  if (p.ldx < p.K || p.ldx % 8 || !aligned16(p.x) || !aligned16(p.w0) || ((uintptr_t)p.s0 & 7) ||
      ((uintptr_t)p.b0 & 7) || (p.x2 && xm == X_SWIGLU && !aligned16(p.x2))) {
    set_error("%s: x rows/weights must be 16-byte and scales/biases 8-byte aligned, ldx %% 8 == 0 (ldx=%d)", who,
              p.ldx);
    return MTP_ERR_ARG;
  }
  const bool dual = (em == E_DUAL || em == E_DUAL_SWIGLU);
  if (dual && (!p.w1 || !p.s1 || !p.b1 || !aligned16(p.w1) || ((uintptr_t)p.s1 & 7) || ((uintptr_t)p.b1 & 7))) {
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
  if (xm != X_PLAIN && !p.x2) {
    set_error("%s: fused producer needs its second input", who);
    return MTP_ERR_ARG;
  }
  if (p.ldy < p.N) {
    set_error("%s: ldy=%d < N=%d", who, p.ldy, p.N);
    return MTP_ERR_ARG;
  }
  (void)ws;
  (void)ws_bytes;
  Plan pl = make_plan(p.M, p.N, p.K);
  p.chunk = pl.chunk;
  if (p.gs == 64)
    launch_x<0>(xm, em, p, pl, st);
  else
    launch_x<1>(xm, em, p, pl, st);
  return launch_check(who);
}

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

MTP_API size_t mtp_qmv_workspace_bytes(int M, int N, int K, int dual) {
  // The current kernels reduce their K split inside the workgroup.
  (void)M;
  (void)N;
  (void)K;
  (void)dual;
  return 0;
}

MTP_API int mtp_qmv_affine4(const void* x, const void* w, const void* scales, const void* biases, void* y,
                            int M, int N, int K, int group_size, void* ws, size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w, scales, biases, y, M, N, K, group_size);
  return qmm_dispatch(X_PLAIN, E_STORE, p, ws, ws_bytes, (hipStream_t)stream, "mtp_qmv_affine4");
}

MTP_API int mtp_qmv_affine4_residual(const void* x, const void* w, const void* scales, const void* biases,
                                     const void* resid, void* y, int M, int N, int K, int group_size, void* ws,
                                     size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w, scales, biases, y, M, N, K, group_size);
  p.resid = (const uint16_t*)resid;
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

MTP_API int mtp_qmv_affine4_rmsnorm_in(const void* x, const void* norm_w, float eps, const void* w,
                                       const void* scales, const void* biases, void* y, int M, int N, int K,
                                       int group_size, void* ws, size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w, scales, biases, y, M, N, K, group_size);
  p.x2 = (const uint16_t*)norm_w;
  p.eps = eps;
  return qmm_dispatch(X_RMSNORM, E_STORE, p, ws, ws_bytes, (hipStream_t)stream, "mtp_qmv_affine4_rmsnorm_in");
}

MTP_API int mtp_qmv_affine4_rmsnorm_f32(const void* x, const void* norm_w, float eps, const void* w,
                                        const void* scales, const void* biases, float* y, int M, int N, int K,
                                        int group_size, void* ws, size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w, scales, biases, nullptr, M, N, K, group_size);
  p.x2 = (const uint16_t*)norm_w;
  p.eps = eps;
  p.yf = y;
  return qmm_dispatch(norm_w ? X_RMSNORM : X_PLAIN, E_STORE, p, ws, ws_bytes, (hipStream_t)stream,
                      "mtp_qmv_affine4_rmsnorm_f32");
}

MTP_API int mtp_qmv_affine4_rmsnorm_dual(const void* x, const void* norm_w, float eps, const void* w0,
                                         const void* s0, const void* b0, const void* w1, const void* s1,
                                         const void* b1, void* y, int M, int N, int K, int group_size, void* ws,
                                         size_t ws_bytes, void* stream) {
  QmmParams p = base_params(x, w0, s0, b0, y, M, N, K, group_size);
  p.x2 = (const uint16_t*)norm_w;
  p.eps = eps;
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
  Plan pl = make_plan(mrows, N, K);
  p.chunk = pl.chunk;
  dim3 grid(pl.n_blocks, p.row_tiles, E);
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
