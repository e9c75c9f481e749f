// The streaming quantized matmul's kernels and launch planning, shared by
// qmv.hip (entry points, validation, dispatch) and the translation units
// that instantiate the kernel variants of one x mode each (qmv_x*.hip), so
// the variants compile in parallel.
#pragma once

#include "qmv_args.hpp"
#include "qmv_stream.hpp"

#include <stdlib.h>

namespace mtp {

// One workgroup = NW waves over 32 output columns (one MFMA column tile) and
// the whole K range. K is split between the waves by "quads" (4 groups =
// 256 k = one 128 B line per weight row): plain modes give wave w the quads
// w, w+NW, ...; dual modes give the first NW/2 waves matrix 0 and the rest
// matrix 1, each half splitting the quads NW/2 ways. Partials meet in LDS and
// are summed in wave order — deterministic, no global atomics. x is staged in
// chunks of p.chunk quads shared by all waves; weight loads run two quads
// ahead of the MFMAs with no data-dependent branches, so every wave keeps
// 128 B per lane in flight.
// Leaves the final values in fin[M][64] (cols 0..31 matrix 0, 32..63 matrix 1).
template <int NW, int R, int XM, int EM, int GSH>
__device__ __forceinline__ void qmm_body(const QmmParams& p, unsigned char* smem, int nb, int M, int row0,
                                         long long woff, long long soff) {
  constexpr int NT = NW * 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int Q = p.K >> 8;            // quads
  const int CHQ = p.chunk;           // quads per staging chunk
  constexpr bool dual = (EM == E_DUAL || EM == E_DUAL_SWIGLU);
  constexpr int KS = dual ? NW / 2 : NW;   // waves sharing one column tile
  const NibConsts nc = nib_consts();
  const int kw = wave % KS;
  const int which = dual ? (wave / KS) : 0;

  uint4* xa = reinterpret_cast<uint4*>(smem);                                 // [CHQ*4][4][2][M]
  float* xs = reinterpret_cast<float*>(smem + (size_t)CHQ * 4 * 8 * M * 16);  // [CHQ*4][32]
  float* red = reinterpret_cast<float*>(smem);  // [NW][32 m][32 c], reuses the staging area
  __shared__ float s_inv_rms[32];

  // ---- RMSNorm statistics (fp32, fixed order) ----
  if (XM == X_RMSNORM) {
    if (p.ss_in) {
      // Partial sums of squares left by the producer's epilogue, one per
      // 32-column block of the row: lane-strided sums then a fixed butterfly.
      for (int m = wave; m < M; m += NW) {
        float ss = 0.f;
        for (int j = lane; j < p.ss_parts; j += 64) ss += p.ss_in[(size_t)j * 32 + row0 + m];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
        if (lane == 0) s_inv_rms[m] = rsqrtf(ss / (float)p.K + p.eps);
      }
    } else {
      for (int m = wave; m < M; m += NW) {
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
  QuadRegs cur, n1;
  load_quad(q < Q ? q : Q - 1, cur);
  load_quad(q + KS < Q ? q + KS : Q - 1, n1);
  for (int c = 0; c < nchunks; ++c) {
    const int cq0 = c * CHQ;
    const int cq1 = min(Q, cq0 + CHQ);
    // ---- stage x for quads [cq0, cq1) in MFMA A order + group sums ----
    __syncthreads();
    const int ng = 4 * (cq1 - cq0);
    for (int pidx = tid; pidx < ng * M; pidx += NT) {
      const int gl = pidx / M;
      const int m = pidx - gl * M;
      const int kbase = 64 * (4 * cq0 + gl);
      const size_t xo = x_row(p, row0, m) + kbase;
      const float inv = (XM == X_RMSNORM) ? s_inv_rms[m] : 1.f;
      uint4 raw[8], raw2[8];
#pragma unroll
      for (int cc = 0; cc < 8; ++cc) {
        raw[cc] = *reinterpret_cast<const uint4*>(p.x + xo + 8 * cc);
        raw2[cc] = producer_aux<XM>(p, xo + 8 * cc, kbase + 8 * cc);
      }
      float sum = 0.f;
#pragma unroll
      for (int cc = 0; cc < 8; ++cc)   // chunk cc covers k offset 8cc = 32*kq + 8*i within the group
        xa[((gl * 4 + (cc & 3)) * 2 + (cc >> 2)) * M + m] = produce_chunk<XM, false>(raw[cc], raw2[cc], inv, sum);
      xs[gl * 32 + m] = sum;
    }
    for (int idx = tid; idx < ng * 32; idx += NT)
      if ((idx & 31) >= M) xs[idx] = 0.f;
    __syncthreads();

    // ---- this wave's quads inside the chunk ----
    for (; q < cq1; q += KS) {
      QuadRegs n2;
      const int qn = q + 2 * KS;
      load_quad(qn < Q ? qn : Q - 1, n2);
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
          G0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, nibbles_to_bf16(w0[i], nc), G0, 0, 0, 0);
          G1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, nibbles_to_bf16(w1[i], nc), G1, 0, 0, 0);
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
      cur = n1;
      n1 = n2;
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
  float* fin = red + NW * 32 * 32;  // [M][64]
  for (int idx = tid; idx < M * 64; idx += NT) {
    const int m = idx >> 6;
    const int c = idx & 63;
    const int mat = c >> 5;
    float v = 0.f;
    if (!dual && mat == 0) {
#pragma unroll
      for (int w = 0; w < NW; ++w) v += red[(w * 32 + m) * 32 + c];
    } else if (dual) {
#pragma unroll
      for (int w = 0; w < KS; ++w) v += red[((mat * KS + w) * 32 + m) * 32 + (c & 31)];
    }
    fin[idx] = v;
  }
  __syncthreads();
}

// Epilogue from fin[m][64]: columns nb*32 + c, output rows row0 + m. The
// residual mode also leaves, per output row, the sum of squares of this
// block's 32 stored values (fixed order) for a following fused RMSNorm.
__device__ __forceinline__ float* fin_of(unsigned char* smem, int NW) {
  return reinterpret_cast<float*>(smem) + NW * 32 * 32;
}

// ---------------------------------------------------------------------------
// Persistent streaming form of the dense verify matmul.
//
// The grid holds at most as many workgroups as the GPU keeps resident; each
// loops over 32-column tiles nb = blockIdx.x, + gridDim.x, ... Within a tile
// the NW waves split K by quads as in qmm_body. The activations are staged
// into LDS once per workgroup when all of K fits (chunk >= K/256 quads), and
// every wave walks one flat sequence of (tile, quad) items with a two-quad
// prefetch that runs across tile boundaries, so the weight stream does not
// drain between tiles. Per tile: LDS reduction of the wave partials (wave
// order, deterministic) and the shared epilogue.
template <int NW, int R, int XM, int EM, int GSH>
__global__ __launch_bounds__(NW * 64) void qmv_chunked_kernel(QmmParams p) {
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr int NT = NW * 64;
  constexpr bool dual = (EM == E_DUAL || EM == E_DUAL_SWIGLU);
  constexpr int KS = dual ? NW / 2 : NW;
  constexpr int XSW = 2 * R;  // group sums per staged group (rows 0..2R-1)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wave % KS;
  const int which = dual ? (wave / KS) : 0;
  const int M = p.M;
  const int Q = p.K >> 8;
  const int CHQ = p.chunk;
  const bool resident = CHQ >= Q;
  const NibConsts nc = nib_consts();
  const int nchunks = cdiv(Q, CHQ);
  const int G = gridDim.x;

  uint4* xa = reinterpret_cast<uint4*>(smem);                                       // [CHQ*4][4][2][M]
  float* xs = reinterpret_cast<float*>(smem + (size_t)CHQ * 4 * 8 * M * 16);        // [CHQ*4][XSW]
  float* red = xs + CHQ * 4 * XSW;                                                  // [NW][M][32]
  float* fin = red + NW * M * 32;                                                   // [M][64]
  __shared__ float s_inv_rms[32];

  // ---- RMSNorm statistics (once: every tile has the same rows) ----
  if (XM == X_RMSNORM) {
    for (int m = wave; m < M; m += NW) {
      float ss = 0.f;
      if (p.ss_in) {
        for (int j = lane; j < p.ss_parts; j += 64) ss += p.ss_in[(size_t)j * 32 + m];
      } else {
        const uint16_t* xr = p.x + (size_t)m * p.ldx;
#pragma unroll 4
        for (int k = lane * 8; k < p.K; k += 64 * 8) {
          uint4 raw = *reinterpret_cast<const uint4*>(xr + k);
          const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            float a = bf2f((uint16_t)(wv[t] & 0xffff)), b = bf2f((uint16_t)(wv[t] >> 16));
            ss += a * a + b * b;
          }
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
  const uint32_t* W = which ? p.w1 : p.w0;
  const uint16_t* Sc = which ? p.s1 : p.s0;
  const uint16_t* Bi = which ? p.b1 : p.b0;
  const int sgroups = p.K >> (6 + GSH);
  const bool arow = c32 < M;

  // This wave's items: tile j of this workgroup, quad q = kw + t*KS.
  const int qw = (Q > kw) ? cdiv(Q - kw, KS) : 0;
  const int ntiles = cdiv(p.n_blocks - (int)blockIdx.x, G);
  const int nitems = ntiles * qw;

  struct QuadRegs {
    uint4 w[4];
    uint32_t s[2], b[2];
  };
  auto load_item = [&](int i, QuadRegs& qr) {
    int j = 0, q = kw < Q ? kw : Q - 1;
    if (qw > 0) {
      const int ii = i < nitems ? i : nitems - 1;
      j = ii / qw;
      q = kw + (ii - j * qw) * KS;
    }
    const int n = ((int)blockIdx.x + j * G) * 32 + c32;
    const int nrow = n < p.N ? n : 0;
    const uint32_t* wp = W + (size_t)nrow * (p.K >> 3) + kq * 4 + 32 * q;
#pragma unroll
    for (int u = 0; u < 4; ++u) qr.w[u] = *reinterpret_cast<const uint4*>(wp + 8 * u);
    const uint16_t* sr = Sc + (size_t)nrow * sgroups;
    const uint16_t* br = Bi + (size_t)nrow * sgroups;
    if (GSH == 0) {
      const uint2 sv = *reinterpret_cast<const uint2*>(sr + 4 * q);
      const uint2 bv = *reinterpret_cast<const uint2*>(br + 4 * q);
      qr.s[0] = sv.x; qr.s[1] = sv.y;
      qr.b[0] = bv.x; qr.b[1] = bv.y;
    } else {
      qr.s[0] = *reinterpret_cast<const uint32_t*>(sr + 2 * q);
      qr.b[0] = *reinterpret_cast<const uint32_t*>(br + 2 * q);
      qr.s[1] = qr.s[0];
      qr.b[1] = qr.b[0];
    }
  };
  auto scale_of = [&](const uint32_t* v, int u) -> float {
    const uint32_t word = (GSH == 0) ? v[u >> 1] : v[0];
    const int half = (GSH == 0) ? (u & 1) : (u >> 1);
    return bf2f((uint16_t)(half ? (word >> 16) : (word & 0xffff)));
  };

  int item = 0;
  QuadRegs cur, n1;
  load_item(0, cur);
  load_item(1, n1);

  for (int j = 0; j < ntiles; ++j) {
    const int nb = (int)blockIdx.x + j * G;
    const bool valid = nb * 32 + c32 < p.N;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;

    for (int c = 0; c < nchunks; ++c) {
      const int cq0 = c * CHQ;
      const int cq1 = min(Q, cq0 + CHQ);
      if (!resident || j == 0) {
        // ---- stage x for quads [cq0, cq1) in MFMA A order + group sums ----
        __syncthreads();
        const int ng = 4 * (cq1 - cq0);
        for (int pidx = tid; pidx < ng * M; pidx += NT) {
          const int gl = pidx / M;
          const int m = pidx - gl * M;
          const int kbase = 64 * (4 * cq0 + gl);
          const size_t xo = (size_t)m * p.ldx + kbase;
          const float inv = (XM == X_RMSNORM) ? s_inv_rms[m] : 1.f;
          uint4 raw[8], raw2[8];
#pragma unroll
          for (int cc = 0; cc < 8; ++cc) {
            raw[cc] = *reinterpret_cast<const uint4*>(p.x + xo + 8 * cc);
            raw2[cc] = producer_aux<XM>(p, xo + 8 * cc, kbase + 8 * cc);
          }
          float sum = 0.f;
#pragma unroll
          for (int cc = 0; cc < 8; ++cc)
            xa[((gl * 4 + (cc & 3)) * 2 + (cc >> 2)) * M + m] = produce_chunk<XM, false>(raw[cc], raw2[cc], inv, sum);
          xs[gl * XSW + m] = sum;
        }
        for (int idx = tid; idx < ng * XSW; idx += NT)
          if ((idx % XSW) >= M) xs[idx] = 0.f;
        __syncthreads();
      }

      // ---- this wave's quads of tile j inside the chunk ----
      int q = cq0 + ((kw - cq0) % KS + KS) % KS;
      for (; q < cq1; q += KS) {
        QuadRegs n2;
        load_item(item + 2, n2);
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
            G0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, nibbles_to_bf16(w0[i], nc), G0, 0, 0, 0);
            G1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, nibbles_to_bf16(w1[i], nc), G1, 0, 0, 0);
          }
          const float s0 = scale_of(cur.s, u), s1 = scale_of(cur.s, u + 1);
          const float cb0 = scale_of(cur.b, u) - 128.f * s0;
          const float cb1 = scale_of(cur.b, u + 1) - 128.f * s1;
          const float* xr0 = xs + (gq + u) * XSW + 4 * kq;
          const float* xr1 = xs + (gq + u + 1) * XSW + 4 * kq;
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int off = 8 * (r >> 2) + (r & 3);
            acc[r] = fmaf(s0, G0[r], fmaf(cb0, xr0[off], acc[r]));
            acc[r] = fmaf(s1, G1[r], fmaf(cb1, xr1[off], acc[r]));
          }
        }
        cur = n1;
        n1 = n2;
        ++item;
      }
    }

    // ---- reduce the K-split waves (wave order) and finish the tile ----
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int m = 8 * (r >> 2) + 4 * kq + (r & 3);
      if (m < M) red[(wave * M + m) * 32 + c32] = valid ? acc[r] : 0.f;
    }
    __syncthreads();
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
    __syncthreads();
    qmm_epilogue<NW, EM>(p, fin, nb, M, 0);
  }
}

template <int NW, int R, int XM, int EM, int GSH, bool PK, bool MF = false, int NRT = 3>
__global__ __launch_bounds__(NW * 64) void qmv_stream_kernel(QmmParams p) {
  qmv_stream_body<NW, R, XM, EM, GSH, PK, MF, NRT>(p, (int)blockIdx.x, (int)gridDim.x, NoHook{});
}


// ---------------------------------------------------------------------------
// Host side: split planning and dispatch.

struct Plan {
  int n_blocks, chunk, nw;
  bool resident;
  size_t lds;
  int split = 0, xq = 0;   // full K split: parts, quads of x each part stages
};

static int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return (v && *v) ? atoi(v) : dflt;
}

// Group-sum rows (2R) the LDS plan reserves: 5..8 rows get R = 8's, which
// the 16x16x32 form (layout 2) uses there (the 32x32x16 form's R = 4 needs
// less), so one plan serves both layouts.
static int r_of(int M) { return M <= 4 ? 4 : (M <= 16 ? 8 : 16); }

// LDS of the gathered (chunked) kernel: staged x per quad (4 groups x
// (8*M*16 B + 32 floats)); the K-split reduction reuses the same area.
static size_t lds_bytes(int chunk_q, int M, int nw) {
  size_t stage = (size_t)chunk_q * 4 * (8 * M * 16 + 32 * 4);
  size_t red = (size_t)nw * 32 * 32 * 4 + (size_t)M * 64 * 4;
  return stage > red ? stage : red;
}

static int max_chunk_quads(int M) {
  int ch = (60 * 1024) / (4 * (8 * M * 16 + 128));
  return ch < 1 ? 1 : ch;
}

// LDS of the streaming kernels: staged x (+ 2R group sums per group), the
// wave partials [NW][M][32], the finished tile [M][64] and a 16 B zero block.
static size_t stream_lds(int chunk_q, int M, int nw) {
  return xa_bytes(4 * chunk_q, M) + (size_t)chunk_q * 4 * 2 * r_of(M) * 4 + (size_t)nw * M * 32 * 4 +
         (size_t)M * 64 * 4;
}

static constexpr size_t kLdsMax = 160 * 1024 - 256;   // gfx950: 160 KiB of LDS per CU

static constexpr size_t kLdsBudget = 65536 - 256;

// Waves per workgroup: 8 when the column tiles alone cannot give every CU
// two workgroups (small N: q|k|v, o, down), else 4. All of K is staged once
// per workgroup when it fits in LDS, else in chunks per tile.
static Plan make_plan(int M, int N, int K) {
  Plan pl;
  pl.n_blocks = cdiv(N, 32);
  const int Q = K / 256;
  const int nw_env = env_int("MTPLX_AMD_QMV_WAVES", 0);
  pl.nw = (nw_env == 4 || nw_env == 8) ? nw_env : (pl.n_blocks < 512 ? 8 : 4);
  const int cap = env_int("MTPLX_AMD_QMV_CHUNK_QUADS", 0);
  pl.resident = cap <= 0 && stream_lds(Q, M, pl.nw) <= kLdsMax;
  if (pl.resident) {
    pl.chunk = Q;
  } else {
    int ch = Q;
    while (ch > 1 && stream_lds(ch, M, pl.nw) > kLdsBudget) --ch;
    if (cap > 0 && cap < ch) ch = cap;
    pl.chunk = ch;
  }
  pl.lds = stream_lds(pl.chunk, M, pl.nw);
  return pl;
}

// Full K split (packed weights, x too large for LDS): the fewest parts whose
// share of x fits, its fp32 partials [tiles][parts][M][64], then one arrival
// counter per tile.
static int full_split_parts(int M, int K, int nw) {
  const int Q = K >> 8;
  for (int S = 2; S <= Q; ++S)
    if (stream_lds(cdiv(Q, S), M, nw) <= kLdsMax) return S;
  return 0;
}
static size_t full_split_partial_bytes(int M, int N, int K, int nw) {
  const size_t b = (size_t)cdiv(N, 32) * full_split_parts(M, K, nw) * M * 64 * sizeof(float);
  return (b + 255) / 256 * 256;
}
static size_t full_split_ws_bytes(int M, int N, int K, int nw) {
  return kCounterBytes + full_split_partial_bytes(M, N, K, nw);
}


// Grid of the streaming kernel: every column tile once when they fit in the
// resident workgroups, else as many workgroups as stay resident (each then
// loops over several tiles).
template <typename K>
static int stream_grid(K kernel, int nt, size_t lds, int n_blocks) {
  const int forced = env_int("MTPLX_AMD_QMV_GRID", 0);
  if (forced > 0) return forced < n_blocks ? forced : n_blocks;
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, nt, lds) != hipSuccess || occ < 1) occ = 1;
  const int resident = occ * device_cus();
  return n_blocks < resident ? n_blocks : resident;
}

template <typename K>
static void launch_one(K k, const Plan& pl, int nt, hipStream_t st, const QmmParams& q) {
  // A failure here surfaces as a launch error, which the caller checks.
  if (pl.lds > 65536) (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.lds);
  hipLaunchKernelGGL(k, dim3(stream_grid(k, nt, pl.lds, pl.n_blocks)), dim3(nt), pl.lds, st, q);
}

// Tail split of the per-tile kernel: when T tiles leave E = T mod CUs
// leftover tiles and E divides the CU count, the T - E full tiles run as
// usual and every leftover tile is split by K into S = CUs / E parts, so the
// last round puts exactly one part on every CU instead of a whole tile on E
// of them; with T <= CUs every tile is split into floor(CUs / T) parts. All
// workgroups must be resident at once (one round).
template <typename K>
static bool tail_launch(K kernel, const Plan& pl, int nt, hipStream_t st, QmmParams q) {
  const int cus = device_cus();
  const int T = pl.n_blocks;
  const int Q = q.K >> 8;
  if (pl.split > 1) {
    // Full K split: as many tile groups as the resident workgroups allow
    // (each group of pl.split workgroups covers the same tiles).
    if (pl.lds > 65536) (void)hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  (int)pl.lds);
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, nt, pl.lds) != hipSuccess || occ < 1) occ = 1;
    int groups = occ * cus / pl.split;
    if (groups > T) groups = T;
    if (groups < 1) groups = 1;
    q.tail_first = 0;
    q.tail_split = pl.split;
    q.full_split = 1;
    q.xq = pl.xq;
    hipLaunchKernelGGL(kernel, dim3(groups * pl.split), dim3(nt), pl.lds, st, q);
    return true;
  }
  // Fewer tiles than CUs (small N: the router, shared-expert and attention
  // projections at M = 16): every tile is split by K into floor(CUs / T)
  // parts (at most one per quad), so the launch keeps up to every CU busy
  // instead of T of them.
  int E, S, grid;
  if (T <= cus) {
    E = T;
    S = cus / T;
    if (S > Q) S = Q;
    if (S < 2) return false;
    grid = T * S;
  } else {
    E = T % cus;
    if (E == 0 || cus % E) return false;
    S = cus / E;
    if (S < 2 || S > Q) return false;
    grid = T - E + cus;
  }
  if (pl.lds > 65536) (void)hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                (int)pl.lds);
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, nt, pl.lds) != hipSuccess) return false;
  if (grid > occ * cus) return false;
  q.tail_first = T - E;
  q.tail_split = S;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(nt), pl.lds, st, q);
  return true;
}

// Ring depth of the layout-2 kernels: one slot when a wave takes at most
// three quads of a tile, else two (graph-timed: o 9.5 -> 8.5 us, q|k|v
// 11.2 -> 9.8 us, gate/up 24.5 -> 21.9 us against three slots).
static bool mf_short_ring(const QmmParams& q, int nw, int em) {
  const int ks = (em == E_DUAL || em == E_DUAL_SWIGLU) ? nw / 2 : nw;
  return cdiv(q.K >> 8, ks) <= 3;
}

// R = 4: up to 4 rows; R = 8: up to 16 rows (quad_mma16x16).
template <int NW, int R, int XM, int EM, int NRT>
static void launch_mf(const QmmParams& q, const Plan& pl, hipStream_t st) {
  if (!(q.tail_ok && tail_launch(qmv_stream_kernel<NW, R, XM, EM, 0, true, true, NRT>, pl, NW * 64, st, q)))
    launch_one(qmv_stream_kernel<NW, R, XM, EM, 0, true, true, NRT>, pl, NW * 64, st, q);
}

template <int NW, int R, int XM, int EM, int GSH>
static void launch_rk(const QmmParams& q, const Plan& pl, hipStream_t st) {
  if constexpr (R == 4 || R == 8) {
    if (q.packed == 2) {   // 16x16x32 layout: M <= 4 at R = 4, M <= 16 at R = 8 (checked by the caller)
      if (mf_short_ring(q, NW, EM))
        launch_mf<NW, R, XM, EM, 1>(q, pl, st);
      else
        launch_mf<NW, R, XM, EM, 2>(q, pl, st);
      return;
    }
  }
  if (q.packed && (R <= 8 || pl.split > 1) && q.tail_ok &&
      tail_launch(qmv_stream_kernel<NW, R, XM, EM, 0, true>, pl, NW * 64, st, q))
    return;
  if constexpr (XM == X_PRE) {   // packed weights only (checked by the caller)
    launch_one(qmv_stream_kernel<NW, R, XM, EM, 0, true>, pl, NW * 64, st, q);
  } else {
    if (q.packed)
      launch_one(qmv_stream_kernel<NW, R, XM, EM, 0, true>, pl, NW * 64, st, q);
    else if (pl.resident)
      launch_one(qmv_stream_kernel<NW, R, XM, EM, GSH, false>, pl, NW * 64, st, q);
    else
      launch_one(qmv_chunked_kernel<NW, R, XM, EM, GSH>, pl, NW * 64, st, q);
  }
}

template <int NW, int XM, int EM, int GSH>
static void launch_n(const QmmParams& p, const Plan& pl, hipStream_t st) {
  QmmParams q = p;
  q.n_blocks = pl.n_blocks;
  if (p.M <= (p.packed == 2 ? 4 : 8))
    launch_rk<NW, 4, XM, EM, GSH>(q, pl, st);
  else if (p.M <= 16)
    launch_rk<NW, 8, XM, EM, GSH>(q, pl, st);
  else
    launch_rk<NW, 16, XM, EM, GSH>(q, pl, st);
}

template <int XM, int EM, int GSH>
static void launch_r(const QmmParams& p, const Plan& pl, hipStream_t st) {
  if (pl.nw == 8)
    launch_n<8, XM, EM, GSH>(p, pl, st);
  else
    launch_n<4, XM, EM, GSH>(p, pl, st);
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


// q|k|v with the RoPE epilogue: packed weights, R = 4 (M <= 8) or 8 (M <= 16);
// layout 2: R = 4 up to 4 rows, R = 8 (16x16x32 on 16 rows) up to 16.
template <int XM>
static void launch_rope(const QmmParams& q, const Plan& pl, hipStream_t st) {
  if (q.packed == 2 && q.M > 4) {
    const bool sh = mf_short_ring(q, pl.nw, E_ROPE_QKV);
    if (pl.nw == 8 && sh)
      launch_one(qmv_stream_kernel<8, 8, XM, E_ROPE_QKV, 0, true, true, 1>, pl, 8 * 64, st, q);
    else if (pl.nw == 8)
      launch_one(qmv_stream_kernel<8, 8, XM, E_ROPE_QKV, 0, true, true, 2>, pl, 8 * 64, st, q);
    else if (sh)
      launch_one(qmv_stream_kernel<4, 8, XM, E_ROPE_QKV, 0, true, true, 1>, pl, 4 * 64, st, q);
    else
      launch_one(qmv_stream_kernel<4, 8, XM, E_ROPE_QKV, 0, true, true, 2>, pl, 4 * 64, st, q);
  } else if (q.packed == 2) {
    const bool sh = mf_short_ring(q, pl.nw, E_ROPE_QKV);
    if (pl.nw == 8 && sh)
      launch_one(qmv_stream_kernel<8, 4, XM, E_ROPE_QKV, 0, true, true, 1>, pl, 8 * 64, st, q);
    else if (pl.nw == 8)
      launch_one(qmv_stream_kernel<8, 4, XM, E_ROPE_QKV, 0, true, true, 2>, pl, 8 * 64, st, q);
    else if (sh)
      launch_one(qmv_stream_kernel<4, 4, XM, E_ROPE_QKV, 0, true, true, 1>, pl, 4 * 64, st, q);
    else
      launch_one(qmv_stream_kernel<4, 4, XM, E_ROPE_QKV, 0, true, true, 2>, pl, 4 * 64, st, q);
  } else if (q.M > 8) {   // 9..16 rows: R = 8 (layout 1)
    if (pl.nw == 8)
      launch_one(qmv_stream_kernel<8, 8, XM, E_ROPE_QKV, 0, true>, pl, 8 * 64, st, q);
    else
      launch_one(qmv_stream_kernel<4, 8, XM, E_ROPE_QKV, 0, true>, pl, 4 * 64, st, q);
  } else if (pl.nw == 8) {
    launch_one(qmv_stream_kernel<8, 4, XM, E_ROPE_QKV, 0, true>, pl, 8 * 64, st, q);
  } else {
    launch_one(qmv_stream_kernel<4, 4, XM, E_ROPE_QKV, 0, true>, pl, 4 * 64, st, q);
  }
}

// One per x mode, each in its own translation unit: launch the kernel
// variant for epilogue em (group size 64 when gsh == 0, else 128).
void qmv_launch_plain(int em, int gsh, const QmmParams& p, const Plan& pl, hipStream_t st);
void qmv_launch_swiglu(int em, int gsh, const QmmParams& p, const Plan& pl, hipStream_t st);
void qmv_launch_pre(int em, int gsh, const QmmParams& p, const Plan& pl, hipStream_t st);
void qmv_launch_rmsnorm(int em, int gsh, const QmmParams& p, const Plan& pl, hipStream_t st);
// q|k|v with the RoPE epilogue (x plain or RMSNorm).
void qmv_launch_rope_qkv(int xm, const QmmParams& p, const Plan& pl, hipStream_t st);

}  // namespace mtp
