// General affine quantized matmul (4- or 8-bit, group 32/64/128) and the
// activation chunk-sum table of the cross-row lane.
//
//   y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/gs] + b[n, k/gs])
//
// Weight format (MLX's affine quantization, as the reference's verify lanes
// read it: mtplx/verify_qmv.py:1256-1377 for 8-bit, mtplx/kernels/
// qmv4_matmul.py:158 / mtplx/verify_crossrow.py:57 for group 32): uint32
// [N, K*bits/32] with little-endian fields (value i of a word in bits
// bits*i .. bits*i + bits - 1), bf16 scales/biases [N, K/gs].
//
// This is the lane for the formats the MFMA streaming kernel does not take
// (8-bit, group 32). It is a VALU kernel: a workgroup of 4 waves owns 64
// output columns, each wave 16 of them with the wave's four 16-lane groups
// splitting every 32-k block round robin; x is staged per 512-k chunk in
// LDS as fp32 with its 32-k block sums, so each block finishes as
// s * sum(q x) + b * sum(x). The four lane groups meet by shuffles (fixed
// order), then lane group 0 stores. Rows run in launches of up to 8.
#include "common.hpp"

namespace mtp {

namespace {

constexpr int kGenKC = 512;                 // k per staged chunk
constexpr int kGenRows = 8;                 // rows per launch
constexpr int kGenPad = kGenKC + kGenKC / 32;   // one pad float per 32-k block: no bank conflicts

struct GenericArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  float* yf;
  // Optional chunk-sum table of the cross-row lane (mtp_chunk_sums layout:
  // [(kb*32 + lane)*8 + m] = sum of x[m, kb*512 + lane*16 .. +16)); when
  // given, each 32-k block sum is read from it (two 16-value slices) instead
  // of being summed from the staged x.
  const float* xsums;
  int M, N, K, gs, ldx, ldy;
};

template <int BITS>
__global__ __launch_bounds__(256) void qmv_generic_kernel(GenericArgs a) {
  constexpr int VPW = 32 / BITS;             // values per word
  constexpr int WPB = 32 / VPW;              // words per 32-k block
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  __shared__ float xs[kGenRows][kGenPad];
  __shared__ float xsum[kGenRows][kGenKC / 32];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g4 = lane >> 4;
  const int col = blockIdx.x * 64 + wave * 16 + (lane & 15);
  const bool cv = col < a.N;
  const int M = a.M;
  const int K = a.K;
  const uint32_t* wr = a.w + (size_t)(cv ? col : 0) * (K / VPW);
  const uint16_t* sr = a.s + (size_t)(cv ? col : 0) * (K / a.gs);
  const uint16_t* br = a.b + (size_t)(cv ? col : 0) * (K / a.gs);
  float acc[kGenRows];
#pragma unroll
  for (int m = 0; m < kGenRows; ++m) acc[m] = 0.f;

  for (int k0 = 0; k0 < K; k0 += kGenKC) {
    const int kc = (K - k0) < kGenKC ? (K - k0) : kGenKC;   // a multiple of 32
    const int nblk = kc >> 5;
    __syncthreads();   // the previous chunk's readers are done
    for (int i = tid; i < M * kc; i += 256) {
      const int m = i / kc, k = i - m * kc;
      xs[m][k + (k >> 5)] = bf2f(a.x[(size_t)m * a.ldx + k0 + k]);
    }
    __syncthreads();
    for (int i = tid; i < M * nblk; i += 256) {
      const int m = i / nblk, blk = i - m * nblk;
      float t = 0.f;
      if (a.xsums) {   // k0 is a multiple of 512: chunk kb = k0 / 512, slices 2 blk and 2 blk + 1
        const float* cs = a.xsums + ((size_t)(k0 >> 9) * 32 + 2 * blk) * 8 + m;
        t = cs[0] + cs[8];
      } else {
        const float* xp = &xs[m][blk * 33];
        for (int j = 0; j < 32; ++j) t += xp[j];
      }
      xsum[m][blk] = t;
    }
    __syncthreads();
    for (int blk = g4; blk < nblk; blk += 4) {
      const int kk = k0 + blk * 32;
      uint32_t wv[WPB];
#pragma unroll
      for (int u = 0; u < WPB; u += 4) {
        const uint4 v = *reinterpret_cast<const uint4*>(wr + kk / VPW + u);
        wv[u] = v.x;
        wv[u + 1] = v.y;
        wv[u + 2] = v.z;
        wv[u + 3] = v.w;
      }
      const int gi = kk / a.gs;
      const float sc = bf2f(sr[gi]), bi = bf2f(br[gi]);
      float qx[kGenRows];
#pragma unroll
      for (int m = 0; m < kGenRows; ++m) qx[m] = 0.f;
#pragma unroll
      for (int j = 0; j < 32; j += 4) {
        float q[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) q[t] = (float)((wv[(j + t) / VPW] >> (BITS * ((j + t) % VPW))) & MASK);
#pragma unroll
        for (int m = 0; m < kGenRows; ++m) {
          if (m < M) {
            const float4 xv = *reinterpret_cast<const float4*>(&xs[m][blk * 33 + j]);
            qx[m] = fmaf(q[0], xv.x, qx[m]);
            qx[m] = fmaf(q[1], xv.y, qx[m]);
            qx[m] = fmaf(q[2], xv.z, qx[m]);
            qx[m] = fmaf(q[3], xv.w, qx[m]);
          }
        }
      }
#pragma unroll
      for (int m = 0; m < kGenRows; ++m)
        if (m < M) acc[m] = fmaf(sc, qx[m], fmaf(bi, xsum[m][blk], acc[m]));
    }
  }
#pragma unroll
  for (int m = 0; m < kGenRows; ++m) {
    acc[m] += __shfl_xor(acc[m], 16, 64);
    acc[m] += __shfl_xor(acc[m], 32, 64);
  }
  if (g4 == 0 && cv) {
#pragma unroll
    for (int m = 0; m < kGenRows; ++m) {
      if (m < M) {
        if (a.yf)
          a.yf[(size_t)m * a.ldy + col] = round_bf(acc[m]);
        else
          a.y[(size_t)m * a.ldy + col] = f2bf(acc[m]);
      }
    }
  }
}

// out[(kb * 32 + lane) * 8 + m] = sum of x[m, kb*512 + lane*16 + i], i < 16,
// added in index order (fp32); rows m >= M are zero.
__global__ __launch_bounds__(256) void chunk_sums_kernel(const uint16_t* x, int M, int K, int ldx, float* out) {
  const int slot = blockIdx.x * 256 + threadIdx.x;
  const int lanes = (K / 512) * 32;
  if (slot >= lanes) return;
  const int base = (slot >> 5) * 512 + (slot & 31) * 16;
  for (int m = 0; m < 8; ++m) {
    float t = 0.f;
    if (m < M)
      for (int i = 0; i < 16; ++i) t += bf2f(x[(size_t)m * ldx + base + i]);
    out[(size_t)slot * 8 + m] = t;
  }
}

}  // namespace

}  // namespace mtp

using namespace mtp;

static int qmv_affine_run(const void* x, const float* xsums, const void* w, const void* scales, const void* biases,
                          void* y, void* yf, int M, int N, int K, int group_size, int bits, void* stream,
                          const char* who) {
  if (!x || !w || !scales || !biases || (!y && !yf) || M < 1 || N < 1 || K < 32 || K % 32) {
    set_error("%s: bad arguments (non-null x/w/scales/biases/output, M, N >= 1, K a positive multiple of 32)", who);
    return MTP_ERR_ARG;
  }
  if (bits != 4 && bits != 8) {
    set_error("%s: %d-bit weights unsupported (4 or 8)", who, bits);
    return MTP_ERR_UNSUPPORTED;
  }
  if ((group_size != 32 && group_size != 64 && group_size != 128) || K % group_size) {
    set_error("%s: group_size %d unsupported or does not divide K=%d (32, 64, 128)", who, group_size, K);
    return MTP_ERR_UNSUPPORTED;
  }
  if (((uintptr_t)w & 15)) {
    set_error("%s: weights must be 16-byte aligned", who);
    return MTP_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((N + 63) / 64);
  for (int r0 = 0; r0 < M; r0 += kGenRows) {
    GenericArgs a;
    a.x = (const uint16_t*)x + (size_t)r0 * K;
    a.w = (const uint32_t*)w;
    a.s = (const uint16_t*)scales;
    a.b = (const uint16_t*)biases;
    a.y = y ? (uint16_t*)y + (size_t)r0 * N : nullptr;
    a.yf = yf ? (float*)yf + (size_t)r0 * N : nullptr;
    a.xsums = xsums;   // (M <= 8 when given: one launch)
    a.M = (M - r0) < kGenRows ? (M - r0) : kGenRows;
    a.N = N;
    a.K = K;
    a.gs = group_size;
    a.ldx = K;
    a.ldy = N;
    if (bits == 4)
      hipLaunchKernelGGL(qmv_generic_kernel<4>, grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL(qmv_generic_kernel<8>, grid, dim3(256), 0, st, a);
    const int rc = launch_check(who);
    if (rc) return rc;
  }
  return MTP_OK;
}

MTP_API int mtp_qmv_affine(const void* x, const void* w, const void* scales, const void* biases, void* y, void* yf,
                           int M, int N, int K, int group_size, int bits, void* stream) {
  return qmv_affine_run(x, nullptr, w, scales, biases, y, yf, M, N, K, group_size, bits, stream, "mtp_qmv_affine");
}

MTP_API int mtp_crossrow_qmm(const void* x, const float* xsums, const void* w, const void* scales,
                             const void* biases, void* y, int M, int N, int K, int group_size, void* stream) {
  const char* who = "mtp_crossrow_qmm";
  if (!xsums || M < 1 || M > kGenRows || K < 512 || K % 512) {
    set_error("%s: need the chunk-sum table (mtp_chunk_sums), 1 <= M <= %d and K a positive multiple of 512", who,
              kGenRows);
    return MTP_ERR_ARG;
  }
  if (group_size != 32 && group_size != 64) {
    set_error("%s: group_size %d unsupported (the cross-row lane takes 32 or 64)", who, group_size);
    return MTP_ERR_UNSUPPORTED;
  }
  return qmv_affine_run(x, xsums, w, scales, biases, y, nullptr, M, N, K, group_size, 4, stream, who);
}

MTP_API int mtp_chunk_sums(const void* x, int M, int K, float* out, void* stream) {
  if (!x || !out || M < 1 || M > 8 || K < 512 || K % 512) {
    set_error("mtp_chunk_sums: bad arguments (1 <= M <= 8, K a positive multiple of 512)");
    return MTP_ERR_ARG;
  }
  const int lanes = (K / 512) * 32;
  hipLaunchKernelGGL(chunk_sums_kernel, dim3((lanes + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, M, K, K, out);
  return launch_check("mtp_chunk_sums");
}
