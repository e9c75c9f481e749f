// Glue around the verify matmuls for the synthetic dense/MoE verify step:
// quantized embedding gather, RoPE on the fused q|k|v rows with per-request
// offsets (writing K/V straight into the ragged cache), standalone RMSNorm.
//
// RoPE is the non-interleaved (rotate-half) form with fp32 angles
// theta_i = pos * 2^(-(2i/D) * log2(base)), as MLX's fast rope computes it;
// per-row positions come from q_start[b] + i on the GPU
// (tests/test_ragged_kv_cache.py:62-100 gate 5, mtplx/ragged_kv_cache.py:201).
#include "common.hpp"

namespace mtp {

// out[m, :] = dequant(W[tok[m], :]) in bf16; 4-bit affine rows [V, H/8].
__global__ void embed_affine4_kernel(const int32_t* tok, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                     uint16_t* out, int M, int H, int gs, int V, int32_t* status) {
  const int m = blockIdx.y;
  const int t = tok[m];
  const bool ok = t >= 0 && t < V;
  if (!ok && threadIdx.x == 0 && blockIdx.x == 0 && status) atomicOr(status, 1);
  for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < H / 8; j += gridDim.x * blockDim.x) {
    uint4 o = make_uint4(0, 0, 0, 0);
    if (ok) {
      const uint32_t word = w[(size_t)t * (H / 8) + j];
      const int g = (8 * j) / gs;
      const float sc = bf2f(s[(size_t)t * (H / gs) + g]);
      const float bi = bf2f(b[(size_t)t * (H / gs) + g]);
      uint16_t e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = f2bf((float)((word >> (4 * i)) & 0xF) * sc + bi);
      o.x = e[0] | ((uint32_t)e[1] << 16);
      o.y = e[2] | ((uint32_t)e[3] << 16);
      o.z = e[4] | ((uint32_t)e[5] << 16);
      o.w = e[6] | ((uint32_t)e[7] << 16);
    }
    *reinterpret_cast<uint4*>(out + (size_t)m * H + 8 * j) = o;
  }
}

// qkv rows [M = B*L, (Hq + 2*Hkv) * D]; q_out [B, Hq, L, D]; cache [B, Hkv, cap, D].
// One thread per (row, head, rotary pair) for q and k; v copied 8 elements per thread.
__global__ void rope_qkv_kernel(const uint16_t* qkv, const int32_t* q_start, const int32_t* q_lens, uint16_t* q_out,
                                uint16_t* kc, uint16_t* vc, int B, int L, int Hq, int Hkv, int D, int cap,
                                float log2_base, int32_t* status, int kv_blocked) {
  const int half = D / 2;
  const int m = blockIdx.y;
  const int b = m / L;
  const int i = m - b * L;
  const int len = q_lens ? q_lens[b] : L;
  const int pos = q_start[b] + i;
  const int width = (Hq + 2 * Hkv) * D;
  const uint16_t* row = qkv + (size_t)m * width;
  const int nrot = (Hq + Hkv) * half;
  for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < nrot + Hkv * D / 8; t += gridDim.x * blockDim.x) {
    if (t < nrot) {
      const int head = t / half;
      const int j = t - head * half;
      const uint16_t* src = row + head * D;
      uint16_t o1, o2;
      rope_pair(bf2f(src[j]), bf2f(src[j + half]), pos, j, D, log2_base, o1, o2);
      if (head < Hq) {
        uint16_t* dst = q_out + (((size_t)b * Hq + head) * L + i) * D;
        dst[j] = o1;
        dst[j + half] = o2;
      } else if (i < len) {
        if (pos < 0 || pos >= cap) {
          if (status) atomicOr(status, 1);
          continue;
        }
        if (kv_blocked) {
          uint16_t* kh = kc + ((size_t)b * Hkv + (head - Hq)) * cap * D;
          kh[kblk_index(pos, j)] = o1;
          kh[kblk_index(pos, j + half)] = o2;
        } else {
          uint16_t* dst = kc + (((size_t)b * Hkv + (head - Hq)) * cap + pos) * D;
          dst[j] = o1;
          dst[j + half] = o2;
        }
      }
    } else if (i < len) {
      const int e = (t - nrot) * 8;
      const int head = e / D;
      const int d = e - head * D;
      if (pos < 0 || pos >= cap) {
        if (status) atomicOr(status, 1);
        continue;
      }
      const uint4 val = *reinterpret_cast<const uint4*>(row + (Hq + Hkv) * D + e);
      if (kv_blocked) {   // operand-major blocks: the 8 values go to 8 d positions of their key block
        uint16_t* vh = vc + ((size_t)b * Hkv + head) * cap * D;
        const uint32_t w4[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          vh[vblk_index(pos, d + 2 * t)] = (uint16_t)(w4[t] & 0xffff);
          vh[vblk_index(pos, d + 2 * t + 1)] = (uint16_t)(w4[t] >> 16);
        }
      } else {
        *reinterpret_cast<uint4*>(vc + (((size_t)b * Hkv + head) * cap + pos) * D + d) = val;
      }
    }
  }
}

// Ragged rows into the operand-major block cache: packed row m belongs to
// request b with row_off[b] <= m < row_off[b+1] (i = m - row_off[b], position
// q_start[b] + i); q -> q_out [B, Hq, Lmax, D]; K/V into request b's blocks
// (head h at kv_off[b] + h * nblk_b, nblk_b = (kv_off[b+1] - kv_off[b]) / Hkv;
// kv_off null: a uniform capacity cap). D = 128.
__global__ void rope_qkv_blocks_kernel(const uint16_t* qkv, const int32_t* row_off, const int32_t* q_start,
                                       const int32_t* kv_off, uint16_t* q_out, uint16_t* kc, uint16_t* vc, int B,
                                       int Lmax, int Hq, int Hkv, int D, int cap, float log2_base, int32_t* status) {
  const int half = D / 2;
  const int m = blockIdx.y;
  int lo = 0, hi = B;   // the b with row_off[b] <= m < row_off[b+1]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (row_off[mid] <= m) lo = mid; else hi = mid;
  }
  const int b = lo;
  const int i = m - row_off[b];
  const int pos = q_start[b] + i;
  const int nblk = kv_off ? (kv_off[b + 1] - kv_off[b]) / Hkv : cap / 32;
  const int capb = 32 * nblk;
  const size_t blk0 = kv_off ? (size_t)kv_off[b] : (size_t)b * Hkv * nblk;
  const bool in_cap = pos >= 0 && pos < capb;
  const int width = (Hq + 2 * Hkv) * D;
  const uint16_t* row = qkv + (size_t)m * width;
  const int nrot = (Hq + Hkv) * half;
  for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < nrot + Hkv * D / 8; t += gridDim.x * blockDim.x) {
    if (t < nrot) {
      const int head = t / half;
      const int j = t - head * half;
      const uint16_t* src = row + head * D;
      uint16_t o1, o2;
      rope_pair(bf2f(src[j]), bf2f(src[j + half]), pos, j, D, log2_base, o1, o2);
      if (head < Hq) {
        uint16_t* dst = q_out + (((size_t)b * Hq + head) * Lmax + i) * D;
        dst[j] = o1;
        dst[j + half] = o2;
      } else if (!in_cap) {
        if (status) atomicOr(status, 1);
      } else {
        uint16_t* kh = kc + (blk0 + (size_t)(head - Hq) * nblk) * 4096;
        kh[kblk_index(pos, j)] = o1;
        kh[kblk_index(pos, j + half)] = o2;
      }
    } else if (!in_cap) {
      if (status) atomicOr(status, 1);
    } else {
      const int e = (t - nrot) * 8;
      const int head = e / D;
      const int d = e - head * D;
      const uint4 val = *reinterpret_cast<const uint4*>(row + (Hq + Hkv) * D + e);
      uint16_t* vh = vc + (blk0 + (size_t)head * nblk) * 4096;
      const uint32_t w4[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        vh[vblk_index(pos, d + 2 * u)] = (uint16_t)(w4[u] & 0xffff);
        vh[vblk_index(pos, d + 2 * u + 1)] = (uint16_t)(w4[u] >> 16);
      }
    }
  }
}

// One workgroup per row. Rows whose width is a multiple of 8 and at most
// 8192 are read once, 16 bytes per load, and kept in registers between the
// sum of squares and the scaled store; others take a strided loop.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* x, const uint16_t* w, uint16_t* out, int H,
                                                      float eps) {
  constexpr int kCh = 4;   // 8-value chunks per thread on the fast path
  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* xr = x + (size_t)m * H;
  uint16_t* orow = out + (size_t)m * H;
  __shared__ float red[4];
  const bool fast = (H % 8) == 0 && H <= 256 * 8 * kCh;
  float ss = 0.f;
  uint4 xv[kCh];
  if (fast) {
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const int k = (tid + c * 256) * 8;
      xv[c] = k < H ? *reinterpret_cast<const uint4*>(xr + k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const uint32_t u[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = __uint_as_float(u[j] << 16), b = __uint_as_float(u[j] & 0xffff0000u);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
  } else {
    for (int k = tid; k < H; k += 256) {
      const float a = bf2f(xr[k]);
      ss += a * a;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float inv = rsqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)H + eps);
  if (fast) {
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
      const int k = (tid + c * 256) * 8;
      if (k < H) {
        const uint4 wv = *reinterpret_cast<const uint4*>(w + k);
        const uint32_t u[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
        const uint32_t g[4] = {wv.x, wv.y, wv.z, wv.w};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a = __uint_as_float(u[j] << 16) * inv * __uint_as_float(g[j] << 16);
          const float b = __uint_as_float(u[j] & 0xffff0000u) * inv * __uint_as_float(g[j] & 0xffff0000u);
          o[j] = (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
        }
        *reinterpret_cast<uint4*>(orow + k) = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  } else {
    for (int k = tid; k < H; k += 256) orow[k] = f2bf(bf2f(xr[k]) * inv * bf2f(w[k]));
  }
}

}  // namespace mtp

using namespace mtp;

MTP_API int mtp_embed_affine4(const int32_t* tokens, const void* w, const void* scales, const void* biases, void* out,
                              int M, int H, int V, int group_size, int32_t* status, void* stream) {
  if (!tokens || !w || !scales || !biases || !out || M < 1 || H < 8 || H % 8 || group_size < 8 ||
      H % group_size || group_size % 8) {
    set_error("mtp_embed_affine4: bad arguments");
    return MTP_ERR_ARG;
  }
  dim3 grid(cdiv(H / 8, 256), M);
  hipLaunchKernelGGL(embed_affine4_kernel, grid, dim3(256), 0, (hipStream_t)stream, tokens, (const uint32_t*)w,
                     (const uint16_t*)scales, (const uint16_t*)biases, (uint16_t*)out, M, H, group_size, V, status);
  return launch_check("mtp_embed_affine4");
}

static int rope_run(const void* qkv, const int32_t* q_start, const int32_t* q_lens, void* q_out, void* k_cache,
                    void* v_cache, int B, int L, int Hq, int Hkv, int D, int cap, float rope_base, int32_t* status,
                    void* stream, int kv_blocked, const char* who) {
  if (!qkv || !q_start || !q_out || !k_cache || !v_cache || B < 1 || L < 1 || Hq < 1 || Hkv < 1 || D < 8 ||
      D % 8 || cap < 1 || !(rope_base > 1.f) || (kv_blocked && (cap % 32 || D != 128))) {
    set_error("%s: bad arguments", who);
    return MTP_ERR_ARG;
  }
  const int work = (Hq + Hkv) * (D / 2) + Hkv * D / 8;
  dim3 grid(cdiv(work, 256), B * L);
  hipLaunchKernelGGL(rope_qkv_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)qkv, q_start, q_lens,
                     (uint16_t*)q_out, (uint16_t*)k_cache, (uint16_t*)v_cache, B, L, Hq, Hkv, D, cap,
                     log2f(rope_base), status, kv_blocked);
  return launch_check(who);
}

MTP_API int mtp_rope_qkv_to_cache(const void* qkv, const int32_t* q_start, const int32_t* q_lens, void* q_out,
                                  void* k_cache, void* v_cache, int B, int L, int Hq, int Hkv, int D, int cap,
                                  float rope_base, int32_t* status, void* stream) {
  return rope_run(qkv, q_start, q_lens, q_out, k_cache, v_cache, B, L, Hq, Hkv, D, cap, rope_base, status, stream, 0,
                  "mtp_rope_qkv_to_cache");
}

MTP_API int mtp_rope_qkv_to_cache_vt(const void* qkv, const int32_t* q_start, const int32_t* q_lens, void* q_out,
                                     void* k_cache, void* v_cache, int B, int L, int Hq, int Hkv, int D, int cap,
                                     float rope_base, int32_t* status, void* stream) {
  return rope_run(qkv, q_start, q_lens, q_out, k_cache, v_cache, B, L, Hq, Hkv, D, cap, rope_base, status, stream, 1,
                  "mtp_rope_qkv_to_cache_vt");
}

MTP_API int mtp_rope_qkv_to_blocks(const void* qkv, int M, const int32_t* row_off, const int32_t* q_start,
                                   const int32_t* kv_off, void* q_out, void* k_blk, void* v_blk, int B, int Lmax,
                                   int Hq, int Hkv, int D, int cap, float rope_base, int32_t* status, void* stream) {
  const char* who = "mtp_rope_qkv_to_blocks";
  if (!qkv || !row_off || !q_start || !q_out || !k_blk || !v_blk || M < 1 || B < 1 || Lmax < 1 || Hq < 1 ||
      Hkv < 1 || D != 128 || !(rope_base > 1.f) || (!kv_off && (cap < 32 || cap % 32))) {
    set_error("%s: bad arguments (D = 128; cap a multiple of 32 without kv_off)", who);
    return MTP_ERR_ARG;
  }
  const int work = (Hq + Hkv) * (D / 2) + Hkv * D / 8;
  dim3 grid(cdiv(work, 256), M);
  hipLaunchKernelGGL(rope_qkv_blocks_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)qkv, row_off,
                     q_start, kv_off, (uint16_t*)q_out, (uint16_t*)k_blk, (uint16_t*)v_blk, B, Lmax, Hq, Hkv, D, cap,
                     log2f(rope_base), status);
  return launch_check(who);
}

MTP_API int mtp_rmsnorm(const void* x, const void* w, void* out, int M, int H, float eps, void* stream) {
  if (!x || !w || !out || M < 1 || H < 1 || (H % 8 == 0 && (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15))) {
    set_error("mtp_rmsnorm: bad arguments (rows of a multiple of 8 need 16-byte aligned x, w, out)");
    return MTP_ERR_ARG;
  }
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)x,
                     (const uint16_t*)w, (uint16_t*)out, H, eps);
  return launch_check("mtp_rmsnorm");
}
