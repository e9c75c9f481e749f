// Operand-major ragged GQA attention for the verify step: the split and
// merge bodies of the standalone kernels (attention.hip).
#pragma once

#include "common.hpp"

#include <stdlib.h>

// mtp_ragged_gqa_attn_blocks' argument block (the layout of include/mtplx_amd.h).
struct mtp_attn_blocks_args {
  const void* q;
  const void* k_blk;
  const void* v_blk;
  const int32_t* q_start;
  const int32_t* q_lens;
  const int32_t* row_off;
  const int32_t* kv_off;
  void* out;
  int B, Hq, Hkv, Lmax, D, cap, split_keys;
  float scale;
  long long total_cap;
  void* ws;
  size_t ws_bytes;
};

namespace mtp {

constexpr int kHD = 128;          // head dim
constexpr int kTileKeys = 32;
constexpr int kVtStride = 34;     // keys per LDS row (padded against bank conflicts)
constexpr float kNegBig = -1.0e30f;

struct AttnParams {
  const uint16_t* q;         // [B, Hq, L, D]
  const uint16_t* k;         // [B, Hkv, cap, D]
  const uint16_t* v;
  const int32_t* q_start;    // [B]
  const int32_t* q_lens;     // [B] or null (all L)
  uint16_t* out;             // [B, Hq, L, D]
  float* part_o;             // [B*Hkv*S][32][D]
  float* part_ml;            // [B*Hkv*S][32][2]
  int B, Hq, Hkv, L, cap, S, split_keys;
  int out_rows;              // 1: out is [B, L, Hq, D] (rows feed the o projection)
  float scale_log2;          // softmax scale * log2(e)
  // Ragged batches (the block-layout entry point): output row of request b's
  // query i is row_off[b] + i (null: b * L + i); request b's K/V blocks are
  // [kv_off[b], kv_off[b+1]), head h's nblk = (kv_off[b+1] - kv_off[b]) / Hkv
  // of them starting at kv_off[b] + h * nblk (null: a uniform capacity cap).
  const int32_t* row_off;
  const int32_t* kv_off;
  // Balanced work (attn_bal_body): per head (request-major), the first
  // partial slot and the number of slots; null for the per-unit layout.
  int32_t* bal_tab;
};

// Capacity (keys) of request b and the index of head h's first 32-key block.
__device__ __forceinline__ int req_cap(const AttnParams& p, int b) {
  return p.kv_off ? 32 * ((p.kv_off[b + 1] - p.kv_off[b]) / p.Hkv) : p.cap;
}
__device__ __forceinline__ size_t req_head_block(const AttnParams& p, int b, int h) {
  if (p.kv_off) {
    const int nb = (p.kv_off[b + 1] - p.kv_off[b]) / p.Hkv;
    return (size_t)p.kv_off[b] + (size_t)h * nb;
  }
  return ((size_t)b * p.Hkv + h) * (size_t)(p.cap >> 5);
}

__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  return (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
}

constexpr int kMaxSplits = 256;

// Operand-major KV blocks (the verify step's own cache, kblk_index /
// vblk_index in common.hpp): every K and V^T MFMA operand of a wave is one
// 1 KB contiguous load, and V needs no LDS transpose.
constexpr int kVtWaves = 4;   // waves per workgroup; each takes TPW 32-key tiles

// Unit = (request, kv head, 128*TPW-key split): four waves take 32*TPW keys
// each and merge in LDS (wave order), so the split partials are 4x fewer than
// with one wave per split.
//
// The body runs one unit with the workgroup's first kVtWaves waves; waves
// past those (a persistent kernel's larger workgroup) only meet its
// barriers. ``lds`` holds attn_vt_lds_bytes(). WT: device-coherent partial
// stores (read on another XCD later in the same kernel).
constexpr int kVtOS = kHD + 4;   // padded row: lanes of one store hit distinct banks
constexpr size_t attn_vt_lds_bytes() { return (size_t)kVtWaves * (32 * kVtOS + 64) * sizeof(float); }

template <int TPW, bool WT>
__device__ __forceinline__ void attn_vt_body(const AttnParams& p, const int unit, unsigned char* lds) {
  constexpr int kVtWaveKeys = TPW * kTileKeys;
  constexpr int kVtUnitKeys = kVtWaves * kVtWaveKeys;
  constexpr int kOS = kVtOS;
  float* s_o = reinterpret_cast<float*>(lds);   // [kVtWaves][32 * kOS]
  float* s_m = s_o + kVtWaves * 32 * kOS;       // [kVtWaves][32]
  float* s_l = s_m + kVtWaves * 32;             // [kVtWaves][32]
  const int tid = threadIdx.x;
  const bool act = tid < kVtWaves * 64;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31;
  const int h2 = lane >> 5;
  const int s = unit % p.S;
  const int bh = unit / p.S;
  const int h = bh % p.Hkv;
  const int b = bh / p.Hkv;
  const int rep = p.Hq / p.Hkv;
  const int qs = p.q_start[b];
  const int L = p.q_lens ? p.q_lens[b] : p.L;
  int kv_end = qs + L;
  if (kv_end > p.cap) kv_end = p.cap;
  const int k0u = s * kVtUnitKeys;
  float* po = p.part_o + (size_t)unit * 32 * kHD;
  float* pml = p.part_ml + (size_t)unit * 64;
  if (k0u >= kv_end) {
    if (tid < 32) {
      st_f32<WT>(pml + 2 * tid, kNegBig);
      st_f32<WT>(pml + 2 * tid + 1, 0.f);
    }
    return;   // uniform over the workgroup
  }
  const int k0 = k0u + wave * kVtWaveKeys;
  const int k1 = (k0 + kVtWaveKeys < kv_end) ? k0 + kVtWaveKeys : kv_end;

  const int qcol = c32;
  const int qr = qcol / p.L;
  const int qi = qcol - qr * p.L;
  const bool qvalid = (qr < rep) && (qi < L);
  const int qbound = qs + qi;
  f32x16 o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = f32x16{};
  float m_run = kNegBig;
  float l_run = 0.f;
  if (act) {
    bf16x8 qop[8];
    {
      const uint16_t* qrow = p.q + ((((size_t)b * p.Hq + h * rep + (qvalid ? qr : 0)) * p.L + (qvalid ? qi : 0)) * kHD);
  #pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint4 raw = qvalid ? *reinterpret_cast<const uint4*>(qrow + 64 * h2 + 8 * i) : make_uint4(0, 0, 0, 0);
        qop[i] = __builtin_bit_cast(bf16x8, raw);
      }
    }
    const uint16_t* kbase = p.k + ((size_t)b * p.Hkv + h) * (size_t)p.cap * kHD;
    const uint16_t* vbase = p.v + ((size_t)b * p.Hkv + h) * (size_t)p.cap * kHD;

    // All tiles of this wave are loaded before any compute (one round trip).
    uint4 kr[TPW][8], vr[TPW][8];
  #pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      const int kt = k0 + tt * kTileKeys;
      const bool kin = kt + c32 < k1;
      const size_t blk = (size_t)((kt < k1 ? kt : k0) >> 5) * 4096 + (size_t)lane * 8;
  #pragma unroll
      for (int i = 0; i < 8; ++i)
        kr[tt][i] = kin ? ld_stream(kbase + blk + i * 512) : make_uint4(0, 0, 0, 0);
  #pragma unroll
      for (int t = 0; t < 4; ++t)
  #pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          vr[tt][2 * t + jj] = ld_stream(vbase + blk + (t * 2 + jj) * 512);
    }
  #pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
      const int kt = k0 + tt * kTileKeys;
      if (kt >= k1) break;   // wave-uniform
      f32x16 st = {};
  #pragma unroll
      for (int i = 0; i < 8; ++i)
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kr[tt][i]), qop[i], st, 0, 0, 0);
      float sv[16];
      float tmax = kNegBig;
  #pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kk = kt + 8 * (r >> 2) + 4 * h2 + (r & 3);
        const bool ok = qvalid && kk < k1 && kk <= qbound;
        sv[r] = ok ? st[r] * p.scale_log2 : -INFINITY;
        tmax = fmaxf(tmax, sv[r]);
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float m_new = fmaxf(m_run, tmax);
      const float corr = exp2f(m_run - m_new);
      m_run = m_new;
      float psum = 0.f;
  #pragma unroll
      for (int r = 0; r < 16; ++r) {
        sv[r] = exp2f(sv[r] - m_new);
        psum += sv[r];
      }
      l_run = l_run * corr + psum;
  #pragma unroll
      for (int t = 0; t < 4; ++t)
  #pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= corr;
      if (kt + kTileKeys > k1) {   // keys past the end: zero V so stale cache bits cannot leak in
  #pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const int kbase_e = kt + 16 * jj + 4 * h2;   // slot e<4: kbase_e+e, e>=4: kbase_e+8+e-4
          uint32_t msk[4];
  #pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int e0 = 2 * w, e1 = 2 * w + 1;
            const int key0 = kbase_e + (e0 < 4 ? e0 : 8 + e0 - 4);
            const int key1 = kbase_e + (e1 < 4 ? e1 : 8 + e1 - 4);
            msk[w] = (key0 < k1 ? 0x0000ffffu : 0u) | (key1 < k1 ? 0xffff0000u : 0u);
          }
  #pragma unroll
          for (int t = 0; t < 4; ++t) {
            uint4& c = vr[tt][2 * t + jj];
            c.x &= msk[0];
            c.y &= msk[1];
            c.z &= msk[2];
            c.w &= msk[3];
          }
        }
      }
      bf16x8 pop[2];
  #pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        uint32_t pk[4];
  #pragma unroll
        for (int t = 0; t < 4; ++t) pk[t] = f2bf2(sv[8 * jj + 2 * t], sv[8 * jj + 2 * t + 1]);
        pop[jj] = __builtin_bit_cast(bf16x8, pk);
      }
  #pragma unroll
      for (int t = 0; t < 4; ++t)
  #pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vr[tt][2 * t + jj]), pop[jj],
                                                          o[t], 0, 0, 0);
    }
  }

  // Merge the four waves in LDS, wave order (deterministic).
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (act && h2 == 0) {
    s_m[wave * 32 + c32] = m_run;
    s_l[wave * 32 + c32] = l_tot;
  }
  __syncthreads();
  if (act) {
    float mq = s_m[c32];
#pragma unroll
    for (int w = 1; w < kVtWaves; ++w) mq = fmaxf(mq, s_m[w * 32 + c32]);
    const float sc = exp2f(m_run - mq);
    float* so_w = s_o + wave * 32 * kOS;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)   // registers 4j..4j+3 are 4 consecutive d
        *reinterpret_cast<float4*>(&so_w[qcol * kOS + 32 * t + 8 * j + 4 * h2]) =
            make_float4(o[t][4 * j] * sc, o[t][4 * j + 1] * sc, o[t][4 * j + 2] * sc, o[t][4 * j + 3] * sc);
  }
  __syncthreads();
  if (!act) return;
  // Only the live query columns (rep * L of the 32): the merge reads no others.
  const int live = rep * p.L;
  for (int idx = 4 * tid; idx < live * kHD; idx += 4 * kVtWaves * 64) {
    const int so = (idx / kHD) * kOS + (idx % kHD);
    float4 v = *reinterpret_cast<const float4*>(&s_o[so]);
#pragma unroll
    for (int w = 1; w < kVtWaves; ++w) {
      const float4 a = *reinterpret_cast<const float4*>(&s_o[w * 32 * kOS + so]);
      v.x += a.x;
      v.y += a.y;
      v.z += a.z;
      v.w += a.w;
    }
    if constexpr (WT) {
      st_f32<WT>(po + idx, v.x);
      st_f32<WT>(po + idx + 1, v.y);
      st_f32<WT>(po + idx + 2, v.z);
      st_f32<WT>(po + idx + 3, v.w);
    } else {
      *reinterpret_cast<float4*>(po + idx) = v;
    }
  }
  if (tid < 32) {
    float M = s_m[tid];
#pragma unroll
    for (int w = 1; w < kVtWaves; ++w) M = fmaxf(M, s_m[w * 32 + tid]);
    float lsum = 0.f;
#pragma unroll
    for (int w = 0; w < kVtWaves; ++w) lsum += s_l[w * 32 + tid] * exp2f(s_m[w * 32 + tid] - M);
    st_f32<WT>(pml + 2 * tid, M);
    st_f32<WT>(pml + 2 * tid + 1, lsum);
  }
}



// One (request b, kv head h) piece over per-request capacities: wave w of the
// four attends keys [k0, k1) of its own (the caller's split of the piece),
// one 32-key tile at a time through an NRG-deep register ring (the next
// tiles' K and V^T operands in flight while this one is computed); the waves
// then merge in LDS in wave order as attn_vt_body does and the workgroup
// writes the piece's partial (o rows to po, (max, l) pairs to pml). qs, L:
// the request's first query position and query count; hblk: the first
// 32-key block of head (b, h) (req_head_block). A wave with k0 >= k1
// contributes nothing. Every thread of the four waves must call it.
template <bool WT, int NRG>
__device__ __forceinline__ void attn_vl_piece(const AttnParams& p, const int b, const int h, const int qs,
                                              const int L, const int k0, const int k1, const size_t hblk,
                                              float* po, float* pml, unsigned char* lds) {
  constexpr int kOS = kVtOS;
  float* s_o = reinterpret_cast<float*>(lds);   // [kVtWaves][32 * kOS]
  float* s_m = s_o + kVtWaves * 32 * kOS;       // [kVtWaves][32]
  float* s_l = s_m + kVtWaves * 32;             // [kVtWaves][32]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c32 = lane & 31;
  const int h2 = lane >> 5;
  const int rep = p.Hq / p.Hkv;
  const int qcol = c32;
  const int qr = qcol / p.L;
  const int qi = qcol - qr * p.L;
  const bool qvalid = (qr < rep) && (qi < L);
  const int qbound = qs + qi;
  f32x16 o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = f32x16{};
  float m_run = kNegBig;
  float l_run = 0.f;
  bf16x8 qop[8];
  {
    const uint16_t* qrow = p.q + ((((size_t)b * p.Hq + h * rep + (qvalid ? qr : 0)) * p.L + (qvalid ? qi : 0)) * kHD);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint4 raw = qvalid ? *reinterpret_cast<const uint4*>(qrow + 64 * h2 + 8 * i) : make_uint4(0, 0, 0, 0);
      qop[i] = __builtin_bit_cast(bf16x8, raw);
    }
  }
  const size_t hb = hblk * 4096;
  const uint16_t* kbase = p.k + hb;
  const uint16_t* vbase = p.v + hb;
  // Tiles at or past k1 reload this wave's last block (valid memory, still in
  // L2 from the wave's own load of it; never used).
  auto load_tile = [&](uint4 (&kr)[8], uint4 (&vr)[8], int kt) {
    const size_t blk = (size_t)((kt < k1 ? kt : k1 - 1) >> 5) * 4096 + (size_t)lane * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) kr[i] = ld_stream(kbase + blk + i * 512);
#pragma unroll
    for (int i = 0; i < 8; ++i) vr[i] = ld_stream(vbase + blk + i * 512);
  };
  auto tile = [&](const uint4 (&kr)[8], uint4 (&vr)[8], int kt) {
    f32x16 st = {};
#pragma unroll
    for (int i = 0; i < 8; ++i)
      st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kr[i]), qop[i], st, 0, 0, 0);
    float sv[16];
    float tmax = kNegBig;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kk = kt + 8 * (r >> 2) + 4 * h2 + (r & 3);
      const bool ok = qvalid && kk < k1 && kk <= qbound;
      sv[r] = ok ? st[r] * p.scale_log2 : -INFINITY;
      tmax = fmaxf(tmax, sv[r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float corr = exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sv[r] = exp2f(sv[r] - m_new);
      psum += sv[r];
    }
    l_run = l_run * corr + psum;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] *= corr;
    if (kt + kTileKeys > k1) {   // keys past the end: zero V so stale cache bits cannot leak in
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int kbase_e = kt + 16 * jj + 4 * h2;   // slot e<4: kbase_e+e, e>=4: kbase_e+8+e-4
        uint32_t msk[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int e0 = 2 * w, e1 = 2 * w + 1;
          const int key0 = kbase_e + (e0 < 4 ? e0 : 8 + e0 - 4);
          const int key1 = kbase_e + (e1 < 4 ? e1 : 8 + e1 - 4);
          msk[w] = (key0 < k1 ? 0x0000ffffu : 0u) | (key1 < k1 ? 0xffff0000u : 0u);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          uint4& c = vr[2 * t + jj];
          c.x &= msk[0];
          c.y &= msk[1];
          c.z &= msk[2];
          c.w &= msk[3];
        }
      }
    }
    bf16x8 pop[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      uint32_t pk[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) pk[t] = f2bf2(sv[8 * jj + 2 * t], sv[8 * jj + 2 * t + 1]);
      pop[jj] = __builtin_bit_cast(bf16x8, pk);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, vr[2 * t + jj]), pop[jj], o[t], 0,
                                                        0, 0);
  };
  if (k0 < k1) {
    // NRG-deep register ring of K and V^T tiles (slot i holds tile kt + 32 i).
    uint4 kr[NRG][8], vr[NRG][8];
#pragma unroll
    for (int i = 0; i < NRG; ++i) load_tile(kr[i], vr[i], k0 + i * kTileKeys);
    int kt = k0;
    do {   // one exit, at the bottom; steps past the end are skipped by uniform branches
#pragma unroll
      for (int i = 0; i < NRG; ++i) {
        if (i == 0 || kt + i * kTileKeys < k1) {
          tile(kr[i], vr[i], kt + i * kTileKeys);
          load_tile(kr[i], vr[i], kt + (i + NRG) * kTileKeys);
        }
      }
      kt += NRG * kTileKeys;
    } while (kt < k1);
  }

  // Merge the four waves in LDS, wave order (deterministic), as attn_vt_body.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (h2 == 0) {
    s_m[wave * 32 + c32] = m_run;
    s_l[wave * 32 + c32] = l_tot;
  }
  __syncthreads();
  {
    float mq = s_m[c32];
#pragma unroll
    for (int w = 1; w < kVtWaves; ++w) mq = fmaxf(mq, s_m[w * 32 + c32]);
    const float sc = exp2f(m_run - mq);
    float* so_w = s_o + wave * 32 * kOS;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<float4*>(&so_w[qcol * kOS + 32 * t + 8 * j + 4 * h2]) =
            make_float4(o[t][4 * j] * sc, o[t][4 * j + 1] * sc, o[t][4 * j + 2] * sc, o[t][4 * j + 3] * sc);
  }
  __syncthreads();
  // Only the live query columns (rep * L of the 32): the merge reads no others.
  const int live = (p.Hq / p.Hkv) * p.L;
  for (int idx = 4 * tid; idx < live * kHD; idx += 4 * kVtWaves * 64) {
    const int so = (idx / kHD) * kOS + (idx % kHD);
    float4 v = *reinterpret_cast<const float4*>(&s_o[so]);
#pragma unroll
    for (int w = 1; w < kVtWaves; ++w) {
      const float4 a = *reinterpret_cast<const float4*>(&s_o[w * 32 * kOS + so]);
      v.x += a.x;
      v.y += a.y;
      v.z += a.z;
      v.w += a.w;
    }
    *reinterpret_cast<float4*>(po + idx) = v;
  }
  if (tid < 32) {
    float M = s_m[tid];
#pragma unroll
    for (int w = 1; w < kVtWaves; ++w) M = fmaxf(M, s_m[w * 32 + tid]);
    float lsum = 0.f;
#pragma unroll
    for (int w = 0; w < kVtWaves; ++w) lsum += s_l[w * 32 + tid] * exp2f(s_m[w * 32 + tid] - M);
    pml[2 * tid] = M;
    pml[2 * tid + 1] = lsum;
  }
}

// Unit = (request, kv head, split of split_keys keys) over per-request
// capacities: the four waves take split_keys / 4 consecutive keys each.
// split_keys is a multiple of 128, so long contexts need few splits and few
// partials.
template <bool WT, int NRG = 2>
__device__ __forceinline__ void attn_vl_body(const AttnParams& p, const int unit, unsigned char* lds) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int s = unit % p.S;
  const int bh = unit / p.S;
  const int h = bh % p.Hkv;
  const int b = bh / p.Hkv;
  const int qs = p.q_start[b];
  const int L = p.q_lens ? p.q_lens[b] : p.L;
  const int capb = req_cap(p, b);
  const int kv_end = (qs + L < capb) ? qs + L : capb;
  const int k0u = s * p.split_keys;
  float* po = p.part_o + (size_t)unit * 32 * kHD;
  float* pml = p.part_ml + (size_t)unit * 64;
  if (k0u >= kv_end) {
    if (tid < 32) {
      st_f32<WT>(pml + 2 * tid, kNegBig);
      st_f32<WT>(pml + 2 * tid + 1, 0.f);
    }
    return;   // uniform over the workgroup
  }
  const int wk = p.split_keys / kVtWaves;
  const int k0 = k0u + wave * wk;
  const int k1 = (k0 + wk < kv_end) ? k0 + wk : kv_end;
  attn_vl_piece<WT, NRG>(p, b, h, qs, L, k0, k1, req_head_block(p, b, h), po, pml, lds);
}

// Balanced work for the per-request-capacity layout. The batch's 32-key
// tiles are numbered request-major, then head, then position (each head of
// request b has nt_b = ceil(kv_end_b / 32) tiles); workgroup w of G takes the
// tiles [w T / G, (w+1) T / G) of the T in all, so every workgroup streams
// the same share of K and V whatever the lengths. Its range falls into
// pieces, one per head it touches; each piece is split over the four waves
// by tiles and leaves one partial. Head bh's partials are the consecutive
// slots from bal_base(bh), one per workgroup that touches it, in workgroup
// order; the merge reads the (base, count) table that workgroup 0 writes.
constexpr int kBalMaxReq = 256;   // requests the per-workgroup prefix table holds
constexpr int kBalReqArrays = 8;   // per-request values the prologue keeps in LDS (ints)
constexpr size_t attn_bal_lds_bytes() {
  return attn_vt_lds_bytes() + (size_t)kBalReqArrays * kBalMaxReq * sizeof(int);
}

// The balanced split of T tiles over the first G workgroups of the grid,
// G = min(grid, T): workgroup w takes tiles [lo(w), lo(w + 1)),
// lo(w) = floor(w T / G). With G <= T every one of them gets a tile, so no
// workgroup inside a head's range of slots is empty and the merge reads only
// written partials (with more workgroups than tiles, empty ones in the middle
// of a head's range would leave slots holding stale partials).
struct BalSplit {
  long long T;
  int G;
  __device__ BalSplit(long long T_, int grid) : T(T_), G((long long)grid < T_ ? grid : (int)T_) {}
  __device__ long long lo(int w) const { return (long long)w * T / G; }
  // Workgroup owning tile x: the largest w with lo(w) <= x.
  __device__ int owner(long long x) const { return (int)(((x + 1) * G - 1) / T); }
};

// Slots (partials) of head (b, h) whose first global tile is P, nt tiles.
__device__ __forceinline__ int bal_nparts(long long P, int nt, const BalSplit& bs) {
  return nt > 0 ? bs.owner(P + nt - 1) - bs.owner(P) + 1 : 0;
}

template <bool WT, int NRG = 2>
__device__ __forceinline__ void attn_bal_body(const AttnParams& p, unsigned char* lds) {
  int* s_nt = reinterpret_cast<int*>(lds + attn_vt_lds_bytes());   // [B] tiles per head of each request
  int* s_pt = s_nt + kBalMaxReq;                                    // [B] first global tile of each request
  int* s_ps = s_pt + kBalMaxReq;                                    // [B] first slot of each request
  int* s_qs = s_ps + kBalMaxReq;                                    // [B] first query position
  int* s_ql = s_qs + kBalMaxReq;                                    // [B] query rows
  int* s_ke = s_ql + kBalMaxReq;                                    // [B] keys [0, kv_end) attended
  int* s_hb = s_ke + kBalMaxReq;                                    // [2B] head 0's first block, blocks per head
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = (int)gridDim.x, w = (int)blockIdx.x;
  const int B = p.B, Hkv = p.Hkv;
  // Each request's values, read from memory once (every load of a thread
  // issued together) and kept in LDS for the pieces below; then the tiles
  // per request and the request-major prefix sums (wave 0, 64 requests at a
  // time with a running carry).
  for (int b = tid; b < B; b += kVtWaves * 64) {
    const int qs = p.q_start[b];
    const int L = p.q_lens ? p.q_lens[b] : p.L;
    int blk0, nbh;   // req_head_block(p, b, 0) and the blocks per head (req_cap / 32)
    if (p.kv_off) {
      blk0 = p.kv_off[b];
      nbh = (p.kv_off[b + 1] - blk0) / Hkv;
    } else {
      nbh = p.cap >> 5;
      blk0 = b * Hkv * nbh;
    }
    int kv_end = (qs + L < 32 * nbh) ? qs + L : 32 * nbh;
    if (kv_end < 0) kv_end = 0;
    s_nt[b] = (kv_end + kTileKeys - 1) / kTileKeys;
    s_qs[b] = qs;
    s_ql[b] = L;
    s_ke[b] = kv_end;
    s_hb[2 * b] = blk0;
    s_hb[2 * b + 1] = nbh;
  }
  __syncthreads();
  if (wave == 0) {
    int carry = 0;
    for (int b0 = 0; b0 < B; b0 += 64) {
      const int b = b0 + lane;
      const int v = b < B ? Hkv * s_nt[b] : 0;
      int incl = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
      }
      if (b < B) s_pt[b] = carry + incl - v;
      carry += __shfl(incl, 63, 64);
    }
  }
  __syncthreads();
  // Values read back from LDS are the same in every lane: readfirstlane
  // keeps them (and the loop below) in scalar registers.
  auto lds_int = [&](const int* a, int i) { return __builtin_amdgcn_readfirstlane(a[i]); };
  const long long T = (long long)lds_int(s_pt, B - 1) + (long long)Hkv * lds_int(s_nt, B - 1);
  const BalSplit bs(T, G);
  if (T == 0) {   // no keys at all: every head has no partial
    if (w == 0 && p.bal_tab)
      for (int i = tid; i < 2 * B * Hkv; i += kVtWaves * 64) p.bal_tab[i] = 0;
    return;
  }
  // Slot prefix: request b's heads take sum_h bal_nparts slots.
  if (wave == 0) {
    int carry = 0;
    for (int b0 = 0; b0 < B; b0 += 64) {
      const int b = b0 + lane;
      int v = 0;
      if (b < B)
        for (int h = 0; h < Hkv; ++h) v += bal_nparts((long long)s_pt[b] + (long long)h * s_nt[b], s_nt[b], bs);
      int incl = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
      }
      if (b < B) s_ps[b] = carry + incl - v;
      carry += __shfl(incl, 63, 64);
    }
  }
  __syncthreads();
  // Workgroup 0 publishes each head's (first slot, slot count) for the merge.
  if (w == 0 && p.bal_tab) {
    for (int bh = tid; bh < B * Hkv; bh += kVtWaves * 64) {
      const int b = bh / Hkv, h = bh - (bh / Hkv) * Hkv;
      int base = s_ps[b];
      for (int hh = 0; hh < h; ++hh) base += bal_nparts((long long)s_pt[b] + (long long)hh * s_nt[b], s_nt[b], bs);
      p.bal_tab[2 * bh] = base;
      p.bal_tab[2 * bh + 1] = bal_nparts((long long)s_pt[b] + (long long)h * s_nt[b], s_nt[b], bs);
    }
  }
  if (w >= bs.G) return;   // past the split's workgroups (fewer tiles than the grid)
  const long long lo = bs.lo(w), hi = bs.lo(w + 1);
  if (lo >= hi) return;     // (not reached: each of the split's workgroups has a tile)
  // Request holding tile lo: the last b with s_pt[b] <= lo (binary search).
  int b = 0;
  {
    int a = 0, z = B - 1;
    while (a < z) {
      const int m = (a + z + 1) >> 1;
      if (lds_int(s_pt, m) <= lo) a = m; else z = m - 1;
    }
    b = a;
  }
  long long x = lo;
  bool first = true;
  while (x < hi) {
    const int nt = lds_int(s_nt, b);
    const long long pb = lds_int(s_pt, b);
    if (nt == 0 || x >= pb + (long long)Hkv * nt) {   // past this request
      ++b;
      continue;
    }
    const int h = (int)(x - pb) / nt;   // x - pb < Hkv * nt
    const long long P = pb + (long long)h * nt;   // head's first global tile
    const int ta = (int)(x - P);
    const int tb = (int)((hi < P + nt ? hi : P + nt) - P);
    int slot = lds_int(s_ps, b);
    for (int hh = 0; hh < h; ++hh) slot += bal_nparts(pb + (long long)hh * nt, nt, bs);
    slot += w - bs.owner(P);
    const int qs = lds_int(s_qs, b);
    const int L = lds_int(s_ql, b);
    const int kv_end = lds_int(s_ke, b);
    const size_t hblk = (size_t)lds_int(s_hb, 2 * b) + (size_t)h * lds_int(s_hb, 2 * b + 1);
    // The four waves take consecutive shares of the piece's tiles.
    const int n = tb - ta;
    const int t0 = ta + (n * wave) / kVtWaves, t1 = ta + (n * (wave + 1)) / kVtWaves;
    const int k0 = t0 * kTileKeys;
    const int k1 = (t1 * kTileKeys < kv_end) ? t1 * kTileKeys : kv_end;
    if (!first) __syncthreads();   // the previous piece's LDS reads are done
    first = false;
    attn_vl_piece<WT, NRG>(p, b, h, qs, L, k0, k1, hblk, p.part_o + (size_t)slot * 32 * kHD,
                           p.part_ml + (size_t)slot * 64, lds);
    x = P + tb;
  }
}

// Merge item = (request, kv head, query column), one per workgroup of
// kMergeGroups x 128 threads: thread (g, d) sums column d over group g's
// contiguous share of the splits, issuing all of its loads together (one
// round trip instead of one per four splits); the groups then add in group
// order, so the result is deterministic. ``lds`` holds attn_merge_lds_bytes().
// Wave 0 writes the weights and the l sum before the body's first barrier:
// a caller that runs several items in one workgroup puts a barrier between
// them.
constexpr int kMergeGroups = 4;
constexpr int kMergeThreads = kMergeGroups * 128;
constexpr size_t attn_merge_lds_bytes() { return (size_t)(kMaxSplits + 2 + kMergeGroups * 128) * sizeof(float); }
static_assert(kMaxSplits % 64 == 0, "wave 0 holds kMaxSplits / 64 splits per lane");

template <bool WT>
__device__ __forceinline__ void attn_merge_body(const AttnParams& p, const int item, unsigned char* lds) {
  float* s_w = reinterpret_cast<float*>(lds);   // [kMaxSplits] split weights
  float* s_red = s_w + kMaxSplits;              // [1]: the l sum
  float* s_acc = s_red + 2;                     // [kMergeGroups][128]
  const int tid = threadIdx.x;
  const int g = tid >> 7, d = tid & 127;
  const int rep = p.Hq / p.Hkv;
  const int rows = rep * p.L;
  const int q = item % rows;
  const int bh = item / rows;
  const int h = bh % p.Hkv;
  const int b = bh / p.Hkv;
  const int L = p.q_lens ? p.q_lens[b] : p.L;
  const int qr = q / p.L, qi = q - (q / p.L) * p.L;
  const int kv_end = p.q_start[b] + L;
  const int capb = req_cap(p, b);
  // The head's partials: splits bh * S .. of the per-unit layout, or the
  // balanced layout's slots from its table.
  int ns, base;
  if (p.bal_tab) {
    base = p.bal_tab[2 * bh];
    ns = p.bal_tab[2 * bh + 1];
  } else {
    base = bh * p.S;
    ns = cdiv(kv_end < capb ? kv_end : capb, p.split_keys);
    if (ns > p.S) ns = p.S;
  }
  const float* ml = p.part_ml + (size_t)base * 64 + 2 * q;
  // This thread's partial-O loads go out first: they do not depend on the
  // split weights, so the max / weight pass below overlaps their round trip.
  const int s0 = (g * ns) / kMergeGroups, s1 = ((g + 1) * ns) / kMergeGroups;
  const float* po = p.part_o + ((size_t)base * 32 + q) * kHD + d;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = (s0 + i < s1) ? po[(size_t)(s0 + i) * 32 * kHD] : 0.f;
  // Wave 0: each split's (max, l) loaded once into registers (lane s % 64),
  // the max as a fixed tree over lanes, the split weights to LDS, and the
  // l sum as a lane-strided fixed tree (deterministic).
  if (tid < 64) {
    constexpr int kPerLane = kMaxSplits / 64;
    float2 mlv[kPerLane];
    float m = kNegBig;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int s = tid + 64 * j;
      mlv[j] = s < ns ? *reinterpret_cast<const float2*>(ml + (size_t)s * 64) : make_float2(kNegBig, 0.f);
      m = fmaxf(m, mlv[j].x);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float l = 0.f;
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) {
      const int s = tid + 64 * j;
      if (s < ns) {
        const float w = exp2f(mlv[j].x - m);
        s_w[s] = w;
        l += __fmul_rn(mlv[j].y, w);   // the weighted l rounded before the sum
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off, 64);
    if (tid == 0) s_red[1] = l;
  }
  __syncthreads();
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (s0 + i < s1) acc += v[i] * s_w[s0 + i];
  for (int c = s0 + 16; c < s1; c += 16) {   // more than 64 splits
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = (c + i < s1) ? po[(size_t)(c + i) * 32 * kHD] : 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (c + i < s1) acc += v[i] * s_w[c + i];
  }
  s_acc[g * 128 + d] = acc;
  __syncthreads();
  if (g != 0) return;
  float tot = s_acc[d];
#pragma unroll
  for (int k = 1; k < kMergeGroups; ++k) tot += s_acc[k * 128 + d];
  const float lsum = s_red[1];
  const float val = (qi < L && lsum > 0.f) ? tot / lsum : 0.f;
  const size_t orow = p.row_off ? (size_t)p.row_off[b] + qi : (size_t)b * p.L + qi;
  const size_t oi = p.out_rows ? ((orow * p.Hq + h * rep + qr) * kHD + d)
                               : ((((size_t)b * p.Hq + h * rep + qr) * p.L + qi) * kHD + d);
  if (p.row_off && qi >= L) return;   // packed rows: request b has only L of them
  st_u16<WT>(p.out + oi, f2bf(val));
}

// Merge item = one (request, kv head) with all its query columns, for
// batches with many heads and few partials each (ragged batches): thread t of
// kMergeHeadThreads takes column t / 8 and 16 consecutive d, and walks the
// head's partials kMergeHeadBatch at a time with every load of a batch in
// flight together (index clamped into the head's slots, so they issue back
// to back), the running max rescaled between batches; fixed order, so the
// result is deterministic.
constexpr int kMergeHeadThreads = 256;
constexpr int kMergeHeadBatch = 8;

template <bool WT>
__device__ __forceinline__ void attn_merge_head_body(const AttnParams& p, const int bh) {
  const int tid = threadIdx.x;
  const int rep = p.Hq / p.Hkv;
  const int rows = rep * p.L;
  const int q = tid >> 3;
  const int d0 = (tid & 7) * 16;
  if (q >= rows) return;
  const int h = bh % p.Hkv;
  const int b = bh / p.Hkv;
  const int L = p.q_lens ? p.q_lens[b] : p.L;
  const int qr = q / p.L, qi = q - (q / p.L) * p.L;
  if (p.row_off && qi >= L) return;   // packed rows: request b has only L of them
  int ns, base;
  if (p.bal_tab) {
    base = p.bal_tab[2 * bh];
    ns = p.bal_tab[2 * bh + 1];
  } else {
    const int kv_end = p.q_start[b] + L;
    const int capb = req_cap(p, b);
    base = bh * p.S;
    ns = cdiv(kv_end < capb ? kv_end : capb, p.split_keys);
    if (ns > p.S) ns = p.S;
  }
  float M = kNegBig, lsum = 0.f;
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  for (int s0 = 0; s0 < ns; s0 += kMergeHeadBatch) {   // ns == 0 (no keys): zeros out
    float4 v[kMergeHeadBatch][4];
    float2 ml[kMergeHeadBatch];
#pragma unroll
    for (int j = 0; j < kMergeHeadBatch; ++j) {
      const int sj = base + (s0 + j < ns ? s0 + j : ns - 1);
      const float* src = p.part_o + ((size_t)sj * 32 + q) * kHD + d0;
#pragma unroll
      for (int c = 0; c < 4; ++c) v[j][c] = *reinterpret_cast<const float4*>(src + 4 * c);
      ml[j] = *reinterpret_cast<const float2*>(p.part_ml + (size_t)sj * 64 + 2 * q);
    }
#pragma unroll
    for (int j = 0; j < kMergeHeadBatch; ++j)
      if (s0 + j >= ns) ml[j] = make_float2(kNegBig, 0.f);   // past the head's slots (uniform)
    float mb = M;
#pragma unroll
    for (int j = 0; j < kMergeHeadBatch; ++j) mb = fmaxf(mb, ml[j].x);
    const float cr = exp2f(M - mb);
    M = mb;
    lsum *= cr;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] *= cr;
#pragma unroll
    for (int j = 0; j < kMergeHeadBatch; ++j) {
      if (s0 + j >= ns) continue;   // uniform: its values are another slot's
      const float w = exp2f(ml[j].x - M);
      lsum += __fmul_rn(ml[j].y, w);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[4 * c] += v[j][c].x * w;
        acc[4 * c + 1] += v[j][c].y * w;
        acc[4 * c + 2] += v[j][c].z * w;
        acc[4 * c + 3] += v[j][c].w * w;
      }
    }
  }
  const bool live = qi < L && lsum > 0.f;
  uint32_t pk[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) pk[i] = pack_bf2(live ? acc[2 * i] / lsum : 0.f, live ? acc[2 * i + 1] / lsum : 0.f);
  const size_t orow = p.row_off ? (size_t)p.row_off[b] + qi : (size_t)b * p.L + qi;
  const size_t oi = p.out_rows ? ((orow * p.Hq + h * rep + qr) * kHD + d0)
                               : ((((size_t)b * p.Hq + h * rep + qr) * p.L + qi) * kHD + d0);
  uint4* dst = reinterpret_cast<uint4*>(p.out + oi);
  dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
}

// Tiles per wave: one (more workgroups, shorter chains) while that keeps the
// partials to merge within kMaxSplits per (request, kv head), else two.
inline int attn_vt_plan(int cap, int* S, int* tpw) {
  const char* env = getenv("MTPLX_AMD_ATTN_TPW");
  *tpw = (env && atoi(env) == 2) || cdiv(cap, kVtWaves * kTileKeys) > kMaxSplits ? 2 : 1;
  *S = cdiv(cap, kVtWaves * kTileKeys * *tpw);
  return (*S <= kMaxSplits) ? MTP_OK : MTP_ERR_UNSUPPORTED;
}

}  // namespace mtp
