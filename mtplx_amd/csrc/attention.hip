// Ragged-batch GQA verify attention over a padded ragged KV cache, gfx950.
//
// Semantics (mtplx/ragged_attention.py:42-85 + MLX SDPA as called from
// mtplx/attention_split.py:347): query row i of request b sits at absolute
// position q_start[b] + i and attends keys j <= q_start[b] + i; GQA maps query
// head hq to kv head hq / (Hq/Hkv); softmax in fp32; bf16 in/out.
//
// Design: a work unit is (request b, kv head h, key split s). The rep*L query
// rows that share kv head h (e.g. 5 heads x 4 verify rows = 20) form the
// 32-row side of v_mfma_f32_32x32x16_bf16, so one wave streams each K/V row of
// the split exactly once:
//   S^T = K Q^T        A = K rows (lane = key, 128 B contiguous per lane)
//   O^T += V^T P^T     B = P^T straight from the S^T accumulators (no shuffle),
//                      A = V^T read from a transposed LDS tile
// Online softmax per query column; each column's 32 keys live in two lanes
// (l, l^32), so the tile max is one shuffle. Splits write (m, l, O) partials
// and a second kernel merges them in split order (deterministic). Offsets are
// read on the GPU; units past a request's length exit at once.
#include "attn_vt.hpp"

#include <stdlib.h>

namespace mtp {


// The V tile sits in LDS in its natural layout (key-major, rows padded to
// kVrowStride elements = 288 B, so the four rows one transposing read spans
// fall in distinct banks). ds_read_b64_tr_b16 returns, to lane i of each
// 16-lane group, element i % 4 of the 4 consecutive bf16 loaded by lane
// 4 e + i / 4, as its slot e (e = 0..3). Lane j of the group therefore
// addresses row key0 + j / 4, columns d0 + 4 (j % 4): lane i receives
// V[key0 + e][d0 + i] in slot e, a V^T MFMA operand's four keys.
constexpr int kVrowStride = kHD + 16;
typedef short v4i16_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v4i16_t lds_read_tr16(const uint16_t* a) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t*)(a));
}

__global__ __launch_bounds__(64) void attn_split_kernel(AttnParams p) {
  __shared__ __align__(16) uint16_t ktile[kTileKeys * kVrowStride];
  __shared__ __align__(16) uint16_t vtile[kTileKeys * kVrowStride];
  const int lane = threadIdx.x;
  const int c32 = lane & 31;
  const int h2 = lane >> 5;
  const int unit = blockIdx.x;
  const int s = unit % p.S;
  const int bh = unit / p.S;
  const int h = bh % p.Hkv;
  const int b = bh / p.Hkv;
  const int rep = p.Hq / p.Hkv;
  const int qs = p.q_start[b];
  const int L = p.q_lens ? p.q_lens[b] : p.L;
  const int kv_end = qs + L;  // keys [0, kv_end) are visible to some row
  const int k0 = s * p.split_keys;
  int k1 = k0 + p.split_keys;
  if (k1 > kv_end) k1 = kv_end;
  if (k1 > p.cap) k1 = p.cap;

  float* po = p.part_o + (size_t)unit * 32 * kHD;
  float* pml = p.part_ml + (size_t)unit * 64;
  if (k0 >= k1) {
    // Empty split: mark so the merge skips it.
    if (lane < 32) {
      pml[2 * lane] = kNegBig;
      pml[2 * lane + 1] = 0.f;
    }
    return;
  }

  // Query column q = r*L + i (head h*rep + r, verify row i).
  const int qcol = c32;
  const int qr = qcol / p.L;
  const int qi = qcol - qr * p.L;
  const bool qvalid = (qr < rep) && (qi < L);
  const int qbound = qs + qi;  // last key this column may see

  // B operand Q^T: lane (q, h2) holds d = 64*h2 + 8*i + e for MFMA i.
  bf16x8 qop[8];
  {
    const uint16_t* qrow = p.q + ((((size_t)b * p.Hq + h * rep + (qvalid ? qr : 0)) * p.L + (qvalid ? qi : 0)) * kHD);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint4 raw = qvalid ? *reinterpret_cast<const uint4*>(qrow + 64 * h2 + 8 * i) : make_uint4(0, 0, 0, 0);
      qop[i] = __builtin_bit_cast(bf16x8, raw);
    }
  }

  f32x16 o[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) o[t] = f32x16{};
  float m_run = kNegBig;
  float l_run = 0.f;

  const uint16_t* kbase = p.k + ((size_t)b * p.Hkv + h) * (size_t)p.cap * kHD;
  const uint16_t* vbase = p.v + ((size_t)b * p.Hkv + h) * (size_t)p.cap * kHD;

  for (int kt = k0; kt < k1; kt += kTileKeys) {
    // The 8 KB K and V tiles with contiguous loads (instruction i: bytes
    // 1024 i + 16 lane, i.e. key 4 i + lane / 16, d 8 (lane % 16)); keys past
    // k1 read as zero (stale cache bits cannot leak into P V).
    uint4 kc[8], vc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = kt + 4 * i + (lane >> 4);
      const bool kin = key < k1;
      const size_t off = (size_t)(kin ? key : kt) * kHD + 8 * (lane & 15);
      kc[i] = kin ? ld_stream(kbase + off) : make_uint4(0, 0, 0, 0);
      vc[i] = kin ? ld_stream(vbase + off) : make_uint4(0, 0, 0, 0);
    }
    __syncthreads();   // the previous tile's LDS reads are done
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int o = (4 * i + (lane >> 4)) * kVrowStride + 8 * (lane & 15);
      *reinterpret_cast<uint4*>(ktile + o) = kc[i];
      *reinterpret_cast<uint4*>(vtile + o) = vc[i];
    }
    __syncthreads();
    // K operands: lane (key c32, half h2) takes d 64 h2 + 8 i .. + 7 of MFMA i.
    uint4 kr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) kr[i] = *reinterpret_cast<const uint4*>(ktile + c32 * kVrowStride + 64 * h2 + 8 * i);
    // S^T[key][q]
    f32x16 st = {};
#pragma unroll
    for (int i = 0; i < 8; ++i)
      st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kr[i]), qop[i], st, 0, 0, 0);


    // Scale, mask, tile max for column q (this lane's 16 keys + lane^32's).
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

    // P^T operands: MFMA j uses registers 8j..8j+7.
    bf16x8 pop[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      uint32_t pk[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) pk[t] = pack_bf2(sv[8 * jj + 2 * t], sv[8 * jj + 2 * t + 1]);
      pop[jj] = __builtin_bit_cast(bf16x8, pk);
    }
    // O^T[d][q] += V^T[d][keys] P^T[keys][q]; slot e of lane (d, h2) in step j
    // is key 16j + (e<4 ? 4*h2+e : 8+4*h2+e-4): two transposing reads, keys
    // 16j + 4 h2 + {0..3} and 16j + 8 + 4 h2 + {0..3}, for d = 32t + lane % 32.
    const int gj = lane & 15;
    const uint16_t* vlane = vtile + (4 * h2 + (gj >> 2)) * kVrowStride + 16 * ((lane >> 4) & 1) + 4 * (gj & 3);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const v4i16_t lo = lds_read_tr16(vlane + 16 * jj * kVrowStride + 32 * t);
        const v4i16_t hi = lds_read_tr16(vlane + (16 * jj + 8) * kVrowStride + 32 * t);
        const uint4 e8 = make_uint4((uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16),
                                    (uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16),
                                    (uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16),
                                    (uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16));
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, e8), pop[jj], o[t], 0, 0, 0);
      }
    }
  }

  // Split partial: l over both halves of the column; O^T rows d, column q.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (h2 == 0) {
    pml[2 * qcol] = m_run;
    pml[2 * qcol + 1] = l_tot;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = 32 * t + 8 * (r >> 2) + 4 * h2 + (r & 3);
      po[qcol * kHD + d] = o[t][r];
    }
}

// Standalone kernels of the operand-major split and merge bodies.
template <int TPW>
__global__ __launch_bounds__(kVtWaves * 64) void attn_vt_kernel(AttnParams p) {
  __shared__ __align__(16) unsigned char lds[attn_vt_lds_bytes()];
  attn_vt_body<TPW, false>(p, (int)blockIdx.x, lds);
}

// Two waves per SIMD (256 registers; 280 unconstrained, one wave): cfg4
// step 25.6-26.0 -> 25.2-25.5 ms, cfg2 within 2%.
template <int NRG>
__global__ __launch_bounds__(kVtWaves * 64, 2) void attn_vl_kernel(AttnParams p) {
  __shared__ __align__(16) unsigned char lds[attn_vt_lds_bytes()];
  attn_vl_body<false, NRG>(p, (int)blockIdx.x, lds);
}

// Balanced work over the per-request-capacity layout (attn_bal_body): one
// round of workgroups, each streaming the same share of the batch's K and V.
template <int NRG>
__global__ __launch_bounds__(kVtWaves * 64, 2) void attn_bal_kernel(AttnParams p) {
  __shared__ __align__(16) unsigned char lds[attn_bal_lds_bytes()];
  attn_bal_body<false, NRG>(p, lds);
}


// Workgroups of the balanced kernel: one per CU (cfg2: 96.8 us at one per
// CU, 99.0 at two, 109 at four, 118 at half the CUs), at most
// (kMaxSplits - 2) * Hkv so that no head has more than kMaxSplits partials
// (a head holds at most 1/Hkv of the tiles, so it meets at most G / Hkv + 2
// workgroups). Partial slots: at most G - 1 plus one per head.
static int attn_bal_grid(int Hkv) {
  const long long g = device_cus();
  const long long lim = (long long)(kMaxSplits - 2) * Hkv;
  return (int)(g < lim ? g : lim);
}
static size_t attn_bal_ws_bytes(int B, int Hkv) {
  const size_t slots = (size_t)attn_bal_grid(Hkv) + (size_t)B * Hkv;
  return slots * 32 * kHD * sizeof(float) + slots * 64 * sizeof(float) + (size_t)2 * B * Hkv * sizeof(int32_t);
}
static bool attn_bal_enabled(int B, int split_keys) {
  static int env = -1;
  if (env < 0) {
    const char* v = getenv("MTPLX_AMD_ATTN_BALANCED");
    env = (v && *v) ? atoi(v) : 1;
  }
  return env != 0 && split_keys <= 0 && B <= kBalMaxReq;
}

// Keys per work unit of the block-layout entry point: about 1024 units over
// the batch's summed capacity (total_cap * Hkv), at least 128 keys (one tile
// per wave), at most 4096, a multiple of 128; then at most kMaxSplits splits
// of the largest capacity.
static int attn_blocks_plan(int Hkv, int cap, long long total_cap, int req, int* S, int* sk_out) {
  int sk = req;
  if (sk <= 0) {
    const long long work = total_cap * Hkv;
    // 1024 units: 512-1024 measured within 2% on cfg2 and cfg4; 2048 and
    // more slower (per-unit partials and ramp), 256 slower on cfg2.
    sk = (int)((work + 1023) / 1024);
    if (sk < 128) sk = 128;
    if (sk > 4096) sk = 4096;
  }
  sk = ((sk + 127) / 128) * 128;
  int s = cdiv(cap, sk);
  if (s > kMaxSplits) {
    sk = ((cdiv(cap, kMaxSplits) + 127) / 128) * 128;
    s = cdiv(cap, sk);
  }
  *S = s;
  *sk_out = sk;
  return MTP_OK;
}

__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(AttnParams p) {
  __shared__ __align__(16) unsigned char lds[attn_merge_lds_bytes()];
  attn_merge_body<false>(p, (int)blockIdx.x, lds);
}

__global__ __launch_bounds__(kMergeHeadThreads) void attn_merge_head_kernel(AttnParams p) {
  attn_merge_head_body<false>(p, (int)blockIdx.x);
}

// The split merge: one workgroup per (request, kv head) with all its query
// columns when the batch has many heads (ragged batches, a few partials per
// head), else one per (request, kv head, query column) (few heads with many
// partials each: the cfg3 step's 8 heads x 32 splits). MTPLX_AMD_ATTN_MERGE_HEAD=0
// keeps the per-column form everywhere. ``per_head`` forces the per-head
// form whatever the batch: a caller-given split length uses it, so a
// request's merged output depends only on its own keys and the split length,
// never on the other requests in the batch (the two forms round differently).
constexpr int kMergeHeadMinHeads = 64;
static void launch_merge(const AttnParams& p, int B, int Hq, int Hkv, int L, hipStream_t st, bool per_head = false) {
  const char* v = getenv("MTPLX_AMD_ATTN_MERGE_HEAD");
  const bool off = v && *v && atoi(v) == 0;
  if (per_head || (!off && B * Hkv >= kMergeHeadMinHeads))
    hipLaunchKernelGGL(attn_merge_head_kernel, dim3((unsigned)(B * Hkv)), dim3(kMergeHeadThreads), 0, st, p);
  else
    hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)(B * Hkv * (Hq / Hkv) * L)), dim3(kMergeThreads), 0, st, p);
}

// Split length: ~2048 work units over the whole capacity (ragged rows leave
// the units past their length empty), 64..4096 keys, a multiple of the tile.
static int attn_plan(int B, int Hkv, int cap, int split_keys_req, int* S, int* split_keys) {
  int sk = split_keys_req;
  if (sk <= 0) {
    const long long total = (long long)cap * B * Hkv;
    sk = (int)((total + 2047) / 2048);
    if (sk < 64) sk = 64;
    if (sk > 4096) sk = 4096;
  }
  sk = ((sk + kTileKeys - 1) / kTileKeys) * kTileKeys;
  int s = cdiv(cap, sk);
  if (s > kMaxSplits) {
    s = kMaxSplits;
    sk = ((cdiv(cap, s) + kTileKeys - 1) / kTileKeys) * kTileKeys;
    s = cdiv(cap, sk);
  }
  *split_keys = sk;
  *S = s;
  return MTP_OK;
}

// ---------------------------------------------------------------------------
// KV cache mechanics (mtplx/ragged_kv_cache.py:201-277, :473-496).

// new [B, Hkv, q, D] -> cache[b, h, ws[b] + i, :]; 16 B per thread.
__global__ void kv_scatter_kernel(uint16_t* kc, uint16_t* vc, const uint16_t* kn, const uint16_t* vn,
                                  const int32_t* ws, int B, int Hkv, int cap, int q, int D, int32_t* status) {
  const size_t n16 = (size_t)B * Hkv * q * D / 8;
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n16; t += (size_t)gridDim.x * blockDim.x) {
    const size_t e = t * 8;
    const int d = (int)(e % D);
    const size_t r = e / D;
    const int i = (int)(r % q);
    const size_t bh = r / q;
    const int b = (int)(bh / Hkv);
    const int pos = ws[b] + i;
    if (pos < 0 || pos >= cap) {
      if (status) atomicOr(status, 1);
      continue;
    }
    const size_t dst = (bh * cap + pos) * D + d;
    *reinterpret_cast<uint4*>(kc + dst) = *reinterpret_cast<const uint4*>(kn + e);
    *reinterpret_cast<uint4*>(vc + dst) = *reinterpret_cast<const uint4*>(vn + e);
  }
}

// Rows with mask[b] take the snapshot over positions [lo, hi) (snapshot zero
// padded past its capacity); other rows untouched.
__global__ void kv_restore_kernel(uint16_t* cur, const uint16_t* snap, const uint8_t* mask, int B, int Hkv,
                                  int cap, int snap_cap, int D, int lo, int hi) {
  const int span = hi - lo;
  const size_t n16 = (size_t)B * Hkv * span * D / 8;
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n16; t += (size_t)gridDim.x * blockDim.x) {
    const size_t e = t * 8;
    const int d = (int)(e % D);
    const size_t r = e / D;
    const int pos = lo + (int)(r % span);
    const size_t bh = r / span;
    const int b = (int)(bh / Hkv);
    if (!mask[b]) continue;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (pos < snap_cap) val = *reinterpret_cast<const uint4*>(snap + (bh * snap_cap + pos) * D + d);
    *reinterpret_cast<uint4*>(cur + (bh * cap + pos) * D + d) = val;
  }
}

// bool mask [B, 1, q_len, key_len]: mask[b,0,i,j] = j <= q_start[b] + i.
__global__ void ragged_mask_kernel(uint8_t* out, const int32_t* qs, int B, int q_len, int key_len) {
  const size_t n = (size_t)B * q_len * key_len;
  for (size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x; t < n; t += (size_t)gridDim.x * blockDim.x) {
    const int j = (int)(t % key_len);
    const size_t r = t / key_len;
    const int i = (int)(r % q_len);
    const int b = (int)(r / q_len);
    out[t] = (j <= qs[b] + i) ? 1 : 0;
  }
}

static int grid_for(size_t n, int block) {
  size_t g = (n + block - 1) / block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

}  // namespace mtp

using namespace mtp;

MTP_API size_t mtp_attn_workspace_bytes(int B, int Hkv, int cap, int split_keys) {
  int S, sk;
  attn_plan(B, Hkv, cap, split_keys, &S, &sk);
  const size_t units = (size_t)B * Hkv * S;
  return units * 32 * kHD * sizeof(float) + units * 64 * sizeof(float);
}

static int attn_run(const void* q, const void* k, const void* v, const int32_t* q_start, const int32_t* q_lens,
                    void* out, int out_rows, int B, int Hq, int Hkv, int L, int D, int cap, float scale,
                    int split_keys, void* ws, size_t ws_bytes, void* stream, const char* who) {
  if (!q || !k || !v || !q_start || !out || B < 1 || Hq < 1 || Hkv < 1 || L < 1 || cap < 1) {
    set_error("%s: bad arguments", who);
    return MTP_ERR_ARG;
  }
  if (D != kHD) {
    set_error("%s: head_dim %d unsupported (128)", who, D);
    return MTP_ERR_UNSUPPORTED;
  }
  if (Hq % Hkv) {
    set_error("%s: Hq=%d not a multiple of Hkv=%d", who, Hq, Hkv);
    return MTP_ERR_ARG;
  }
  if ((Hq / Hkv) * L > 32) {
    set_error("%s: (Hq/Hkv)*L = %d query rows per kv head exceeds 32", who, (Hq / Hkv) * L);
    return MTP_ERR_UNSUPPORTED;
  }
  AttnParams p = {};
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v;
  p.q_start = q_start;
  p.q_lens = q_lens;
  p.out = (uint16_t*)out;
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.L = L;
  p.cap = cap;
  p.out_rows = out_rows;
  attn_plan(B, Hkv, cap, split_keys, &p.S, &p.split_keys);
  p.scale_log2 = scale * 1.4426950408889634f;
  const size_t need = mtp_attn_workspace_bytes(B, Hkv, cap, split_keys);
  if (!ws || ws_bytes < need) {
    set_error("%s: workspace %zu B < required %zu B", who, ws_bytes, need);
    return MTP_ERR_WORKSPACE;
  }
  const size_t units = (size_t)B * Hkv * p.S;
  p.part_o = (float*)ws;
  p.part_ml = p.part_o + units * 32 * kHD;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(attn_split_kernel, dim3((unsigned)units), dim3(64), 0, st, p);
  int rc = launch_check(who);
  if (rc) return rc;
  launch_merge(p, B, Hq, Hkv, L, st);
  return launch_check(who);
}

MTP_API int mtp_ragged_gqa_attn(const void* q, const void* k, const void* v, const int32_t* q_start,
                                const int32_t* q_lens, void* out, int B, int Hq, int Hkv, int L, int D, int cap,
                                float scale, int split_keys, void* ws, size_t ws_bytes, void* stream) {
  return attn_run(q, k, v, q_start, q_lens, out, 0, B, Hq, Hkv, L, D, cap, scale, split_keys, ws, ws_bytes, stream,
                  "mtp_ragged_gqa_attn");
}

MTP_API int mtp_ragged_gqa_attn_rows(const void* q, const void* k, const void* v, const int32_t* q_start,
                                     const int32_t* q_lens, void* out, int B, int Hq, int Hkv, int L, int D, int cap,
                                     float scale, int split_keys, void* ws, size_t ws_bytes, void* stream) {
  return attn_run(q, k, v, q_start, q_lens, out, 1, B, Hq, Hkv, L, D, cap, scale, split_keys, ws, ws_bytes, stream,
                  "mtp_ragged_gqa_attn_rows");
}

MTP_API size_t mtp_attn_vt_workspace_bytes(int B, int Hkv, int cap) {
  int S = 0, tpw = 1;
  if (B < 1 || Hkv < 1 || cap < 1 || attn_vt_plan(cap, &S, &tpw) != MTP_OK) return 0;
  const size_t units = (size_t)B * Hkv * S;
  return units * 32 * kHD * sizeof(float) + units * 64 * sizeof(float);
}

MTP_API int mtp_ragged_gqa_attn_rows_vt(const void* q, const void* k, const void* v_vt, const int32_t* q_start,
                                        const int32_t* q_lens, void* out, int B, int Hq, int Hkv, int L, int D,
                                        int cap, float scale, void* ws, size_t ws_bytes, void* stream) {
  const char* who = "mtp_ragged_gqa_attn_rows_vt";
  if (!q || !k || !v_vt || !q_start || !out || B < 1 || Hq < 1 || Hkv < 1 || L < 1 || cap < 32 || cap % 32) {
    set_error("%s: bad arguments (cap must be a positive multiple of 32)", who);
    return MTP_ERR_ARG;
  }
  if (D != kHD) {
    set_error("%s: head_dim %d unsupported (128)", who, D);
    return MTP_ERR_UNSUPPORTED;
  }
  if (Hq % Hkv || (Hq / Hkv) * L > 32) {
    set_error("%s: need Hq %% Hkv == 0 and (Hq/Hkv)*L <= 32 (Hq=%d Hkv=%d L=%d)", who, Hq, Hkv, L);
    return MTP_ERR_UNSUPPORTED;
  }
  AttnParams p{};
  p.q = (const uint16_t*)q;
  p.k = (const uint16_t*)k;
  p.v = (const uint16_t*)v_vt;
  p.q_start = q_start;
  p.q_lens = q_lens;
  p.out = (uint16_t*)out;
  p.B = B;
  p.Hq = Hq;
  p.Hkv = Hkv;
  p.L = L;
  p.cap = cap;
  p.out_rows = 1;
  p.scale_log2 = scale * 1.4426950408889634f;
  int tpw = 1;
  if (attn_vt_plan(cap, &p.S, &tpw) != MTP_OK) {
    set_error("%s: capacity %d needs more than %d splits", who, cap, kMaxSplits);
    return MTP_ERR_UNSUPPORTED;
  }
  p.split_keys = kVtWaves * kTileKeys * tpw;
  const size_t need = mtp_attn_vt_workspace_bytes(B, Hkv, cap);
  if (!ws || ws_bytes < need) {
    set_error("%s: workspace %zu < %zu", who, ws_bytes, need);
    return MTP_ERR_WORKSPACE;
  }
  const size_t units = (size_t)B * Hkv * p.S;
  p.part_o = (float*)ws;
  p.part_ml = (float*)ws + units * 32 * kHD;
  if (tpw == 1)
    hipLaunchKernelGGL(attn_vt_kernel<1>, dim3((unsigned)units), dim3(kVtWaves * 64), 0, (hipStream_t)stream, p);
  else
    hipLaunchKernelGGL(attn_vt_kernel<2>, dim3((unsigned)units), dim3(kVtWaves * 64), 0, (hipStream_t)stream, p);
  int rc = launch_check(who);
  if (rc) return rc;
  launch_merge(p, B, Hq, Hkv, L, (hipStream_t)stream);
  return launch_check(who);
}

MTP_API int mtp_kv_scatter(void* k_cache, void* v_cache, const void* k_new, const void* v_new,
                           const int32_t* write_start, int B, int Hkv, int cap, int q, int D, int32_t* status,
                           void* stream) {
  if (!k_cache || !v_cache || !k_new || !v_new || !write_start || B < 1 || Hkv < 1 || cap < 1 || q < 1 ||
      D < 8 || D % 8) {
    set_error("mtp_kv_scatter: bad arguments (D must be a multiple of 8)");
    return MTP_ERR_ARG;
  }
  const size_t n16 = (size_t)B * Hkv * q * D / 8;
  hipLaunchKernelGGL(kv_scatter_kernel, dim3(grid_for(n16, 256)), dim3(256), 0, (hipStream_t)stream,
                     (uint16_t*)k_cache, (uint16_t*)v_cache, (const uint16_t*)k_new, (const uint16_t*)v_new,
                     write_start, B, Hkv, cap, q, D, status);
  return launch_check("mtp_kv_scatter");
}

MTP_API int mtp_kv_restore_masked(void* cur, const void* snap, const uint8_t* row_mask, int B, int Hkv, int cap,
                                  int snap_cap, int D, int lo, int hi, void* stream) {
  if (!cur || !snap || !row_mask || B < 1 || Hkv < 1 || cap < 1 || snap_cap < 0 || D < 8 || D % 8 || lo < 0 ||
      hi > cap || lo > hi) {
    set_error("mtp_kv_restore_masked: bad arguments");
    return MTP_ERR_ARG;
  }
  if (hi == lo) return MTP_OK;
  const size_t n16 = (size_t)B * Hkv * (hi - lo) * D / 8;
  hipLaunchKernelGGL(kv_restore_kernel, dim3(grid_for(n16, 256)), dim3(256), 0, (hipStream_t)stream,
                     (uint16_t*)cur, (const uint16_t*)snap, row_mask, B, Hkv, cap, snap_cap, D, lo, hi);
  return launch_check("mtp_kv_restore_masked");
}

MTP_API int mtp_ragged_causal_mask(uint8_t* out, const int32_t* q_start, int B, int q_len, int key_len,
                                   void* stream) {
  if (!out || !q_start || B < 1 || q_len < 1 || key_len < 1) {
    set_error("mtp_ragged_causal_mask: bad arguments");
    return MTP_ERR_ARG;
  }
  const size_t n = (size_t)B * q_len * key_len;
  hipLaunchKernelGGL(ragged_mask_kernel, dim3(grid_for(n, 256)), dim3(256), 0, (hipStream_t)stream, out, q_start, B,
                     q_len, key_len);
  return launch_check("mtp_ragged_causal_mask");
}

MTP_API size_t mtp_attn_blocks_workspace_bytes(int B, int Hkv, int cap, long long total_cap, int split_keys) {
  if (B < 1 || Hkv < 1 || cap < 32) return 0;
  int S, sk;
  attn_blocks_plan(Hkv, cap, total_cap > 0 ? total_cap : (long long)B * cap, split_keys, &S, &sk);
  const size_t units = (size_t)B * Hkv * S;
  const size_t unit_bytes = units * 32 * kHD * sizeof(float) + units * 64 * sizeof(float);
  if (!attn_bal_enabled(B, split_keys)) return unit_bytes;
  const size_t bal = attn_bal_ws_bytes(B, Hkv);
  return bal > unit_bytes ? bal : unit_bytes;
}

MTP_API int mtp_ragged_gqa_attn_blocks(const mtp_attn_blocks_args* a, void* stream) {
  const char* who = "mtp_ragged_gqa_attn_blocks";
  if (!a || !a->q || !a->k_blk || !a->v_blk || !a->q_start || !a->out || a->B < 1 || a->Hq < 1 || a->Hkv < 1 ||
      a->Lmax < 1 || a->cap < 32 || a->cap % 32) {
    set_error("%s: bad arguments (cap a positive multiple of 32)", who);
    return MTP_ERR_ARG;
  }
  if (a->D != kHD) {
    set_error("%s: head_dim %d unsupported (128)", who, a->D);
    return MTP_ERR_UNSUPPORTED;
  }
  if (a->Hq % a->Hkv || (a->Hq / a->Hkv) * a->Lmax > 32) {
    set_error("%s: need Hq %% Hkv == 0 and (Hq/Hkv)*Lmax <= 32 (Hq=%d Hkv=%d Lmax=%d)", who, a->Hq, a->Hkv, a->Lmax);
    return MTP_ERR_UNSUPPORTED;
  }
  AttnParams p{};
  p.q = (const uint16_t*)a->q;
  p.k = (const uint16_t*)a->k_blk;
  p.v = (const uint16_t*)a->v_blk;
  p.q_start = a->q_start;
  p.q_lens = a->q_lens;
  p.row_off = a->row_off;
  p.kv_off = a->kv_off;
  p.out = (uint16_t*)a->out;
  p.B = a->B;
  p.Hq = a->Hq;
  p.Hkv = a->Hkv;
  p.L = a->Lmax;
  p.cap = a->cap;
  p.out_rows = 1;
  p.scale_log2 = a->scale * 1.4426950408889634f;
  const long long total = a->total_cap > 0 ? a->total_cap : (long long)a->B * a->cap;
  if (attn_bal_enabled(a->B, a->split_keys)) {
    // One round of workgroups with equal shares of the batch's tiles; the
    // merge reads each head's partial slots from the table.
    const int G = attn_bal_grid(a->Hkv);
    const size_t need = attn_bal_ws_bytes(a->B, a->Hkv);
    if (!a->ws || a->ws_bytes < need) {
      set_error("%s: workspace %zu < %zu (mtp_attn_blocks_workspace_bytes)", who, a->ws_bytes, need);
      return MTP_ERR_WORKSPACE;
    }
    const size_t slots = (size_t)G + (size_t)a->B * a->Hkv;
    p.part_o = (float*)a->ws;
    p.part_ml = (float*)a->ws + slots * 32 * kHD;
    p.bal_tab = reinterpret_cast<int32_t*>((float*)a->ws + slots * (32 * kHD + 64));
    p.S = 1;
    p.split_keys = kTileKeys;
    // One ring slot: 96.8 us on cfg2 against 128.2 with two (the deeper
    // ring keeps twice the bytes in flight, which this HBM serves worse).
    hipLaunchKernelGGL(attn_bal_kernel<1>, dim3((unsigned)G), dim3(kVtWaves * 64), 0, (hipStream_t)stream, p);
    int rc = launch_check(who);
    if (rc) return rc;
    launch_merge(p, a->B, a->Hq, a->Hkv, a->Lmax, (hipStream_t)stream);
    return launch_check(who);
  }
  attn_blocks_plan(a->Hkv, a->cap, total, a->split_keys, &p.S, &p.split_keys);
  const size_t need = mtp_attn_blocks_workspace_bytes(a->B, a->Hkv, a->cap, a->total_cap, a->split_keys);
  if (!a->ws || a->ws_bytes < need) {
    set_error("%s: workspace %zu < %zu (mtp_attn_blocks_workspace_bytes)", who, a->ws_bytes, need);
    return MTP_ERR_WORKSPACE;
  }
  const size_t units = (size_t)a->B * a->Hkv * p.S;
  p.part_o = (float*)a->ws;
  p.part_ml = (float*)a->ws + units * 32 * kHD;
  // One ring slot: 105.6 us on cfg2 against 123.1 with two (122 and 129 with
  // three and four).
  hipLaunchKernelGGL(attn_vl_kernel<1>, dim3((unsigned)units), dim3(kVtWaves * 64), 0, (hipStream_t)stream, p);
  int rc = launch_check(who);
  if (rc) return rc;
  // A given split length: the per-head merge in every batch (batch-invariant rows).
  launch_merge(p, a->B, a->Hq, a->Hkv, a->Lmax, (hipStream_t)stream, a->split_keys > 0);
  return launch_check(who);
}
