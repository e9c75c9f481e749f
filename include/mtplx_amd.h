/*
 * C ABI of the MI355X (gfx950) speculative-verify hot path.
 *
 * Conventions for every entry point:
 *   - returns 0 on success, a negative MTP_ERR_* code otherwise; the message
 *     is in mtp_last_error() (thread-local);
 *   - all pointers are device pointers (hipMalloc / torch CUDA tensors) unless
 *     stated; bf16 tensors are passed as raw 16-bit patterns (void*);
 *   - work is enqueued on `stream` (a hipStream_t, NULL = default stream) and
 *     is asynchronous; nothing allocates device memory: callers pass a
 *     workspace sized by the matching *_workspace_bytes() query;
 *   - workspaces hold self-resetting arrival counters: give each stream its
 *     own workspace, zero-filled once when first allocated.
 *
 * Reference interfaces replaced are cited as file:line of youssofal/MTPLX.
 */
#ifndef MTPLX_AMD_H
#define MTPLX_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MTP_OK = 0,
  MTP_ERR_ARG = -1,
  MTP_ERR_UNSUPPORTED = -2,
  MTP_ERR_WORKSPACE = -3,
  MTP_ERR_HIP = -4
};

const char* mtp_last_error(void);

/* ---- 4-bit affine quantized verify matmul ------------------------------
 * y[M,N] = x[M,K] @ dequant(w)^T, w uint32 [N,K/8] little-endian nibbles,
 * scales/biases bf16 [N,K/group_size], group_size 64 or 128, 1 <= M <= 32,
 * K % 64 == 0, x/w 16-byte aligned. fp32 accumulation, bf16 output.
 * Replaces: mtplx/verify_qmv.py:194 multi3_qmv4_matmul, :1217
 * stocklike_qmv4_matmul, mtplx/kernels/qmv4_matmul.py:185 qmv4_matmul,
 * mtplx/verify_kernels.py:580 vk_qmm_m4_impl (-> _run_ksplit :531), and the
 * M<=16 routes of mtplx/nax_verify.py:754 (nax_qmm_m4 :977, m6 :628, m16 :690).
 * `dual` selects the two-matrix workspace size (mtp_qmv_affine4_dual). */
size_t mtp_qmv_workspace_bytes(int M, int N, int K, int dual);
int mtp_qmv_affine4(const void* x, const void* w, const void* scales, const void* biases, void* y, int M, int N,
                    int K, int group_size, void* ws, size_t ws_bytes, void* stream);

/* 1 when the RoPE epilogue (emode 4 of mtp_qmv_affine4_ex) takes M rows of a
 * K-wide x into an N-wide q|k|v projection (M <= 16, all of x in LDS), else
 * 0. No reference counterpart: it tells the fused verify step whether the
 * q|k|v projection can write RoPE'd rows and the K/V cache itself. */
int mtp_qmv_rope_fusable(int M, int N, int K);

/* General affine quantized matmul for the formats the MFMA kernel does not
 * take: bits 4 or 8, group_size 32, 64 or 128, any M >= 1 (launches of 8
 * rows), K a multiple of 32 and of group_size, w 16-byte aligned. Weights
 * uint32 [N, K*bits/32] (little-endian bit fields), scales/biases bf16
 * [N, K/gs]; x bf16 [M, K]; output bf16 y or (y NULL) fp32 yf holding bf16
 * values, [M, N]. fp32 accumulation, VALU (not the HBM-rate lane).
 * Replaces: mtplx/verify_qmv.py:1377 stocklike_qmv8_matmul (8-bit verify
 * rows, eligibility :1256), the group-32 routes of
 * mtplx/kernels/qmv4_matmul.py:185 qmv4_matmul and
 * mtplx/verify_crossrow.py:249 crossrow_qmm, and the mx.quantized_matmul
 * fallback those lanes take on other shapes. */
int mtp_qmv_affine(const void* x, const void* w, const void* scales, const void* biases, void* y, void* yf, int M,
                   int N, int K, int group_size, int bits, void* stream);

/* Activation chunk sums of the cross-row lane (mtplx/verify_crossrow.py:111
 * make_chunk_sums): out[(kb*32 + lane)*8 + m] = sum over i < 16 of
 * x[m, kb*512 + lane*16 + i] (fp32, index order), rows m >= M zero;
 * 1 <= M <= 8, K a multiple of 512; out holds K/512*32*8 floats. */
int mtp_chunk_sums(const void* x, int M, int K, float* out, void* stream);

/* The cross-row lane's matmul with its precomputed chunk sums
 * (mtplx/verify_crossrow.py:249 crossrow_qmm(..., xsums=make_chunk_sums(x))):
 * 4-bit affine, group 32 or 64, 1 <= M <= 8, K a multiple of 512; x bf16
 * [M, K], xsums the mtp_chunk_sums table of x; y bf16 [M, N]. Each 32-k
 * block's bias term b * sum(x) reads its sum from the table (two 16-value
 * slices) instead of re-summing the staged x; otherwise as mtp_qmv_affine. */
int mtp_crossrow_qmm(const void* x, const float* xsums, const void* w, const void* scales, const void* biases,
                     void* y, int M, int N, int K, int group_size, void* stream);

/* y = bf16(bf16(x @ W^T) + resid) — the residual add that follows o_proj and
 * down_proj in the verify forward (mlx-lm decoder layer `h + r`).
 * resid may alias y. ss_out (NULL = skip) receives, for each 32-column block
 * j and row m, ss_out[j*32 + m] = sum of squares of the stored y values: the
 * statistic a following fused RMSNorm needs (pass it as that call's ss_in). */
int mtp_qmv_affine4_residual(const void* x, const void* w, const void* scales, const void* biases,
                             const void* resid, void* y, float* ss_out, int M, int N, int K, int group_size,
                             void* ws, size_t ws_bytes, void* stream);

/* Gate/up pair sharing one read of x. swiglu=0: y0 = x@W0^T, y1 = x@W1^T
 * (mtplx/verify_qmv.py:614 multi3_dual_qmv4_matmul, :833 parallel dual);
 * swiglu=1: y0 = silu(x@W0^T) * (x@W1^T), y1 unused. */
int mtp_qmv_affine4_dual(const void* x, const void* w0, const void* s0, const void* b0, const void* w1,
                         const void* s1, const void* b1, void* y0, void* y1, int M, int N, int K, int group_size,
                         int swiglu, void* ws, size_t ws_bytes, void* stream);

/* y = (silu(gate) * up) @ W^T (+ resid if resid != NULL).
 * Replaces mtplx/verify_qmv.py:1063 multi3_swiglu_down_qmv4_matmul. */
int mtp_qmv_affine4_swiglu_in(const void* gate, const void* up, const void* w, const void* scales,
                              const void* biases, const void* resid, void* y, int M, int N, int K, int group_size,
                              void* ws, size_t ws_bytes, void* stream);

/* y = rmsnorm(x; norm_w, eps) @ W^T, the norm fused into the matmul's
 * activation staging (the layer's input_layernorm + q|k|v projection).
 * ss_in: the producer's ss_out for x (K/32 blocks), or NULL to compute the
 * row statistics here. */
int mtp_qmv_affine4_rmsnorm_in(const void* x, const void* norm_w, const float* ss_in, float eps, const void* w,
                               const void* scales,
                               const void* biases, void* y, int M, int N, int K, int group_size, void* ws,
                               size_t ws_bytes, void* stream);

/* fp32 logits: y = float(bf16(rmsnorm(x) @ W^T)) (norm_w NULL = no norm);
 * the lm_head of the verify rows feeding the sampler. */
int mtp_qmv_affine4_rmsnorm_f32(const void* x, const void* norm_w, const float* ss_in, float eps, const void* w,
                                const void* scales,
                                const void* biases, float* y, int M, int N, int K, int group_size, void* ws,
                                size_t ws_bytes, void* stream);

/* y = silu(rmsnorm(x)@W0^T) * (rmsnorm(x)@W1^T): post-attention norm + gate/up. */
int mtp_qmv_affine4_rmsnorm_dual(const void* x, const void* norm_w, const float* ss_in, float eps, const void* w0,
                                 const void* s0,
                                 const void* b0, const void* w1, const void* s1, const void* b1, void* y, int M,
                                 int N, int K, int group_size, void* ws, size_t ws_bytes, void* stream);

/* ---- Tile-major packed weights + generic entry -----------------------------
 * mtp_pack_affine4 rewrites one 4-bit affine matrix (MLX layout above) into
 * the layout the streaming kernel reads with full-line loads: per 32-row tile
 * and 256-column quad, 1152 words = 4 x 256 words of nibbles in wave-load
 * order, then 32 rows x (4 scales, 4 biases) bf16; rows past N are zero.
 * No reference counterpart: the reference reads MLX's layout directly
 * (mtplx/verify_kernels.py:69-88); this is the MI355X memory layout of the
 * same values, produced once at load time. */
size_t mtp_pack_affine4_bytes(int N, int K);
int mtp_pack_affine4(const void* w, const void* scales, const void* biases, void* out, int N, int K, int group_size,
                     void* stream);
/* Layout 2, the same size, for M <= 16 on the 16x16x32 MFMA (packed = 2 in
 * mtp_qmv_args): in block (t, q), load u = 64-group u of the quad, and lane l
 * gets word jj = 2kk + h = word 8u + 4kk + l/16 of row 32t + 16h + l%16;
 * nibble order and the scale/bias words as in layout 1. No reference
 * counterpart (a memory layout of the same values). */
int mtp_pack_affine4_mf16(const void* w, const void* scales, const void* biases, void* out, int N, int K,
                          int group_size, void* stream);

/* Every verify-matmul variant through one argument block. xmode: 0 = x,
 * 1 = silu(x)*x2 (x2 = up), 2 = rmsnorm(x; norm weight x2, eps, ss_in),
 * 3 = x with its per-32-column row sums in x_sums ([K/32][32] fp32, as the
 * y_sums output below writes them; packed weights only);
 * emode: 0 = store (y0 bf16, or yf fp32 when set), 1 = + resid (ss_out
 * optional), 2 = two outputs (w1 -> y1), 3 = silu(x@W0^T)*(x@W1^T).
 * packed = 1: w0/w1 come from mtp_pack_affine4 (s0/b0/s1/b1 unused);
 * packed = 2: from mtp_pack_affine4_mf16, M <= 16 only (16x16x32 MFMA).
 * ldx/ldy <= 0 mean K/N.
 * ws/ws_bytes: with packed weights, a workspace of mtp_qmv_workspace_bytes
 * (256-byte aligned, zeroed once before first use and then left to the
 * library; calls sharing one workspace must be stream-ordered). The per-tile
 * kernel then splits the leftover tiles of its last round by K over all CUs
 * (tiles mod CUs must divide the CU count), or, with fewer tiles than CUs,
 * every tile into floor(CUs / tiles) parts (M <= 16); the parts are summed in
 * a fixed order. Without a workspace it runs unsplit. schedule must be 0.
 * emode 4 = q|k|v projection with RoPE and the cache write fused into the
 * epilogue (the work of mtp_rope_qkv_to_cache / _vt below, same rounding):
 * rope points at the outputs; y0 is unused; packed weights whose rows are in
 * RoPE tile order - packed row 32t + c of head h = t / (D/32), sub-block
 * sb = t % (D/32) is original row h*D + 16 sb + c % 16 + (c / 16) * D/2 -
 * so each 32-column tile holds 16 rotate-half pairs. M <= 8, M = B * L. */
typedef struct mtp_rope_out {
  const int32_t* q_start; /* [B] first position of each request's rows */
  const int32_t* q_lens;  /* [B] rows written to the cache, or NULL (= L) */
  void* q_out;            /* [B, Hq, L, D] bf16 */
  void* k_cache;          /* blocked = 1: operand-major blocks (below); 0: [B, Hkv, cap, D] */
  void* v_cache;
  int32_t* status;        /* bit 0 set when a position falls outside [0, cap); may be NULL */
  int L, Hq, Hkv, D, cap, blocked;
  float rope_base;
} mtp_rope_out;
typedef struct mtp_qmv_args {
  const void* x;
  const void* x2;
  const float* ss_in;
  const void* w0;
  const void* s0;
  const void* b0;
  const void* w1;
  const void* s1;
  const void* b1;
  void* y0;
  void* y1;
  float* yf;
  const void* resid;
  float* ss_out;
  float eps;
  int M, N, K, group_size, ldx, ldy;
  int xmode, emode, packed;
  void* ws;
  size_t ws_bytes;
  const mtp_rope_out* rope; /* emode 4 only */
  int schedule;             /* must be 0 (the per-tile kernel) */
  /* xmode 3 input sums; y_sums (emode 0, 1, 3, optional): the per-32-column
   * row sums of the stored y0 values as [N/32][32] fp32, in column order -
   * the x_sums of a following xmode 3 call on y0. */
  const float* x_sums;
  float* y_sums;
} mtp_qmv_args;
int mtp_qmv_affine4_ex(const mtp_qmv_args* args, void* stream);


/* ---- 4-bit quantized matmul for 9..64 verify rows (MFMA) --------------------
 * The continuous-batched ragged verify (M = sum_b (K_b + 1) rows, up to 64):
 * each weight quad is read once and applied to all M rows on
 * v_mfma_f32_32x32x16_bf16, x streaming through LDS by 256-k quads. Weights in
 * the tile-major layout of mtp_pack_affine4 (w0; w1 = the up matrix of the
 * pair); same arithmetic as mtp_qmv_affine4_ex (dequantised weights never
 * rounded, fp32 accumulation). emode 0: y bf16 (or yf fp32 of the
 * bf16-rounded value); 1: y = bf16(bf16(x W^T) + resid) (resid may alias y);
 * 3: y = bf16(bf16(silu(bf16(x W0^T))) * bf16(x W1^T)). ldx/ldy <= 0 mean
 * K/N; x rows 16-byte aligned. ws: mtp_qmm_workspace_bytes (256-byte aligned,
 * zeroed once, then left to the library; calls sharing it stream-ordered),
 * needed when the call splits leftover column groups by K.
 * Replaces the M > 16 route of mtplx/nax_verify.py:754 (stock
 * mx.quantized_matmul) and mtplx/nax_verify.py:690 nax_qmm_m16 for the
 * batched verify lane (mtplx/batched_decode.py:338-395). */
typedef struct mtp_qmm_args {
  const void* x;
  const void* w0;
  const void* w1;
  void* y;
  float* yf;
  const void* resid;
  int M, N, K, group_size, ldx, ldy, emode;
  void* ws;
  size_t ws_bytes;
} mtp_qmm_args;
size_t mtp_qmm_workspace_bytes(int M, int N, int K, int dual);
int mtp_qmm_affine4_mfma(const mtp_qmm_args* args, void* stream);

/* ---- Ragged KV cache + attention -----------------------------------------
 * Cache layout [B, Hkv, cap, D] bf16 (mtplx/ragged_kv_cache.py:71).
 * Scatter: cache[b,h,write_start[b]+i,:] = new[b,h,i,:]
 * (RaggedBatchKVCache.update_and_fetch, mtplx/ragged_kv_cache.py:201-277).
 * Positions outside [0,cap) are skipped and flagged in *status (device int32,
 * may be NULL). */
int mtp_kv_scatter(void* k_cache, void* v_cache, const void* k_new, const void* v_new, const int32_t* write_start,
                   int B, int Hkv, int cap, int q, int D, int32_t* status, void* stream);

/* Rows with row_mask[b] != 0 take snap over positions [lo,hi) (zero past
 * snap_cap) — RaggedBatchKVCache.restore_masked, mtplx/ragged_kv_cache.py:473-496. */
int mtp_kv_restore_masked(void* cur, const void* snap, const uint8_t* row_mask, int B, int Hkv, int cap,
                          int snap_cap, int D, int lo, int hi, void* stream);

/* uint8 mask [B,1,q_len,key_len], mask[b,0,i,j] = j <= q_start[b]+i
 * (mtplx/ragged_attention.py:42 ragged_causal_mask). */
int mtp_ragged_causal_mask(uint8_t* out, const int32_t* q_start, int B, int q_len, int key_len, void* stream);

/* out = softmax(q k^T * scale, ragged causal mask) v with GQA (D = 128,
 * (Hq/Hkv)*L <= 32). q,out [B,Hq,L,D]; k,v [B,Hkv,cap,D]; q_start int32 [B]
 * on the device; q_lens int32 [B] or NULL. split_keys <= 0 picks the default.
 * Replaces the stock SDPA on the ragged lane (mtplx/attention_split.py:347 with
 * the mask of mtplx/ragged_attention.py:42) and the packed-GQA verify kernel
 * (mtplx/kernels/sdpa_gqa_packed.py:299 sdpa_gqa_packed_tail). */
size_t mtp_attn_workspace_bytes(int B, int Hkv, int cap, int split_keys);
int mtp_ragged_gqa_attn(const void* q, const void* k, const void* v, const int32_t* q_start, const int32_t* q_lens,
                        void* out, int B, int Hq, int Hkv, int L, int D, int cap, float scale, int split_keys,
                        void* ws, size_t ws_bytes, void* stream);
/* Same, out written as [B, L, Hq, D] rows (the o_proj input layout). */
int mtp_ragged_gqa_attn_rows(const void* q, const void* k, const void* v, const int32_t* q_start,
                             const int32_t* q_lens, void* out, int B, int Hq, int Hkv, int L, int D, int cap,
                             float scale, int split_keys, void* ws, size_t ws_bytes, void* stream);

/* Operand-major KV blocks, the verify step's own cache (head dim 128). Per
 * (request, kv head), 32-key blocks of 4096 bf16 in which each attention MFMA
 * operand of a wave is one 1 KB contiguous load:
 *   K[key][d] at block*4096 + ((i*2 + h2)*32 + key%32)*8 + d%8,
 *       i = (d/8)%8, h2 = d/64;
 *   V[key][d] at block*4096 + ((t*2 + jj)*64 + h2*32 + d%32)*8 + e,
 *       t = d/32, jj = (key%32)/16, r = key%16, h2 = (r%8)/4,
 *       e = r < 8 ? r%4 : 4 + r%4.
 * Same results as mtp_ragged_gqa_attn_rows / mtp_rope_qkv_to_cache on the
 * same values; cap must be a multiple of 32. No reference counterpart: the
 * reference cache (mtplx/ragged_kv_cache.py:71) is [B, Hkv, cap, D]; this is
 * the MI355X layout of the same values for the fused verify step. */
size_t mtp_attn_vt_workspace_bytes(int B, int Hkv, int cap);
int mtp_ragged_gqa_attn_rows_vt(const void* q, const void* k_blk, const void* v_blk, const int32_t* q_start,
                                const int32_t* q_lens, void* out, int B, int Hq, int Hkv, int L, int D, int cap,
                                float scale, void* ws, size_t ws_bytes, void* stream);
int mtp_rope_qkv_to_cache_vt(const void* qkv, const int32_t* q_start, const int32_t* q_lens, void* q_out,
                             void* k_cache, void* v_cache, int B, int L, int Hq, int Hkv, int D, int cap,
                             float rope_base, int32_t* status, void* stream);

/* Ragged batches over the operand-major block cache, per-request capacities:
 * the continuous-batched verify lane (mtplx/batched_decode.py:338-395,
 * mtplx/ragged_kv_cache.py:201-277 with per-row q lengths). Request b has
 * q_lens[b] query rows (<= Lmax) at positions q_start[b] + i; q is
 * [B, Hq, Lmax, D]; its output rows are packed at row_off[b] + i of out
 * [rows, Hq * D] (row_off NULL: b * Lmax + i). Its K/V live in blocks
 * [kv_off[b], kv_off[b+1]) of k_blk / v_blk (4096 bf16 per 32-key block, the
 * layout above; head h's nblk_b = (kv_off[b+1] - kv_off[b]) / Hkv blocks
 * start at kv_off[b] + h * nblk_b); kv_off NULL means a uniform capacity cap.
 * cap is the largest request capacity (a multiple of 32), total_cap the sum
 * of the capacities (<= 0: B * cap), split_keys the keys per work unit (a
 * multiple of 128). split_keys <= 0 (and B <= 256) gives balanced work
 * instead: one workgroup per CU, each taking an equal share of all the
 * batch's (request, head, 32-key tile) work up to each request's
 * q_start + q_len, whatever the lengths. (Hq/Hkv) * Lmax <= 32, D = 128. */
typedef struct mtp_attn_blocks_args {
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
} mtp_attn_blocks_args;
size_t mtp_attn_blocks_workspace_bytes(int B, int Hkv, int cap, long long total_cap, int split_keys);
int mtp_ragged_gqa_attn_blocks(const mtp_attn_blocks_args* args, void* stream);
/* RoPE on packed ragged q|k|v rows [M, (Hq+2Hkv)*D] (row m of request b with
 * row_off[b] <= m < row_off[b+1], position q_start[b] + m - row_off[b]):
 * q -> q_out [B, Hq, Lmax, D], K/V into the blocks as above (kv_off NULL:
 * uniform cap). Positions outside [0, capacity) are skipped and flag *status. */
int mtp_rope_qkv_to_blocks(const void* qkv, int M, const int32_t* row_off, const int32_t* q_start,
                           const int32_t* kv_off, void* q_out, void* k_blk, void* v_blk, int B, int Lmax, int Hq,
                           int Hkv, int D, int cap, float rope_base, int32_t* status, void* stream);

/* ---- Verify-step glue -------------------------------------------------------
 * RoPE (rotate-half, fp32 angles) on fused q|k|v rows [B*L, (Hq+2Hkv)*D] at
 * positions q_start[b]+i; q -> q_out [B,Hq,L,D], k/v written into the cache
 * (the per-row RoPE offset of tests/test_ragged_kv_cache.py:62-100 followed by
 * update_and_fetch). */
int mtp_rope_qkv_to_cache(const void* qkv, const int32_t* q_start, const int32_t* q_lens, void* q_out,
                          void* k_cache, void* v_cache, int B, int L, int Hq, int Hkv, int D, int cap,
                          float rope_base, int32_t* status, void* stream);
int mtp_rmsnorm(const void* x, const void* w, void* out, int M, int H, float eps, void* stream);
/* out[m] = dequant(w[tokens[m]]) — 4-bit quantized embedding rows [V, H/8]. */
int mtp_embed_affine4(const int32_t* tokens, const void* w, const void* scales, const void* biases, void* out,
                      int M, int H, int V, int group_size, int32_t* status, void* stream);

/* ---- Expert-sorted MoE -----------------------------------------------------
 * Routing: per token top-k of fp32 router logits[t * ld + e] (+ skew[e] when
 * skew != NULL; ld <= 0 means E) in (value desc, id asc) order, and softmax
 * weights renormalised over the k: softmax over all experts, top-k of the
 * probabilities, norm_topk_prob (mtplx/models/qwen4_exp.py:1430-1437). */
int mtp_moe_route(const float* logits, int ld, const float* skew, int T, int E, int top_k, int32_t* ids,
                  float* weights, void* stream);

/* Stable counting sort of topk_ids int32 [T, top_k] (R = T*top_k <= 8192,
 * E <= 4096): row_map = order // top_k, sorted_ids = flat[order],
 * inv_order = argsort(order), expert_off int32 [E+1], active int32 [1+E] =
 * (count, active expert ids ascending); active[0] = -1 flags an id outside
 * [0, E). Replaces mtplx/moe_sorted_gather.py:221 sort_rows. */
size_t mtp_moe_workspace_bytes(int T, int top_k, int E);
int mtp_moe_sort(const int32_t* topk_ids, int T, int top_k, int E, uint32_t* row_map, uint32_t* sorted_ids,
                 uint32_t* inv_order, int32_t* expert_off, int32_t* active, void* ws, size_t ws_bytes, void* stream);

/* Gathered 4-bit matmul over expert-sorted rows: sorted row i (expert e with
 * expert_off[e] <= i < expert_off[e+1]) computes x[row_map[i]] @ deq(W[e])^T
 * (row_map NULL: x[i]). Weights [E, rows_per_expert, K/8]; xmode 0 = x,
 * 1 = silu(x)*x2; emode 0 = store y [R, N], 3 = silu(x@W0^T)*(x@W1^T) with
 * W1 the up rows (mtplx/moe_sorted_gather.py:241 gather_qmm_rows, :288
 * swiglu_rows, :339 switch_linear; mlx gather_qmm(sorted_indices=True) at
 * :170). max_rows_per_expert bounds any expert's row count (<= T). */
int mtp_gather_qmv_affine4(const void* x, const void* x2, const uint32_t* row_map, const int32_t* expert_off,
                           const int32_t* active, const void* w0, const void* s0, const void* b0, const void* w1,
                           const void* s1, const void* b1, void* y, int max_rows_per_expert, int E, int N, int K,
                           int group_size, int xmode, int emode, int rows_per_expert, void* ws, size_t ws_bytes,
                           void* stream);

/* The same gathered matmul over the tile-major pack (mtp_pack_affine4) of
 * the [E * rows_per_expert, K] expert matrix, x plain (gathered through
 * row_map when given): emode 0 = store y [R, N], 3 = silu(x@Wg^T)*(x@Wu^T)
 * with expert e's N gate rows at e * rows_per_expert and its N up rows next.
 * Each workgroup streams several column tiles of one expert behind one
 * staging of its rows (the dense verify kernels' body); experts with at most
 * 4 rows and those with more run as two launches. N and rows_per_expert
 * multiples of 32, K of 256, group size 64 or 128. Replaces the same
 * reference calls as mtp_gather_qmv_affine4 (mtplx/moe_sorted_gather.py:241,
 * :288; mtplx/models/qwen4_exp.py:1544-1577). */
int mtp_gather_qmv_affine4_packed(const void* x, const uint32_t* row_map, const int32_t* expert_off,
                                  const int32_t* active, const void* wp, void* y, int max_rows_per_expert, int E,
                                  int N, int K, int group_size, int emode, int rows_per_expert, void* stream);

/* mtp_gather_qmv_affine4_packed for one row class of experts: row_class 1
 * runs only the experts with 1-4 rows, 2 only those with 5 or more, 0 both
 * (the call above). Each class is a launch of its own, so a caller can put
 * them on two streams and run them side by side (the 5+-row class is latency
 * bound at cfg5). Same arguments otherwise; the same rows of y are written
 * as by the call above. Replaces the same reference call sites. */
int mtp_gather_qmv_affine4_packed_rows(const void* x, const uint32_t* row_map, const int32_t* expert_off,
                                       const int32_t* active, const void* wp, void* y, int max_rows_per_expert, int E,
                                       int N, int K, int group_size, int emode, int rows_per_expert, int row_class,
                                       void* stream);

/* mtp_gather_qmv_affine4_packed_rows over the layout-2 pack
 * (mtp_pack_affine4_mf16) of the same [E * rows_per_expert, K] matrix: the
 * 16x16x32 MFMA quads, in the 4-row form for the 1-4-row class and the
 * 16-row form for 16-row tiles. Same arguments and outputs. Replaces the same
 * reference call sites (mtplx/moe_sorted_gather.py:241, :288;
 * mtplx/models/qwen4_exp.py:1544-1577). */
int mtp_gather_qmv_affine4_packed_mf16(const void* x, const uint32_t* row_map, const int32_t* expert_off,
                                       const int32_t* active, const void* wp, void* y, int max_rows_per_expert, int E,
                                       int N, int K, int group_size, int emode, int rows_per_expert, int row_class,
                                       void* stream);

/* Expert offsets int32 [E+1] and the active list [1+E] (as mtp_moe_sort
 * writes them) from ids already sorted ascending, the sorted_indices of the
 * reference entry points (mtplx/moe_sorted_gather.py:241 gather_qmm_rows,
 * :288 swiglu_rows, :339 switch_linear); active[0] = -1 flags an id outside
 * [0, E) or a descent. */
int mtp_moe_segments(const int32_t* sorted_ids, int R, int E, int32_t* expert_off, int32_t* active, void* stream);

/* The sparse block's tail (mtplx/models/qwen4_exp.py:1438-1445, unsort of
 * :1544-1577): routed = bf16(sum_j route_w[t,j] * y_sorted[inv_order[t*k+j]]);
 * sh = bf16(sigmoid(shared_gate[t * gate_ld]) * shared[t]) (shared_gate NULL:
 * shared[t]; shared NULL: no shared expert); out[t] = bf16(resid[t] +
 * bf16(routed + sh)) (resid NULL: the block output alone). resid may alias out. */
int mtp_moe_combine(const void* y_sorted, const uint32_t* inv_order, const float* route_w, const void* shared,
                    const float* shared_gate, int gate_ld, const void* resid, void* out, int T, int top_k, int H,
                    void* stream);
/* mtp_moe_combine that also writes the sums of squares of out's stored
 * values, ss_out[j * 32 + t] over 32-column block j (H % 32 == 0, T <= 32):
 * the statistics the next layer's fused input RMSNorm reads, as the dense
 * residual epilogues write them. */
int mtp_moe_combine_ss(const void* y_sorted, const uint32_t* inv_order, const float* route_w, const void* shared,
                       const float* shared_gate, int gate_ld, const void* resid, void* out, float* ss_out, int T,
                       int top_k, int H, void* stream);

/* ---- Exact speculative accept / reject ------------------------------------
 * target_logits fp32 [B*(K+1), V] (row K of each request = bonus row),
 * draft_logits fp32 [B*K, V], draft_ids int32 [B,K], uniforms fp64 [B,K+1]
 * consumed in stream order. Law: mtplx/sampling.py:131-391 (softmax with T,
 * top-k value desc/id asc, top-p over full-vocab mass, min(1,p/q), residual
 * max(p-q,0) renormalised, Generator.choice = cdf/searchsorted); loop order
 * mtplx/generation.py:15560-15790, bonus :16085-16110. temperature <= 0 is the
 * greedy lane (no uniforms). Any top_k >= 0 (0 or >= V: no top-k bound) and
 * top_p (outside (0, 1): no nucleus); supports wider than 64 ids take the
 * wide-law kernels. Penalties are applied to the logits beforehand
 * (mtp_apply_logit_deltas).
 * Outputs: out_tokens int32 [B,K+1] (committed ids, -1 padded), n_accepted
 * int32 [B], accept_probs fp64 [B,K] (-1 = not examined), status int32 [B]
 * (1 = non-finite logits: mtplx/sampling.py:32 NonFiniteLogitsError).
 * Workspace: mtp_sampler_workspace_bytes(B*(2K+1), V, top_k). */
size_t mtp_sampler_workspace_bytes(int rows, int V, int top_k);
int mtp_spec_accept(const float* target_logits, const float* draft_logits, const int32_t* draft_ids,
                    const double* uniforms, int B, int K, int V, double temperature, int top_k, double top_p,
                    int32_t* out_tokens, int32_t* n_accepted, double* accept_probs, int32_t* status, void* ws,
                    size_t ws_bytes, void* stream);


/* The same step for a ragged batch (the continuous-batched verify lane,
 * mtplx/batched_decode.py:338-395): request b has depth K_b = k_lens[b]
 * (1 <= K_b <= K_max); its target rows are target_logits rows
 * t_off[b] .. t_off[b] + K_b (n_target rows in all) and its draft rows and
 * draft ids are rows / entries d_off[b] .. d_off[b] + K_b - 1 (n_draft in
 * all); uniforms [B, K_max+1] (request b consumes at most K_b + 1); outputs
 * as above with K = K_max. A request whose rows fall outside the buffers
 * (K_b < 0 or K_b > K_max, t_off[b] + K_b >= n_target, d_off[b] + K_b >
 * n_draft, or a negative offset) is checked on the device and skipped: its
 * status is 2, its tokens and accept probabilities -1, n_accepted 0.
 * Workspace: mtp_sampler_workspace_bytes(n_target + n_draft, V, top_k). */
int mtp_spec_accept_ragged(const float* target_logits, int n_target, const float* draft_logits, int n_draft,
                           const int32_t* t_off, const int32_t* d_off, const int32_t* k_lens, const int32_t* draft_ids,
                           const double* uniforms, int B, int K_max, int V, double temperature, int top_k, double top_p,
                           int32_t* out_tokens, int32_t* n_accepted, double* accept_probs, int32_t* status, void* ws,
                           size_t ws_bytes, void* stream);

/* mtp_spec_accept without a workspace argument. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workspace is a file-scope device array of 8 MiB per GPU, kept until the
 * process ends; a call that would need more (mtp_sampler_workspace_bytes)
 * returns MTP_ERR_UNSUPPORTED. It allocates nothing. Every call on one GPU
 * shares that array: calls that overlap on a GPU race, so order them on one
 * stream. */
int mtp_spec_accept_noalloc(const float* target_logits, const float* draft_logits, const int32_t* draft_ids,
                            const double* uniforms, int B, int K, int V, double temperature, int top_k, double top_p,
                            int32_t* out_tokens, int32_t* n_accepted, double* accept_probs, int32_t* status,
                            void* stream);

/* Per-row sparse law (ids ascending, fp64 probs, count) and optionally one
 * draw per row with uniforms[r]: mtplx/sampling.py:259 distribution_from_logits
 * + :342 sample_from_distribution; mtplx/fast_sampling.py:637
 * sparse_distribution_from_mlx_logits. out_ids/out_probs are [rows, ld_out],
 * ld_out >= the support bound (1 when greedy, else min(top_k, V) or V for
 * top_k = 0); slots past a row's count hold -1 / 0. Workspace:
 * mtp_sampler_workspace_bytes(rows, V, top_k). */
int mtp_sample_rows(const float* logits, int rows, int V, double temperature, int top_k, double top_p,
                    const double* uniforms, int32_t* out_ids, double* out_probs, int ld_out, int32_t* out_count,
                    int32_t* sampled, int32_t* status, void* ws, size_t ws_bytes, void* stream);

/* Sparse additive penalties on raw logits, in place, before temperature:
 * logits[row_ids[i] * ld + token_ids[i]] += -deltas[i] in fp32, the device twin
 * mtplx/fast_sampling.py:42-81 apply_penalties_mlx of mtplx/sampling.py:212
 * apply_penalties (delta = frequency * count + presence * (count > 0), or an
 * overlay value, computed by the caller and cast to fp32). (row, token) pairs
 * must be unique within a call; an index outside [0, rows) x [0, V) sets
 * *status (may be NULL) and is skipped. */
int mtp_apply_logit_deltas(float* logits, long long ld, int rows, int V, const int32_t* row_ids,
                           const int32_t* token_ids, const float* deltas, int n, int32_t* status, void* stream);

/* Diagnostic with no counterpart in the reference: writes the 64x16 register
 * image of one v_mfma_f32_32x32x16_bf16 on a known operand pattern (tests use
 * it to pin the lane layout the kernels assume). */
int mtp_probe_mfma_layout(float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MTPLX_AMD_H */
