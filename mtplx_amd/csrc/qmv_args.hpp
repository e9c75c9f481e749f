// Argument blocks of the streaming-matmul C ABI (the same layout as
// include/mtplx_amd.h), read by qmv.hip.
#pragma once

#include "qmv_common.hpp"

struct mtp_rope_out {
  const int32_t* q_start;
  const int32_t* q_lens;
  void* q_out;
  void* k_cache;
  void* v_cache;
  int32_t* status;
  int L, Hq, Hkv, D, cap, blocked;
  float rope_base;
};

struct mtp_qmv_args {
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
  const mtp_rope_out* rope;
  int schedule;
  const float* x_sums;
  float* y_sums;
};

namespace mtp {
// Argument block -> kernel parameters (mode ranges checked; the rest by qmm_check).
int qmv_args_params(const mtp_qmv_args* a, QmmParams* out, const char* who);
int qmm_check_args(int xm, int em, const QmmParams& p, const char* who);
size_t stream_lds_bytes(int chunk_q, int M, int nw);
}  // namespace mtp

// mtp_qmm_affine4_mfma's argument block (the same layout as include/mtplx_amd.h).
struct mtp_qmm_args {
  const void* x;
  const void* w0;
  const void* w1;
  void* y;
  float* yf;
  const void* resid;
  int M, N, K, group_size, ldx, ldy, emode;
  void* ws;
  size_t ws_bytes;
};
