// Shared definitions for the gfx950 verify-path kernels and their C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#define MTP_API extern "C" __attribute__((visibility("default")))

// Error codes returned by every entry point (0 = ok).
enum {
  MTP_OK = 0,
  MTP_ERR_ARG = -1,          // bad shape / pointer / size argument
  MTP_ERR_UNSUPPORTED = -2,  // valid but not implemented (e.g. group_size 32)
  MTP_ERR_WORKSPACE = -3,    // workspace too small
  MTP_ERR_HIP = -4,          // a HIP runtime call failed
};

namespace mtp {

// Thread-local message for mtp_last_error().
void set_error(const char* fmt, ...);

// Compute units of the current device (cached per device).
int device_cus();

inline int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return MTP_ERR_HIP;
  }
  return MTP_OK;
}

// Launch-status check used after every kernel launch.
inline int launch_check(const char* what) {
  return hip_check(hipGetLastError(), what);
}

typedef uint16_t bf16_t;  // raw bfloat16 bits at the ABI

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// float -> bf16 bits, round to nearest even (gfx950's v_cvt_pk_bf16_f32;
// NaN stays NaN).
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Two floats -> packed bf16 pair (lo in bits 0..15), one conversion.
__device__ __forceinline__ uint32_t f2bf2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

__host__ __device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

// Rotate-half RoPE of the pair (d, d + D/2) at position pos, fp32 angle
// theta = pos * 2^(-(2d/D) * log2(base)); outputs rounded to bf16. Shared by
// the standalone RoPE kernel and the fused q|k|v matmul epilogue so both
// round identically.
// The products and sums below use explicitly rounded operations, so no
// kernel's contraction choices change them: every writer and epilogue (and
// the precomputed angle table) produce the same bits for the same inputs.
__device__ __forceinline__ void rope_angle(int pos, int d, int D, float log2_base, float& sn, float& cs) {
  const float inv_freq = exp2f(__fmul_rn(-((float)(2 * d) / (float)D), log2_base));
  const float theta = __fmul_rn((float)pos, inv_freq);
  sincosf(theta, &sn, &cs);
}
__device__ __forceinline__ void rope_apply(float x1, float x2, float sn, float cs, uint16_t& o1, uint16_t& o2) {
  o1 = f2bf(__fmaf_rn(x1, cs, -__fmul_rn(x2, sn)));
  o2 = f2bf(__fmaf_rn(x1, sn, __fmul_rn(x2, cs)));
}
__device__ __forceinline__ void rope_pair(float x1, float x2, int pos, int d, int D, float log2_base, uint16_t& o1,
                                          uint16_t& o2) {
  float sn, cs;
  rope_angle(pos, d, D, log2_base, sn, cs);
  rope_apply(x1, x2, sn, cs, o1, o2);
}

// MFMA operand-major KV cache layout (the verify step's own cache, head dim
// 128): per (request, kv head), 32-key blocks of 4096 elements in which every
// attention MFMA operand of a wave is 64 lanes x 16 contiguous bytes.
//   K block: operand i (0..7) of lane (key kk, half h2) = d 64 h2 + 8 i .. +7,
//            at ((i*2 + h2)*32 + kk)*8.
//   V block: operand (t, jj) of lane (d = 32t + c, half h2) = keys
//            16 jj + {4h2 + e (e<4), 8 + 4h2 + e-4 (e>=4)}, at
//            ((t*2 + jj)*64 + h2*32 + c)*8 + e.
__host__ __device__ __forceinline__ size_t kblk_index(int key, int d) {
  const int c = d >> 3, i = c & 7, h2 = c >> 3;
  return (size_t)(key >> 5) * 4096 + ((size_t)(i * 2 + h2) * 32 + (key & 31)) * 8 + (d & 7);
}
__host__ __device__ __forceinline__ size_t vblk_index(int key, int d) {
  const int kk = key & 31, jj = kk >> 4, r = kk & 15;
  const int h2 = (r & 7) >> 2, e = (r < 8) ? (r & 3) : 4 + (r & 3);
  const int t = d >> 5, c = d & 31;
  return (size_t)(key >> 5) * 4096 + ((size_t)(t * 2 + jj) * 64 + h2 * 32 + c) * 8 + e;
}

// 16-byte load of data read once per launch (the attention's K/V blocks):
// the non-temporal hint keeps the stream from displacing reused lines in the
// caches (cfg2 attention 97-99 us against 107-110 us with plain loads). The
// matmuls' weight quads use plain loads: non-temporal ones fetched ~6% more
// bytes there for no gain in time.
typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const void* p) {
  const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Global stores of kernel outputs. WT: device-coherent stores (written
// through to memory, no fence needed), for outputs that another XCD reads
// later in the same kernel.
template <bool WT>
__device__ __forceinline__ void st_u16(uint16_t* a, uint16_t v) {
  if constexpr (WT)
    __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *a = v;
}
template <bool WT>
__device__ __forceinline__ void st_f32(float* a, float v) {
  if constexpr (WT)
    __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *a = v;
}

}  // namespace mtp
