// q|k|v projection variants with the RoPE + K/V-write epilogue (their own
// translation unit; kernels in qmv_kernels.hpp).
#include "qmv_kernels.hpp"

namespace mtp {

void qmv_launch_rope_qkv(int xm, const QmmParams& p, const Plan& pl, hipStream_t st) {
  if (xm == X_RMSNORM)
    launch_rope<X_RMSNORM>(p, pl, st);
  else
    launch_rope<X_PLAIN>(p, pl, st);
}

}  // namespace mtp
