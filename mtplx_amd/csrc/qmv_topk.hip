// lm_head variants with the sampler's chunk partials fused into the epilogue
// (E_STORE_TOPK; their own translation unit, kernels in qmv_kernels.hpp).
#include "qmv_kernels.hpp"

namespace mtp {

template <int XM>
static void launch_topk_x(const QmmParams& q, const Plan& pl, hipStream_t st) {
  // One workgroup per group of consecutive tiles: the group count is the
  // scratch's record count, so the grid is exactly that.
  const int grid = cdiv(q.n_blocks, q.topk_tpw);
  auto go = [&](auto kern, int nt) {
    // A failure here surfaces as a launch error, which the caller checks.
    if (pl.lds > 65536) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  (int)pl.lds);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(nt), pl.lds, st, q);
  };
  if (q.packed == 2) {
    const bool sh = mf_short_ring(q, pl.nw, E_STORE_TOPK);
    if (pl.nw == 8) {
      if (sh)
        go(qmv_stream_kernel<8, 4, XM, E_STORE_TOPK, 0, true, true, 1>, 512);
      else
        go(qmv_stream_kernel<8, 4, XM, E_STORE_TOPK, 0, true, true, 2>, 512);
    } else {
      if (sh)
        go(qmv_stream_kernel<4, 4, XM, E_STORE_TOPK, 0, true, true, 1>, 256);
      else
        go(qmv_stream_kernel<4, 4, XM, E_STORE_TOPK, 0, true, true, 2>, 256);
    }
  } else if (pl.nw == 8) {
    go(qmv_stream_kernel<8, 4, XM, E_STORE_TOPK, 0, true>, 512);
  } else {
    go(qmv_stream_kernel<4, 4, XM, E_STORE_TOPK, 0, true>, 256);
  }
}

void qmv_launch_topk(int xm, const QmmParams& p, const Plan& pl, hipStream_t st) {
  if (xm == X_RMSNORM)
    launch_topk_x<X_RMSNORM>(p, pl, st);
  else
    launch_topk_x<X_PLAIN>(p, pl, st);
}

}  // namespace mtp
