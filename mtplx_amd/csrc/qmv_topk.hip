// lm_head variants with the sampler's chunk partials fused into the epilogue
// (E_STORE_TOPK; their own translation unit, kernels in qmv_kernels.hpp).
#include "qmv_kernels.hpp"

namespace mtp {

// The grid streams the tiles as the E_STORE kernel would (as many
// workgroups as stay resident, at most 1024 so that 64 sets of at most 16
// cover it); the LDS adds the workgroup's stored logits (tiles per
// workgroup x 32 per row) and, when the staged-x area is too small, the
// merge staging. Returns the number of records per row (sets), or -1.
template <typename Kern>
static int launch_topk_kernel(Kern kern, int nt, QmmParams q, Plan pl, hipStream_t st) {
  const int cus = device_cus();
  const size_t base = pl.lds;
  const size_t stage = (size_t)pl.nw * kTopkStageKeys * sizeof(uint64_t);
  const bool extra_stage = xa_bytes(4 * pl.chunk, q.M) < stage;
  int grid = q.n_blocks < 1024 ? q.n_blocks : 1024;
  for (int it = 0; it < 3; ++it) {   // LDS depends on tiles per workgroup, occupancy on LDS
    const int tpw = cdiv(q.n_blocks, grid);
    pl.lds = base + (size_t)q.M * tpw * 32 * sizeof(float) + (extra_stage ? stage : 0);
    if (pl.lds > 65536) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  (int)pl.lds);
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, nt, pl.lds) != hipSuccess || occ < 1) occ = 1;
    const int resident = occ * cus;
    if (grid <= resident) break;
    grid = resident;
  }
  const int tpw = cdiv(q.n_blocks, grid);
  if (tpw > 32) return -1;   // a workgroup's record holds at most 1024 ids
  q.topk_tpw = tpw;
  q.topk_wpg = cdiv(grid, kTopkParts);
  pl.lds = base + (size_t)q.M * tpw * 32 * sizeof(float) + (extra_stage ? stage : 0);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(nt), pl.lds, st, q);
  return cdiv(grid, q.topk_wpg);
}

template <int XM>
static int launch_topk_x(const QmmParams& q, const Plan& pl, hipStream_t st) {
  if (q.packed == 2) {
    const bool sh = mf_short_ring(q, pl.nw, E_STORE_TOPK);
    if (pl.nw == 8)
      return sh ? launch_topk_kernel(qmv_stream_kernel<8, 4, XM, E_STORE_TOPK, 0, true, true, 1>, 512, q, pl, st)
                : launch_topk_kernel(qmv_stream_kernel<8, 4, XM, E_STORE_TOPK, 0, true, true, 2>, 512, q, pl, st);
    return sh ? launch_topk_kernel(qmv_stream_kernel<4, 4, XM, E_STORE_TOPK, 0, true, true, 1>, 256, q, pl, st)
              : launch_topk_kernel(qmv_stream_kernel<4, 4, XM, E_STORE_TOPK, 0, true, true, 2>, 256, q, pl, st);
  }
  if (pl.nw == 8) return launch_topk_kernel(qmv_stream_kernel<8, 4, XM, E_STORE_TOPK, 0, true>, 512, q, pl, st);
  return launch_topk_kernel(qmv_stream_kernel<4, 4, XM, E_STORE_TOPK, 0, true>, 256, q, pl, st);
}

int qmv_launch_topk(int xm, const QmmParams& p, const Plan& pl, hipStream_t st) {
  return xm == X_RMSNORM ? launch_topk_x<X_RMSNORM>(p, pl, st) : launch_topk_x<X_PLAIN>(p, pl, st);
}

}  // namespace mtp
