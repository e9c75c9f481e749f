// Streaming quantized matmul variants for x mode X_SWIGLU (one translation
// unit per x mode so they compile in parallel; kernels in qmv_kernels.hpp).
#include "qmv_kernels.hpp"

namespace mtp {

void qmv_launch_swiglu(int em, int gsh, const QmmParams& p, const Plan& pl, hipStream_t st) {
  if (gsh)
    launch_e<X_SWIGLU, 1>(em, p, pl, st);
  else
    launch_e<X_SWIGLU, 0>(em, p, pl, st);
}

}  // namespace mtp
