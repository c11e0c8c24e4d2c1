// Prefill path for E8-D4 layers with more than 16 activation rows.
//
// Batch tiles of 16 rows through the decode matvec: each tile re-streams Q.

#include "common.h"
#include "kernels.h"

namespace eptq {

int launch_gemm_e8d4(const LinearArgs& a, hipStream_t s) {
  for (int b0 = 0; b0 < a.B; b0 += kMatvecMaxBatch) {
    LinearArgs t = a;
    t.B = a.B - b0 < kMatvecMaxBatch ? a.B - b0 : kMatvecMaxBatch;
    t.x = a.x + (size_t)b0 * a.N;
    t.y = a.y + (size_t)b0 * 8 * a.M;
    const int rc = launch_matvec<KIND_E8D4>(t, s);
    if (rc) return rc;
  }
  return 0;
}

}  // namespace eptq
