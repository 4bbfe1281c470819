// Instantiations of the skinny kernel with the fused activation-producer prologue, W4
// weights of groups of 64 or more (kernels/norm.py feeding kernels/w4.py).
#include "skinny_kernel.h"

namespace qlin {

hipError_t launch_skinny_pro_w4(const SkLaunch& L, const SkArgs& a, hipStream_t st) {
  QL_CASE_PRO(WK_W4, false, EPI_STORE, 8, false)
  QL_CASE_PRO(WK_W4, true, EPI_STORE, 8, false)
  QL_CASE_PRO(WK_W4, false, EPI_STORE, 4, false)
  QL_CASE_PRO(WK_W4, true, EPI_STORE, 4, false)
  QL_CASE_PRO(WK_W4, false, EPI_GATEUP_Q, 8, false)
  QL_CASE_PRO(WK_W4, true, EPI_GATEUP_Q, 8, false)
  QL_CASE_PRO(WK_W4, false, EPI_GATEUP_Q, 4, false)
  QL_CASE_PRO(WK_W4, true, EPI_GATEUP_Q, 4, false)
  return hipErrorInvalidValue;
}

}  // namespace qlin
