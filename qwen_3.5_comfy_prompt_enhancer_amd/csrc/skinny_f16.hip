// Instantiations of the skinny kernel for fp16 activations (the A16 decode core).
#include "skinny_kernel.h"

namespace qlin {

hipError_t launch_skinny_f16(const SkLaunch& L, const SkArgs& a, hipStream_t st) {
  QL_CASE(ACT_F16, WK_W8, false, EPI_STORE, 8, true, KS_ANY)
  QL_CASE(ACT_F16, WK_W8, false, EPI_STORE, 16, false, KS_ANY)
  QL_CASE(ACT_F16, WK_W4, false, EPI_STORE, 8, false, KS_STEP4)
  QL_CASE(ACT_F16, WK_W4, false, EPI_STORE, 16, false, KS_STEP4)
  QL_CASE(ACT_F16, WK_W4, true, EPI_STORE, 8, false, KS_STEP4)
  QL_CASE(ACT_F16, WK_W4, true, EPI_STORE, 16, false, KS_STEP4)
  QL_CASE(ACT_F16, WK_W4, false, EPI_STORE, 8, false, KS_ANY)
  QL_CASE(ACT_F16, WK_W4, false, EPI_STORE, 16, false, KS_ANY)
  QL_CASE(ACT_F16, WK_W4, true, EPI_STORE, 8, false, KS_ANY)
  QL_CASE(ACT_F16, WK_W4, true, EPI_STORE, 16, false, KS_ANY)
  // one-pass 64-column tiles
  QL_CASE(ACT_F16, WK_W8, false, EPI_STORE, 4, false, KS_ANY)
  QL_CASE(ACT_F16, WK_W4, false, EPI_STORE, 4, false, KS_STEP4)
  QL_CASE(ACT_F16, WK_W4, true, EPI_STORE, 4, false, KS_STEP4)
  QL_CASE(ACT_F16, WK_W4, false, EPI_STORE, 4, false, KS_ANY)
  QL_CASE(ACT_F16, WK_W4, true, EPI_STORE, 4, false, KS_ANY)
  return hipErrorInvalidValue;
}

}  // namespace qlin
