// Instantiations of the skinny kernel for int8 activations and int8 weights (engine
// signature: gemm_i8, proj3, mlp_gate_up(_quant)).
#include "skinny_kernel.h"

namespace qlin {

hipError_t launch_skinny_i8w8(const SkLaunch& L, const SkArgs& a, hipStream_t st) {
  QL_CASE(ACT_I8, WK_W8, false, EPI_STORE, 8, true, KS_STEP2)
  QL_CASE(ACT_I8, WK_W8, false, EPI_STORE, 16, false, KS_STEP2)
  QL_CASE(ACT_I8, WK_W8, false, EPI_GATEUP, 8, false, KS_STEP2)
  QL_CASE(ACT_I8, WK_W8, false, EPI_GATEUP_Q, 8, false, KS_STEP2)
  // one-pass 64-column tiles
  QL_CASE(ACT_I8, WK_W8, false, EPI_STORE, 4, false, KS_STEP2)
  QL_CASE(ACT_I8, WK_W8, false, EPI_GATEUP, 4, false, KS_STEP2)
  QL_CASE(ACT_I8, WK_W8, false, EPI_GATEUP_Q, 4, false, KS_STEP2)
  return hipErrorInvalidValue;
}

}  // namespace qlin
