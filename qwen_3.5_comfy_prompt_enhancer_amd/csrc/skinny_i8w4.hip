// Instantiations of the skinny kernel for int8 activations and W4 weights (engine
// signature: gemm_w4, proj3_w4, mlp_gate_up(_quant)_w4).
#include "skinny_kernel.h"

namespace qlin {

#define QL_I8W4(KSV)                                             \
  QL_CASE(ACT_I8, WK_W4, false, EPI_STORE, 8, false, KSV)        \
  QL_CASE(ACT_I8, WK_W4, false, EPI_STORE, 16, false, KSV)       \
  QL_CASE(ACT_I8, WK_W4, true, EPI_STORE, 8, false, KSV)         \
  QL_CASE(ACT_I8, WK_W4, true, EPI_STORE, 16, false, KSV)        \
  QL_CASE(ACT_I8, WK_W4, false, EPI_GATEUP, 8, false, KSV)       \
  QL_CASE(ACT_I8, WK_W4, true, EPI_GATEUP, 8, false, KSV)        \
  QL_CASE(ACT_I8, WK_W4, false, EPI_GATEUP_Q, 8, false, KSV)     \
  QL_CASE(ACT_I8, WK_W4, true, EPI_GATEUP_Q, 8, false, KSV)     \
  QL_CASE(ACT_I8, WK_W4, false, EPI_STORE, 4, false, KSV)        \
  QL_CASE(ACT_I8, WK_W4, true, EPI_STORE, 4, false, KSV)         \
  QL_CASE(ACT_I8, WK_W4, false, EPI_GATEUP, 4, false, KSV)       \
  QL_CASE(ACT_I8, WK_W4, true, EPI_GATEUP, 4, false, KSV)        \
  QL_CASE(ACT_I8, WK_W4, false, EPI_GATEUP_Q, 4, false, KSV)     \
  QL_CASE(ACT_I8, WK_W4, true, EPI_GATEUP_Q, 4, false, KSV)

hipError_t launch_skinny_i8w4(const SkLaunch& L, const SkArgs& a, hipStream_t st) {
  QL_I8W4(KS_STEP2)
  QL_I8W4(KS_ANY)
  return hipErrorInvalidValue;
}

}  // namespace qlin
