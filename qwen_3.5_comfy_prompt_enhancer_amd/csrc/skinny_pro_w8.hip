// Instantiations of the skinny kernel with the fused activation-producer prologue,
// int8 weights (rmsnorm_quant + proj3 / mlp_gate_up_quant / gemm_i8, gate_mul_quant +
// gemm_i8, norm_gated_quant + gemm_i8: kernels/norm.py feeding kernels/gemm.py).
#include "skinny_kernel.h"

namespace qlin {

hipError_t launch_skinny_pro_w8(const SkLaunch& L, const SkArgs& a, hipStream_t st) {
  QL_CASE_PRO(WK_W8, false, EPI_STORE, 8, true)
  QL_CASE_PRO(WK_W8, false, EPI_STORE, 4, false)
  QL_CASE_PRO(WK_W8, false, EPI_GATEUP_Q, 8, false)
  QL_CASE_PRO(WK_W8, false, EPI_GATEUP_Q, 4, false)
  return hipErrorInvalidValue;
}

}  // namespace qlin
