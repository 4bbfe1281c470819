// Standalone activation-producer launches (kernels/norm.py:28-57, 95-137, 168-188):
// 16-bit activations -> int8 codes [M][K] + fp32 scales [M][K/64] in global memory.
// They serve the reference-signature rmsnorm_quant / gate_mul_quant /
// norm_gated_quant, and the fused calls whose plan has no room for a prologue (wide
// launches, the tiled prefill kernel).  The arithmetic is producers.h's pro_block,
// the same the fused prologue runs.
#include "producers.h"

namespace qlin {

namespace {

constexpr int kProThreads = 256;

// One workgroup per row.
__global__ __launch_bounds__(kProThreads) void producer_kernel(const ProArgs p, int K) {
  __shared__ float lr[1];
  ProOut o;
  o.lq = nullptr;
  o.ls = nullptr;
  o.ldq = 0;
  o.lng = 0;
  o.lsb = 1;
  o.emit = true;
  const ProGeo G = pro_geo(p, blockIdx.x, 1, 0, K);
  ProPre pp;
  pro_issue(p, K, G, pp);
  pro_block(p, K, G, pp, o, lr);
}

__global__ void pro_exp_kernel(const float* x, float* y, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = pro_exp(x[i]);
}

}  // namespace

hipError_t launch_producer(const ProArgs& p, int M, int K, hipStream_t st) {
  if (M <= 0) return hipSuccess;
  hipLaunchKernelGGL(producer_kernel, dim3((unsigned)M), dim3(kProThreads), 0, st, p, K);
  return hipGetLastError();
}

hipError_t launch_pro_exp(const float* x, float* y, int n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(pro_exp_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, n);
  return hipGetLastError();
}

}  // namespace qlin
