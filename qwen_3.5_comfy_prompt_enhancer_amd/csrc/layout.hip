// Element-wise layout kernels: W4 unpack and W4 / W8 dequantization to fp32.
// They expose the exact integer / fp32 values the GEMM kernels consume so the
// unpack and dequant can be checked bit for bit (quant_formats.py:6-9,
// kernels/w4.py:51-61, 103-104).
#include "qlin_dev.h"
#include "qlin_internal.h"

namespace qlin {

// nib[k][n] = nibble k of column n: byte (k/2, n), low nibble for even k.
__global__ void w4_unpack_kernel(const uint8_t* __restrict__ p, int K, int N, uint8_t* __restrict__ out) {
  const long long total = (long long)(K / 2) * N;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long jrow = i / N, col = i - jrow * N;
    const uint8_t b = p[i];
    out[(2 * jrow) * N + col] = b & 0x0F;
    out[(2 * jrow + 1) * N + col] = b >> 4;
  }
}

// out[k][n] = (nibble - z) * scale[k/group][n] in fp32; z = 8 when zeros are absent.
__global__ void w4_dequant_kernel(const uint8_t* __restrict__ p, const void* s, int sdt,
                                  const uint8_t* __restrict__ z, int group, int K, int N,
                                  float* __restrict__ out) {
  const long long total = (long long)(K / 2) * N;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long jrow = i / N, col = i - jrow * N;
    const uint8_t b = p[i];
    const long long k0 = 2 * jrow;
    const long long g0 = (k0 / group) * N + col, g1 = ((k0 + 1) / group) * N + col;
    const int z0 = z ? (int)z[g0] : 8, z1 = z ? (int)z[g1] : 8;
    out[k0 * N + col] = (float)((int)(b & 0x0F) - z0) * load_scale(s, sdt, g0);
    out[(k0 + 1) * N + col] = (float)((int)(b >> 4) - z1) * load_scale(s, sdt, g1);
  }
}

// out[k][n] = w[k][n] * scale[n] in fp32.
__global__ void w8_dequant_kernel(const int8_t* __restrict__ w, const void* s, int sdt, int K, int N,
                                  float* __restrict__ out) {
  const long long total = (long long)K * N;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long col = i % N;
    out[i] = (float)w[i] * load_scale(s, sdt, col);
  }
}

static dim3 grid_for(long long total) {
  long long blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return dim3((unsigned)blocks);
}

hipError_t launch_w4_unpack(const uint8_t* p, int K, int N, uint8_t* out, hipStream_t st) {
  hipLaunchKernelGGL(w4_unpack_kernel, grid_for((long long)(K / 2) * N), dim3(256), 0, st, p, K, N, out);
  return hipGetLastError();
}

hipError_t launch_w4_dequant(const uint8_t* p, const void* s, int sdt, const uint8_t* z, int group, int K,
                             int N, float* out, hipStream_t st) {
  hipLaunchKernelGGL(w4_dequant_kernel, grid_for((long long)(K / 2) * N), dim3(256), 0, st, p, s, sdt, z,
                     group, K, N, out);
  return hipGetLastError();
}

hipError_t launch_w8_dequant(const int8_t* w, const void* s, int sdt, int K, int N, float* out,
                             hipStream_t st) {
  hipLaunchKernelGGL(w8_dequant_kernel, grid_for((long long)K * N), dim3(256), 0, st, w, s, sdt, K, N, out);
  return hipGetLastError();
}

}  // namespace qlin
