// Layout kernels.  W4 unpack and W4 / W8 dequantization to fp32 expose the exact
// integer / fp32 values the GEMM kernels consume, so the unpack and dequant can be
// checked bit for bit (quant_formats.py:6-9, kernels/w4.py:51-61, 103-104).  The
// load-time producers of the packed layouts, symmetric W4 per (group, column) and
// W8 per column (quant_formats.py:253-275), requantize fp32 weights on the GPU with
// the same arithmetic: fp32 amax, clamp at 1e-8, one correctly rounded division for
// the scale and one per weight, round half to even.
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

// ---------------------------------------------------------------------------
// Requantization (quant_formats.py:253-275).  Byte and fp32 element work, bound
// by HBM: every weight is read from HBM once (the second pass of a column's group
// or of the per-column quantization hits the caches) and its code written once.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t code_w4(float w, float sc) {
  return (uint32_t)(int)(fminf(fmaxf(rintf(w / sc), -8.0f), 7.0f) + 8.0f);
}

// W4, 4 columns per thread (N % 4 == 0): 16-byte loads, one 4-byte store per row pair.
__global__ void requant_w4_x4_kernel(const float* __restrict__ w, int K, int N, int group,
                                     uint8_t* __restrict__ packed, uint16_t* __restrict__ sbf) {
  const int n = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
  const int gi = blockIdx.y;
  if (n >= N) return;
  const float* col = w + (long long)gi * group * N + n;
  f32x4 amax = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < group; ++r) {
    const f32x4 v = *(const f32x4*)(col + (long long)r * N);
#pragma unroll
    for (int c = 0; c < 4; ++c) amax[c] = fmaxf(amax[c], fabsf(v[c]));
  }
  float sc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) sc[c] = fmaxf(amax[c], 1e-8f) / 7.0f;
  uint8_t* prow = packed + (long long)gi * (group / 2) * N + n;
  for (int r = 0; r < group; r += 2) {
    const f32x4 v0 = *(const f32x4*)(col + (long long)r * N);
    const f32x4 v1 = *(const f32x4*)(col + (long long)(r + 1) * N);
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) word |= (code_w4(v0[c], sc[c]) | (code_w4(v1[c], sc[c]) << 4)) << (8 * c);
    *(uint32_t*)(prow + (long long)(r / 2) * N) = word;
  }
  *(u32x2*)(sbf + (long long)gi * N + n) =
      u32x2{(uint32_t)f32_to_bf16(sc[0]) | ((uint32_t)f32_to_bf16(sc[1]) << 16),
            (uint32_t)f32_to_bf16(sc[2]) | ((uint32_t)f32_to_bf16(sc[3]) << 16)};
}

// W4: thread = (group g, column n).  sc = max(amax, 1e-8) / 7 over the group's rows;
// code = clamp(rint(w / sc), -8, 7) + 8; even K in the low nibble (quant_formats.py:
// 223-229, 246-250); the scale is stored as bf16 (round to nearest even).
__global__ void requant_w4_kernel(const float* __restrict__ w, int K, int N, int group,
                                  uint8_t* __restrict__ packed, uint16_t* __restrict__ sbf) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int gi = blockIdx.y;
  if (n >= N) return;
  const float* col = w + (long long)gi * group * N + n;
  float amax = 0.0f;
  for (int r = 0; r < group; ++r) amax = fmaxf(amax, fabsf(col[(long long)r * N]));
  const float sc = fmaxf(amax, 1e-8f) / 7.0f;
  uint8_t* prow = packed + (long long)gi * (group / 2) * N + n;
  for (int r = 0; r < group; r += 2) {
    const float q0 = fminf(fmaxf(rintf(col[(long long)r * N] / sc), -8.0f), 7.0f) + 8.0f;
    const float q1 = fminf(fmaxf(rintf(col[(long long)(r + 1) * N] / sc), -8.0f), 7.0f) + 8.0f;
    prow[(long long)(r / 2) * N] = (uint8_t)((int)q0 | ((int)q1 << 4));
  }
  sbf[(long long)gi * N + n] = f32_to_bf16(sc);
}

// W8, pass 1: the bits of max |w| over a block of rows of each column, merged with an
// unsigned atomic max (the order of non-negative floats is that of their bits) into
// `bits`, which starts at zero.
__global__ void w8_amax_kernel(const float* __restrict__ w, int K, int N, int rows, unsigned* __restrict__ bits) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int r0 = blockIdx.y * rows, r1 = min(K, r0 + rows);
  float amax = 0.0f;
  for (int r = r0; r < r1; ++r) amax = fmaxf(amax, fabsf(w[(long long)r * N + n]));
  atomicMax(bits + n, bitcast<unsigned>(amax));
}

// the same, 4 columns per thread (N % 4 == 0)
__global__ void w8_amax_x4_kernel(const float* __restrict__ w, int K, int N, int rows, unsigned* __restrict__ bits) {
  const int n = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
  if (n >= N) return;
  const int r0 = blockIdx.y * rows, r1 = min(K, r0 + rows);
  f32x4 amax = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int r = r0; r < r1; ++r) {
    const f32x4 v = *(const f32x4*)(w + (long long)r * N + n);
#pragma unroll
    for (int c = 0; c < 4; ++c) amax[c] = fmaxf(amax[c], fabsf(v[c]));
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) atomicMax(bits + n + c, bitcast<unsigned>(amax[c]));
}

__global__ void fill_u32_kernel(unsigned* __restrict__ p, int n, unsigned v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// W8, pass 2: code = clamp(rint(w / sc), -127, 127) with sc = max(amax, 1e-8) / 127.
__global__ void w8_quant_kernel(const float* __restrict__ w, int K, int N, const unsigned* __restrict__ bits,
                                int8_t* __restrict__ q) {
  const long long total = (long long)K * N;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const int n = (int)(i % N);
    const float sc = fmaxf(bitcast<float>(bits[n]), 1e-8f) / 127.0f;
    q[i] = (int8_t)(int)fminf(fmaxf(rintf(w[i] / sc), -127.0f), 127.0f);
  }
}

__device__ __forceinline__ uint32_t code_w8(float w, float sc) {
  return (uint32_t)(int)fminf(fmaxf(rintf(w / sc), -127.0f), 127.0f) & 0xFFu;
}

// the same, 4 consecutive elements per thread (N % 4 == 0, so they share a row)
__global__ void w8_quant_x4_kernel(const float* __restrict__ w, int K, int N, const unsigned* __restrict__ bits,
                                   int8_t* __restrict__ q) {
  const long long total4 = (long long)K * N / 4;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total4;
       i += (long long)gridDim.x * blockDim.x) {
    const int n = (int)((4 * i) % N);
    const f32x4 v = *(const f32x4*)(w + 4 * i);
    const u32x4 b = *(const u32x4*)(bits + n);
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) word |= code_w8(v[c], fmaxf(bitcast<float>(b[c]), 1e-8f) / 127.0f) << (8 * c);
    *(uint32_t*)(q + 4 * i) = word;
  }
}

// W8, pass 3: the amax bits become the fp32 scale, in place.
__global__ void w8_scale_kernel(int N, unsigned* __restrict__ bits) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n < N) bits[n] = bitcast<unsigned>(fmaxf(bitcast<float>(bits[n]), 1e-8f) / 127.0f);
}

// ---------------------------------------------------------------------------
// External int4 formats -> the engine layout (quant_formats.py:199-229, 355-466).
// GPTQ packs 8 K-nibbles of one column per int32 word (nibble j = bits 4j..4j+3 =
// row 8w + j), so the engine's pair bytes (even K low, odd K high) are the word's
// little-endian bytes: packed[4w + t][n] = byte t of qweight[w][n].  AWQ packs 8
// N-nibbles of one row per word in the order [0, 2, 4, 6, 1, 3, 5, 7]; column 8c + j
// sits at nibble kAwqRev[j] = [0, 4, 1, 5, 2, 6, 3, 7][j] of word c.
// ---------------------------------------------------------------------------

__constant__ int kAwqRev[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// thread = (word row w, column n): one word in, its 4 bytes to 4 packed rows
__global__ void repack_gptq_kernel(const uint32_t* __restrict__ qw, int K, int N, uint8_t* __restrict__ packed) {
  const long long total = (long long)(K / 8) * N;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long w = i / N, n = i - w * N;
    const uint32_t v = qw[i];
#pragma unroll
    for (int t = 0; t < 4; ++t) packed[(4 * w + t) * N + n] = (uint8_t)(v >> (8 * t));
  }
}

// 4 columns per thread (N % 4 == 0): one 16-byte load, a 4x4 byte transpose, four
// 4-byte stores (row 4w + t gets byte t of the four words)
__global__ void repack_gptq_x4_kernel(const uint32_t* __restrict__ qw, int K, int N, uint8_t* __restrict__ packed) {
  const long long total4 = (long long)(K / 8) * N / 4;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total4;
       i += (long long)gridDim.x * blockDim.x) {
    const long long e = 4 * i, w = e / N, n = e - w * N;
    const u32x4 v = *(const u32x4*)(qw + e);
    uint32_t t4[4];
    tr4(v.x, v.y, v.z, v.w, t4);
#pragma unroll
    for (int t = 0; t < 4; ++t) *(uint32_t*)(packed + (4 * w + t) * N + n) = t4[t];
  }
}

// thread = (packed row r, word c): rows 2r and 2r+1 of word column c -> 8 pair bytes
__global__ void repack_awq_kernel(const uint32_t* __restrict__ qw, int K, int N, uint8_t* __restrict__ packed) {
  const int W = N / 8;
  const long long total = (long long)(K / 2) * W;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long r = i / W, c = i - r * W;
    const uint32_t lo = qw[(2 * r) * W + c], hi = qw[(2 * r + 1) * W + c];
    uint32_t b[2] = {0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int sh = 4 * kAwqRev[j];
      const uint32_t byte = ((lo >> sh) & 0xFu) | (((hi >> sh) & 0xFu) << 4);
      b[j >> 2] |= byte << (8 * (j & 3));
    }
    *(u32x2*)(packed + r * N + 8 * c) = u32x2{b[0], b[1]};
  }
}

// z[g][8c + j] = nibble (awq ? kAwqRev[j] : j) of qzeros[g][c], plus `add`
// compressed-tensors int4 (quant_formats.py:282-354): weight_packed int32 [N][W], 8
// straight-order K nibbles per word, one output feature per row.  Byte i of word w
// holds nibbles k = 8w + 2i (low) and 8w + 2i + 1 (high): exactly the engine's pair
// byte of packed row 4w + i, column n.  So the engine layout [K/2][N] is the byte
// transpose of the [N][4W] byte view, cut to K/2 rows.  A 64 x 64 byte tile goes
// through LDS: loaded as dwords along a source row, stored 16 bytes along N.
__global__ void repack_ct_kernel(const uint32_t* __restrict__ qw, int N, int W, int KB,
                                 uint8_t* __restrict__ packed) {
  __shared__ uint8_t t[64][64 + 4];  // [column n - n0][packed row j - j0]
  const int n0 = blockIdx.x * 64, j0 = blockIdx.y * 64;
  const int tid = threadIdx.x;
  {
    const int r = tid >> 2, c = (tid & 3) * 16;  // source row n0 + r, bytes j0 + c ...
    const int n = n0 + r;
    if (n < N) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int j = j0 + c + 4 * q;  // first byte of the word
        if (j < KB) {
          const uint32_t v = qw[(long long)n * W + (j >> 2)];
#pragma unroll
          for (int b = 0; b < 4; ++b) t[r][c + 4 * q + b] = (uint8_t)(v >> (8 * b));
        }
      }
    }
  }
  __syncthreads();
  const int jr = tid >> 2, c = (tid & 3) * 16;  // packed row j0 + jr, columns n0 + c ...
  const int j = j0 + jr, n = n0 + c;
  if (j < KB && n < N) {  // N % 16 == 0: the 16 columns are all in range
    uint32_t w4[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      w4[q] = (uint32_t)t[c + 4 * q][jr] | ((uint32_t)t[c + 4 * q + 1][jr] << 8) |
              ((uint32_t)t[c + 4 * q + 2][jr] << 16) | ((uint32_t)t[c + 4 * q + 3][jr] << 24);
    *(u32x4*)(packed + (long long)j * N + n) = u32x4{w4[0], w4[1], w4[2], w4[3]};
  }
}

__global__ void zeros_unpack_kernel(const uint32_t* __restrict__ qz, int G, int N, int awq, int add,
                                    uint8_t* __restrict__ z) {
  const long long total = (long long)G * N;
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < total;
       i += (long long)gridDim.x * blockDim.x) {
    const long long g = i / N;
    const int n = (int)(i - g * N), c = n >> 3, j = n & 7;
    const int pos = awq ? kAwqRev[j] : j;
    z[i] = (uint8_t)(((qz[g * (N / 8) + c] >> (4 * pos)) & 0xFu) + (uint32_t)add);
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

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

hipError_t launch_requant_w4(const float* w, int K, int N, int group, uint8_t* packed, uint16_t* sbf,
                             hipStream_t st) {
  if (N % 4 == 0 && aligned16(w) && aligned16(packed) && aligned16(sbf))
    hipLaunchKernelGGL(requant_w4_x4_kernel, dim3((unsigned)((N / 4 + 255) / 256), (unsigned)(K / group)), dim3(256),
                       0, st, w, K, N, group, packed, sbf);
  else
    hipLaunchKernelGGL(requant_w4_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)(K / group)), dim3(256), 0,
                       st, w, K, N, group, packed, sbf);
  return hipGetLastError();
}

hipError_t launch_requant_w8(const float* w, int K, int N, int8_t* q, float* scale, hipStream_t st) {
  unsigned* bits = (unsigned*)scale;  // amax bits first, the scale at the end
  const unsigned cb = (unsigned)((N + 255) / 256);
  constexpr int kRows = 64;  // rows per amax block: enough blocks to fill the chip
  hipLaunchKernelGGL(fill_u32_kernel, dim3(cb), dim3(256), 0, st, bits, N, 0u);
  if (N % 4 == 0 && aligned16(w) && aligned16(q) && aligned16(scale)) {
    hipLaunchKernelGGL(w8_amax_x4_kernel, dim3((unsigned)((N / 4 + 255) / 256), (unsigned)((K + kRows - 1) / kRows)),
                       dim3(256), 0, st, w, K, N, kRows, bits);
    hipLaunchKernelGGL(w8_quant_x4_kernel, grid_for((long long)K * N / 4), dim3(256), 0, st, w, K, N, bits, q);
  } else {
    hipLaunchKernelGGL(w8_amax_kernel, dim3(cb, (unsigned)((K + kRows - 1) / kRows)), dim3(256), 0, st, w, K, N,
                       kRows, bits);
    hipLaunchKernelGGL(w8_quant_kernel, grid_for((long long)K * N), dim3(256), 0, st, w, K, N, bits, q);
  }
  hipLaunchKernelGGL(w8_scale_kernel, dim3(cb), dim3(256), 0, st, N, bits);
  return hipGetLastError();
}

hipError_t launch_repack_gptq(const int32_t* qw, int K, int N, uint8_t* packed, hipStream_t st) {
  if (N % 4 == 0 && aligned16(qw) && aligned16(packed))
    hipLaunchKernelGGL(repack_gptq_x4_kernel, grid_for((long long)(K / 8) * N / 4), dim3(256), 0, st,
                       (const uint32_t*)qw, K, N, packed);
  else
    hipLaunchKernelGGL(repack_gptq_kernel, grid_for((long long)(K / 8) * N), dim3(256), 0, st, (const uint32_t*)qw,
                       K, N, packed);
  return hipGetLastError();
}

hipError_t launch_repack_awq(const int32_t* qw, int K, int N, uint8_t* packed, hipStream_t st) {
  hipLaunchKernelGGL(repack_awq_kernel, grid_for((long long)(K / 2) * (N / 8)), dim3(256), 0, st,
                     (const uint32_t*)qw, K, N, packed);
  return hipGetLastError();
}

hipError_t launch_repack_ct(const int32_t* qw, int N, int W, int K, uint8_t* packed, hipStream_t st) {
  const int KB = K / 2;
  hipLaunchKernelGGL(repack_ct_kernel, dim3((unsigned)((N + 63) / 64), (unsigned)((KB + 63) / 64)), dim3(256), 0, st,
                     (const uint32_t*)qw, N, W, KB, packed);
  return hipGetLastError();
}

hipError_t launch_zeros_unpack(const int32_t* qz, int G, int N, int awq, int add, uint8_t* z, hipStream_t st) {
  hipLaunchKernelGGL(zeros_unpack_kernel, grid_for((long long)G * N), dim3(256), 0, st, (const uint32_t*)qz, G, N,
                     awq, add, z);
  return hipGetLastError();
}

}  // namespace qlin
