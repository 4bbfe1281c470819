// Engine-signature calls outside the fast kernels' layout rules, gfx950: any N and
// pointers aligned only to their element size (the fast kernels need N % 16 == 0 and
// 16-byte aligned rows).  The reference's kernels mask every edge (kernels/gemm.py:50-57,
// kernels/w4.py:75-104), so a caller may hand it a weight of 4000 columns or a view
// into a larger tensor; this kernel takes those calls.
//
// One wave per (row, 64 output columns), one column per lane; every element read with
// a load of its own size, so no alignment beyond the element is assumed.  Arithmetic
// per output (the fast kernels' per-block fold, one K split, blocks in increasing K):
//   W8: acc = fma(float(dot_b), a_s[b], acc) over 64-wide blocks b, dot_b exact in int32;
//   W4: acc = fma(float(dot), a_s * w_s, acc) over sub-blocks of min(group, 64), dot of
//       the codes with (nibble - z) exact in int32 (kernels/w4.py:75-104);
// then the fast kernels' epilogues: y = fma(acc, column scale, residual) (W4: scale 1)
// stored as bf16 / fp16; or h = silu(g) * u, stored as bf16 or requantized per 64
// columns (kernels/gemm.py:195-211).  A row's result does not depend on M, so rows of
// a batch equal single-row calls and chunked prompts equal unchunked ones.
#include <algorithm>

#include "qlin_dev.h"
#include "qlin_internal.h"

namespace qlin {

namespace {

template <int WK>
__global__ __launch_bounds__(64) void edge_kernel(const EdgeArgs a) {
  const int lane = (int)threadIdx.x;
  const int c = (int)blockIdx.x * 64 + lane;
  const bool valid = c < a.ncols;
  const int cc = valid ? c : a.ncols - 1;  // lanes past the last column compute a valid one and store nothing
  const bool gate_up = a.epi != EPI_STORE;
  // the column's weight set(s): gate/up use seg[0] and seg[1] for the same column
  int si = 0;
  if (!gate_up)
    for (int i = 1; i < a.nseg; ++i) si = cc >= a.seg[i].col0 ? i : si;
  const int nsets = gate_up ? 2 : 1;
  const int nb = a.K / 64;
  const int sub = (WK == WK_W4 && a.group < 64) ? a.group : 64;
  for (int m = (int)blockIdx.y; m < a.M; m += (int)gridDim.y) {
    const int8_t* xr = a.x + (long long)m * a.K;
    const float* xsr = a.xs + (long long)m * nb;
    float acc[2] = {0.0f, 0.0f};
    for (int k0 = 0; k0 < a.K; k0 += sub) {
      const float as = xsr[k0 >> 6];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (t >= nsets) break;
        const Seg& S = a.seg[gate_up ? t : si];
        const int n = S.n;
        const int cl = cc - S.col0;
        int dot = 0;
        if constexpr (WK == WK_W8) {
          const int8_t* w = (const int8_t*)S.w + (long long)k0 * n + cl;
          for (int k = 0; k < sub; ++k) dot += (int)xr[k0 + k] * (int)w[(long long)k * n];
          acc[t] = fmaf((float)dot, as, acc[t]);
        } else {
          const long long gi = (long long)(k0 / a.group) * n + cl;
          const int z = S.z ? (int)S.z[gi] : 8;
          const uint8_t* w = S.w + (long long)(k0 >> 1) * n + cl;
          for (int k = 0; k < sub; k += 2) {
            const int b = w[(long long)(k >> 1) * n];
            dot += (int)xr[k0 + k] * ((b & 15) - z) + (int)xr[k0 + k + 1] * ((b >> 4) - z);
          }
          acc[t] = fmaf((float)dot, as * load_scale(S.s, a.sdt, gi), acc[t]);
        }
      }
    }
    float cs[2] = {1.0f, 1.0f};
    if constexpr (WK == WK_W8) {
      for (int t = 0; t < nsets; ++t) {
        const Seg& S = a.seg[gate_up ? t : si];
        cs[t] = load_scale(S.s, a.sdt, cc - S.col0);
      }
    }
    if (!gate_up) {
      float y = acc[0] * cs[0];
      if (a.res) y = fmaf(acc[0], cs[0], load_act16(a.res, a.odt, (long long)m * a.ldr + cc));
      if (valid) ((uint16_t*)a.out)[(long long)m * a.ldo + c] = to_out16(y, a.odt);
    } else {
      float h = silu(acc[0] * cs[0]) * (acc[1] * cs[1]);
      if (a.epi == EPI_GATEUP) {
        if (valid) ((uint16_t*)a.out)[(long long)m * a.ldo + c] = f32_to_bf16(h);
      } else {
        // the bf16 round trip, then the group's amax over the wave (64 columns)
        h = bf16_to_f32(f32_to_bf16(h));
        float am = valid ? fabsf(h) : 0.0f;
#pragma unroll
        for (int s = 1; s < 64; s <<= 1) am = fmaxf(am, __shfl_xor(am, s));
        const float sc = fmaxf(am / 127.0f, 1e-8f);
        if (valid) a.oq[(long long)m * a.ncols + c] = (int8_t)round_i8(h / sc);
        if (lane == 0) a.os[(long long)m * (a.ncols / 64) + blockIdx.x] = sc;
      }
    }
  }
}

}  // namespace

hipError_t launch_edge(const EdgeArgs& a, int wk, hipStream_t st) {
  if (a.M <= 0 || a.ncols <= 0) return hipSuccess;
  const dim3 grid((unsigned)((a.ncols + 63) / 64), (unsigned)std::min(a.M, 65535));
  if (wk == WK_W8) hipLaunchKernelGGL(edge_kernel<WK_W8>, grid, dim3(64), 0, st, a);
  else hipLaunchKernelGGL(edge_kernel<WK_W4>, grid, dim3(64), 0, st, a);
  return hipGetLastError();
}

}  // namespace qlin
