// Activation producers of the engine path (kernels/norm.py), gfx950 device code.
//
// Every engine-signature linear consumes int8 activations with one fp32 scale per
// 64 columns.  Three kernels of the reference make them from 16-bit activations:
//   rmsnorm_quant     y = x * rsqrt(mean(x^2) + eps) * (w (+ 1))        norm.py:28-57
//   gate_mul_quant    y = a * sigmoid(G[gate column])                    norm.py:168-188
//   norm_gated_quant  y = bf16(x * rsqrt(mean_head(x^2) + eps) * w * silu(z))
//                                                                        norm.py:95-137
// followed by `s = max(amax / 127, 1e-8)`, `q = round_i8(y / s)` per 64 columns
// (norm.py:15-25).
//
// pro_block() computes them for a block of rows and a K range; the standalone
// producer kernels (producers.hip) and the prologue of the fused skinny launches
// (skinny_kernel.h) both call it, so a row's codes do not depend on which of them
// made it.  The arithmetic is fixed operation by operation -- float32, every
// operation rounded, no fused multiply-add (contraction is switched off in these
// functions) -- so the oracle can restate it exactly:
//   * sum of squares: 8-element chunks; lane l of a team folds chunks l, l + lanes,
//     ... in order, then an xor butterfly over the team (64 lanes for a row, hd / 8
//     lanes for a head);
//   * rsqrt(v) = 1 / sqrt(v), both correctly rounded;
//   * exp: Cody-Waite reduction and a degree-7 Taylor polynomial (pro_exp).
#pragma once

#include "qlin_dev.h"
#include "qlin_internal.h"

namespace qlin {

// exp(x) = 2^n exp(r), n = rint(x log2 e), r = (x - n ln2_hi) - n ln2_lo; exp(r) by the
// degree-7 Taylor polynomial in Horner form (|r| <= ln2 / 2: under 2 ulp).  +inf above
// 88, 0 below -87, so no result is subnormal.
__device__ __forceinline__ float pro_exp(float x) {
#pragma clang fp contract(off)
  if (x > 88.0f) return __builtin_inff();
  if (x < -87.0f) return 0.0f;
  const float n = __builtin_rintf(x * 0x1.715476p+0f);
  const float r = (x - n * 0x1.62e4p-1f) - n * 0x1.7f7d1cp-20f;
  float p = 0x1.a01a02p-13f;
  p = p * r + 0x1.6c16c2p-10f;
  p = p * r + 0x1.111112p-7f;
  p = p * r + 0x1.555556p-5f;
  p = p * r + 0x1.555556p-3f;
  p = p * r + 0x1p-1f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return __builtin_ldexpf(p, (int)n);
}

__device__ __forceinline__ float pro_sigmoid(float x) {
#pragma clang fp contract(off)
  return 1.0f / (1.0f + pro_exp(-x));
}

// 1 / sqrt(ss / n + eps), every operation correctly rounded.
__device__ __forceinline__ float pro_rms_inv(float ss, int n, float eps) {
#pragma clang fp contract(off)
  const float var = ss / (float)n;
  return 1.0f / __builtin_sqrtf(var + eps);
}

// 8 consecutive 16-bit values (bf16 or fp16) -> fp32; p + idx 16-byte aligned.
__device__ __forceinline__ void pro_ld8(const void* p, int dt, long long idx, float v[8]) {
  const u32x4 q = *(const u32x4*)((const uint16_t*)p + idx);
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    v[e] = (dt == DT_BF16) ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
  }
}

// 8 consecutive values of a norm weight (bf16, fp16 or fp32) -> fp32.
__device__ __forceinline__ void pro_ldw8(const void* p, int dt, long long idx, float v[8]) {
  if (dt == DT_F32) {
    const f32x4 a = *(const f32x4*)((const float*)p + idx);
    const f32x4 b = *(const f32x4*)((const float*)p + idx + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = a[e], v[4 + e] = b[e];
  } else {
    pro_ld8(p, dt, idx, v);
  }
}

// Sum over a team of `lanes` consecutive lanes (a power of two) by an xor butterfly:
// every lane of the team ends with the same value.
__device__ __forceinline__ float pro_team_sum(float acc, int lanes) {
#pragma clang fp contract(off)
  for (int m = lanes >> 1; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
  return acc;
}

// One lane's share of a sum of squares: chunks c0, c0 + step, ... below nc, 8 values
// each, in order.
__device__ __forceinline__ float pro_sumsq_part(const void* x, int dt, long long off, int c0, int step, int nc) {
#pragma clang fp contract(off)
  float acc = 0.0f;
  for (int c = c0; c < nc; c += step) {
    float v[8];
    pro_ld8(x, dt, off + 8LL * c, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = acc + v[e] * v[e];
  }
  return acc;
}

// int8 codes of one 64-column group held as 8 values by each lane of an aligned
// 8-lane team: s = max(amax / 127, 1e-8), q = round_i8(y / s) (kernels/norm.py:19-22).
__device__ __forceinline__ float pro_quant8(const float y[8], uint32_t& lo, uint32_t& hi) {
  float am = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(y[e]));
  am = fmaxf(am, __shfl_xor(am, 1));
  am = fmaxf(am, __shfl_xor(am, 2));
  am = fmaxf(am, __shfl_xor(am, 4));
  const float s = fmaxf(am / 127.0f, 1e-8f);
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e >> 2] |= ((uint32_t)round_i8(y[e] / s) & 0xFFu) << (8 * (e & 3));
  lo = w[0];
  hi = w[1];
  return s;
}

// Where a producer block puts its codes: an LDS block (row stride ldq bytes, scales
// [rows][ng] after it) and/or the global code and scale matrices.
struct ProOut {
  uint8_t* lq;  // LDS codes [rows][ldq bytes] for the K range [kb, ke), or nullptr
  float* ls;    // LDS scales [rows][lng]
  int ldq;
  int lng;      // (ke - kb) / 64
  bool emit;    // also write p.q / p.s
};

// One (row, 64-column group) item of an 8-lane team: the lane's 8 columns start at k.
__device__ __forceinline__ void pro_put(const ProArgs& p, const ProOut& o, int K, int row0, int r, int kb, int k,
                                        int t8, const float y[8]) {
  uint32_t lo, hi;
  const float s = pro_quant8(y, lo, hi);
  if (o.lq) {
    *(u32x2*)(o.lq + (long long)r * o.ldq + (k - kb)) = u32x2{lo, hi};
    if (t8 == 0) o.ls[r * o.lng + (k - kb) / 64] = s;
  }
  if (o.emit) {
    *(u32x2*)(p.q + (long long)(row0 + r) * K + k) = u32x2{lo, hi};
    if (t8 == 0) p.s[(long long)(row0 + r) * (K / 64) + k / 64] = s;
  }
}

// Codes and scales of rows [row0, row0 + rows) over the K range [kb, ke) (multiples of
// 64).  Called by every thread of the workgroup (it holds barriers); `lr` is LDS for
// `rows` floats.
__device__ __forceinline__ void pro_block(const ProArgs& p, int K, int row0, int rows, int kb, int ke,
                                          const ProOut& o, float* lr) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int ng = (ke - kb) >> 6;
  if (p.kind == PRO_RMSNORM || p.kind == PRO_GATE_MUL) {
    if (p.kind == PRO_RMSNORM) {
      // each row's inverse RMS over the whole row, one wave per row
      const int wave = tid >> 6, lane = tid & 63, nw = nthr >> 6;
      for (int r = wave; r < rows; r += nw) {
        const long long off = (long long)(row0 + r) * p.ldx;
        const float ss = pro_team_sum(pro_sumsq_part(p.x, p.xdt, off, lane, 64, K >> 3), 64);
        if (lane == 0) lr[r] = pro_rms_inv(ss, K, p.eps);
      }
      __syncthreads();
    }
    const int t8 = tid & 7;
    for (int it = tid >> 3; it < rows * ng; it += nthr >> 3) {
      const int r = it / ng;
      const int k = kb + (it - r * ng) * 64 + 8 * t8;
      float x[8], y[8];
      if (p.kind == PRO_RMSNORM) {
        float w[8];
        pro_ld8(p.x, p.xdt, (long long)(row0 + r) * p.ldx + k, x);
        pro_ldw8(p.w, p.wdt, k, w);
        const float ri = lr[r];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float we = p.one_plus ? w[e] + 1.0f : w[e];
          y[e] = (x[e] * ri) * we;
        }
      } else {
        // gates of head h sit at [h * 2 hd + hd, (h + 1) * 2 hd) of the gate row
        float gv[8];
        pro_ld8(p.x, p.xdt, (long long)(row0 + r) * p.ldx + k, x);
        const long long gc = (long long)(k / p.hd) * (2 * p.hd) + p.hd + (k % p.hd);
        pro_ld8(p.g, p.xdt, (long long)(row0 + r) * p.ldg + gc, gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = x[e] * pro_sigmoid(gv[e]);
      }
      pro_put(p, o, K, row0, r, kb, k, t8, y);
    }
  } else {
    // PRO_NORM_GATED: teams of hd / 8 lanes, one (row, head) each; a head's groups are
    // written where they fall inside [kb, ke)
    const int T = p.hd >> 3;
    const int tl = tid & (T - 1);
    const int h0 = kb / p.hd, h1 = (ke + p.hd - 1) / p.hd;
    const int nh = h1 - h0;
    for (int it = tid / T; it < rows * nh; it += nthr / T) {
      const int r = it / nh;
      const int h = h0 + (it - r * nh);
      const long long off = (long long)(row0 + r) * K + (long long)h * p.hd;
      float x[8], zv[8], w[8], y[8];
      pro_ld8(p.x, p.xdt, off + 8 * tl, x);
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = acc + x[e] * x[e];
      const float ri = pro_rms_inv(pro_team_sum(acc, T), p.hd, p.eps);
      pro_ld8(p.g, p.xdt, (long long)(row0 + r) * p.ldg + (long long)h * p.hd + 8 * tl, zv);
      pro_ldw8(p.w, p.wdt, 8 * tl, w);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float sz = zv[e] * pro_sigmoid(zv[e]);
        y[e] = bf16_to_f32(f32_to_bf16(((x[e] * ri) * w[e]) * sz));
      }
      const int k = h * p.hd + 8 * tl;
      // every lane of the team takes part in the 8-lane amax; only columns inside the
      // range are stored
      uint32_t lo, hi;
      const float s = pro_quant8(y, lo, hi);
      if (k >= kb && k < ke) {
        if (o.lq) {
          *(u32x2*)(o.lq + (long long)r * o.ldq + (k - kb)) = u32x2{lo, hi};
          if ((tl & 7) == 0) o.ls[r * o.lng + (k - kb) / 64] = s;
        }
        if (o.emit) {
          *(u32x2*)(p.q + (long long)(row0 + r) * K + k) = u32x2{lo, hi};
          if ((tl & 7) == 0) p.s[(long long)(row0 + r) * (K / 64) + k / 64] = s;
        }
      }
    }
  }
  __syncthreads();
}

}  // namespace qlin
