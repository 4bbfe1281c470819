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

// Sum over a team of `lanes` consecutive lanes (a power of two) by an xor butterfly:
// every lane of the team ends with the same value.
__device__ __forceinline__ float pro_team_sum(float acc, int lanes) {
#pragma clang fp contract(off)
  for (int m = lanes >> 1; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
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
  float* ls;    // LDS scales: row r, 64-column group b of the range at ls[r * lng + b * lsb]
  int ldq;
  int lng;      // row stride of ls ((ke - kb) / 64 for a [rows][groups] block)
  int lsb;      // group stride of ls (1 for a [rows][groups] block)
  bool emit;    // also write p.q / p.s
};

// Loads of the producer's 16-bit inputs: plain, or (COH) device-coherent buffer loads
// for inputs that an earlier part of the same launch may have written (the decode
// chain), which plain loads could read stale from another XCD's L2.
// The thread index; under COH (inside the decode chain's persistent loop) as a value
// the compiler cannot hoist out of the loop, so what derives from it is not kept live
// across the loop.
template <bool COH>
__device__ __forceinline__ int pro_tid() {
  int t = (int)threadIdx.x;
  if constexpr (COH) asm volatile("" : "+v"(t));
  return t;
}

template <bool COH>
__device__ __forceinline__ u32x4 pro_ld(const void* p, long long idx16) {
  if constexpr (COH) {
    return __builtin_amdgcn_raw_buffer_load_b128(part_rsrc(p, 0x7FFFFFF0u), (unsigned)(idx16 * 2), 0, kCpolSc1);
  } else {
    return *(const u32x4*)((const uint16_t*)p + idx16);
  }
}

// The global copies of the codes (emit): device-coherent stores under COH, so a later
// part of the same launch may read them.
template <bool COH>
__device__ __forceinline__ void pro_emit(const ProArgs& p, int K, int row, int k, uint32_t lo, uint32_t hi,
                                         bool scale, float s) {
  if constexpr (COH) {
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{lo, hi}, part_rsrc(p.q, 0x7FFFFFF0u),
                                          (unsigned)((long long)row * K + k), 0, kCpolSc1);
    if (scale)
      __builtin_amdgcn_raw_buffer_store_b32(bitcast<uint32_t>(s), part_rsrc(p.s, 0x7FFFFFF0u),
                                            (unsigned)(((long long)row * (K / 64) + k / 64) * 4), 0, kCpolSc1);
  } else {
    *(u32x2*)(p.q + (long long)row * K + k) = u32x2{lo, hi};
    if (scale) p.s[(long long)row * (K / 64) + k / 64] = s;
  }
}

// One (row, 64-column group) item of an 8-lane team: the lane's 8 columns start at k.
template <bool COH>
__device__ __forceinline__ void pro_put(const ProArgs& p, const ProOut& o, int K, int row0, int r, int kb, int k,
                                        int t8, const float y[8]) {
  uint32_t lo, hi;
  const float s = pro_quant8(y, lo, hi);
  if (o.lq) {
    *(u32x2*)(o.lq + (long long)r * o.ldq + (k - kb)) = u32x2{lo, hi};
    if (t8 == 0) o.ls[r * o.lng + ((k - kb) / 64) * o.lsb] = s;
  }
  if (o.emit) pro_emit<COH>(p, K, row0 + r, k, lo, hi, t8 == 0, s);
}

// Chunks of a row's sum of squares a lane loads ahead (K <= 64 * 8 * kProSumPre);
// longer rows load the rest when they are summed.
constexpr int kProSumPre = 8;

// The loads of a producer block that go out before the linear's first weight loads.
// A wave's memory loads complete in issue order, so loads issued after the weights
// would wait for them: issued first, they return while the weights stream in.
// PRE: chunks prefetched (any count gives the same sums: a lane folds its chunks in
// increasing order either way); fewer hold fewer registers while weights stream.
template <int PRE>
struct ProPreN {
  u32x4 xs[PRE];         // rmsnorm: this lane's first chunks of its wave's first row
  u32x4 x, g;            // the thread's first item: 8 activations, 8 gates / z values
  u32x4 w0, w1;          // and 8 norm-weight values (w1: the second half of fp32 ones)
};
using ProPre = ProPreN<kProSumPre>;

__device__ __forceinline__ u32x4 pro_raw(const void* p, long long idx16) {
  return *(const u32x4*)((const uint16_t*)p + idx16);
}

__device__ __forceinline__ void pro_cvt8(u32x4 q, int dt, float v[8]) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    v[e] = (dt == DT_BF16) ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
  }
}

// Raw norm-weight values k .. k+7 (16-bit: one vector; fp32: two).
__device__ __forceinline__ void pro_raw_w(const void* p, int dt, long long k, u32x4& w0, u32x4& w1) {
  if (dt == DT_F32) {
    w0 = *(const u32x4*)((const float*)p + k);
    w1 = *(const u32x4*)((const float*)p + k + 4);
  } else {
    w0 = pro_raw(p, k);
    w1 = w0;
  }
}

__device__ __forceinline__ void pro_cvt_w(u32x4 w0, u32x4 w1, int dt, float v[8]) {
  if (dt == DT_F32) {
    const uint32_t a[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = bitcast<float>(a[e]);
  } else {
    pro_cvt8(w0, dt, v);
  }
}

// Geometry of a producer block: rows [row0, row0 + rows), K range [kb, ke) (multiples
// of 64).  rmsnorm / gate_mul items are (row, 64-column group) for 8-lane teams;
// norm_gated items are (row, head) for teams of hd / 8 lanes.
struct ProGeo {
  int row0, rows, kb, ke;
  int ng;      // 64-column groups of the range
  int T;       // norm_gated: team size; 8 otherwise
  int h0, nh;  // norm_gated: heads overlapping the range
};

__device__ __forceinline__ ProGeo pro_geo(const ProArgs& p, int row0, int rows, int kb, int ke) {
  ProGeo g;
  g.row0 = row0;
  g.rows = rows;
  g.kb = kb;
  g.ke = ke;
  g.ng = (ke - kb) >> 6;
  g.T = (p.kind == PRO_NORM_GATED) ? (p.hd >> 3) : 8;
  g.h0 = (p.kind == PRO_NORM_GATED) ? kb / p.hd : 0;
  g.nh = (p.kind == PRO_NORM_GATED) ? (ke + p.hd - 1) / p.hd - g.h0 : 0;
  return g;
}

// Issues the block's first loads (every thread: its wave's first row for rmsnorm's
// sum of squares, its first item).  Branch-free: every load goes out, from clamped
// in-bounds addresses, and pro_block uses only the applicable ones (a load whose
// result is merged at a control-flow join is waited for at the join, which would
// hold the weight loads behind it).
template <bool COH = false, int PRE = kProSumPre>
__device__ __forceinline__ void pro_issue(const ProArgs& p, int K, const ProGeo& G, ProPreN<PRE>& pp) {
  const int tid = pro_tid<COH>();
  const int wave = tid >> 6, lane = tid & 63;
  const bool ng_kind = p.kind == PRO_NORM_GATED;
  // rmsnorm's chunks (other kinds read the same in-bounds addresses and ignore them)
  const long long soff = (long long)(G.row0 + min(wave, G.rows - 1)) * p.ldx;
  const int nc = K >> 3;
#pragma unroll
  for (int i = 0; i < PRE; ++i) pp.xs[i] = pro_ld<COH>(p.x, soff + 8LL * min(lane + 64 * i, nc - 1));
  // the first item
  long long xi, gi, wi;
  if (ng_kind) {
    const int tl = tid & (G.T - 1);
    const int it = min(tid / G.T, G.rows * G.nh - 1);
    const int r = it / G.nh, h = G.h0 + (it - r * G.nh);
    xi = (long long)(G.row0 + r) * K + (long long)h * p.hd + 8 * tl;
    gi = (long long)(G.row0 + r) * p.ldg + (long long)h * p.hd + 8 * tl;
    wi = 8 * tl;
  } else {
    const int it = min(tid >> 3, G.rows * G.ng - 1);
    const int r = it / G.ng;
    const int k = G.kb + (it - r * G.ng) * 64 + 8 * (tid & 7);
    xi = (long long)(G.row0 + r) * p.ldx + k;
    gi = (long long)(G.row0 + r) * p.ldg + (long long)(k / max(p.hd, 1)) * (2 * p.hd) + p.hd + (k % max(p.hd, 1));
    wi = k;
  }
  // kinds without gates or norm weight read fixed addresses of x instead (distinct from
  // the item's own, so the compiler cannot turn them into copies behind a branch)
  const bool has_g = p.kind != PRO_RMSNORM, has_w = p.kind != PRO_GATE_MUL;
  pp.x = pro_ld<COH>(p.x, xi);
  pp.g = pro_ld<COH>(has_g ? p.g : p.x, has_g ? gi : 0);
  const bool f32w = has_w && p.wdt == DT_F32;
  const uint8_t* wb = has_w ? (const uint8_t*)p.w + wi * (f32w ? 4 : 2) : (const uint8_t*)p.x + 16;
  pp.w0 = *(const u32x4*)wb;
  pp.w1 = *(const u32x4*)(wb + (f32w ? 16 : 0));
}

// Codes and scales of the block (pro_issue's loads first, then the rest), into LDS
// and / or the global code matrices.  Called by every thread of the workgroup (it
// holds barriers); `lr` is LDS for `rows` floats.
template <bool COH = false, int PRE = kProSumPre>
__device__ __forceinline__ void pro_block(const ProArgs& p, int K, const ProGeo& G, const ProPreN<PRE>& pp,
                                          const ProOut& o, float* lr) {
#pragma clang fp contract(off)
  const int tid = pro_tid<COH>();
  const int nthr = blockDim.x;
  const int rows = G.rows, row0 = G.row0, kb = G.kb, ke = G.ke, ng = G.ng;
  if (p.kind == PRO_RMSNORM || p.kind == PRO_GATE_MUL) {
    if (p.kind == PRO_RMSNORM) {
      // each row's inverse RMS over the whole row, one wave per row; the chunks of a
      // lane are folded in order: the prefetched ones, then the rest
      const int wave = tid >> 6, lane = tid & 63, nw = nthr >> 6;
      const int nc = K >> 3;
      for (int r = wave; r < rows; r += nw) {
        const long long off = (long long)(row0 + r) * p.ldx;
        float acc = 0.0f;
        int c0 = lane;
        if (r == wave) {
#pragma unroll
          for (int i = 0; i < PRE; ++i) {
            if (lane + 64 * i < nc) {
              float v[8];
              pro_cvt8(pp.xs[i], p.xdt, v);
#pragma unroll
              for (int e = 0; e < 8; ++e) acc = acc + v[e] * v[e];
            }
          }
          c0 = lane + 64 * PRE;
        }
        for (int c = c0; c < nc; c += 64) {
          float v[8];
          pro_cvt8(pro_ld<COH>(p.x, off + 8LL * c), p.xdt, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc = acc + v[e] * v[e];
        }
        const float ss = pro_team_sum(acc, 64);
        if (lane == 0) lr[r] = pro_rms_inv(ss, K, p.eps);
      }
      __syncthreads();
    }
    const int t8 = tid & 7;
    for (int it = tid >> 3; it < rows * ng; it += nthr >> 3) {
      const int r = it / ng;
      const int k = kb + (it - r * ng) * 64 + 8 * t8;
      const bool first = it == (tid >> 3);
      float x[8], y[8];
      pro_cvt8(first ? pp.x : pro_ld<COH>(p.x, (long long)(row0 + r) * p.ldx + k), p.xdt, x);
      if (p.kind == PRO_RMSNORM) {
        float w[8];
        u32x4 w0 = pp.w0, w1 = pp.w1;
        if (!first) pro_raw_w(p.w, p.wdt, k, w0, w1);
        pro_cvt_w(w0, w1, p.wdt, w);
        const float ri = lr[r];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float we = p.one_plus ? w[e] + 1.0f : w[e];
          y[e] = (x[e] * ri) * we;
        }
      } else {
        // gates of head h sit at [h * 2 hd + hd, (h + 1) * 2 hd) of the gate row
        float gv[8];
        const long long gc = (long long)(k / p.hd) * (2 * p.hd) + p.hd + (k % p.hd);
        pro_cvt8(first ? pp.g : pro_ld<COH>(p.g, (long long)(row0 + r) * p.ldg + gc), p.xdt, gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = x[e] * pro_sigmoid(gv[e]);
      }
      pro_put<COH>(p, o, K, row0, r, kb, k, t8, y);
    }
  } else {
    // PRO_NORM_GATED: teams of hd / 8 lanes, one (row, head) each; a head's groups are
    // written where they fall inside [kb, ke)
    const int T = G.T;
    const int tl = tid & (T - 1);
    const int nh = G.nh;
    for (int it = tid / T; it < rows * nh; it += nthr / T) {
      const int r = it / nh;
      const int h = G.h0 + (it - r * nh);
      const bool first = it == tid / T;
      const long long off = (long long)(row0 + r) * K + (long long)h * p.hd;
      float x[8], zv[8], w[8], y[8];
      pro_cvt8(first ? pp.x : pro_ld<COH>(p.x, off + 8 * tl), p.xdt, x);
      float acc = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = acc + x[e] * x[e];
      const float ri = pro_rms_inv(pro_team_sum(acc, T), p.hd, p.eps);
      pro_cvt8(first ? pp.g : pro_ld<COH>(p.g, (long long)(row0 + r) * p.ldg + (long long)h * p.hd + 8 * tl),
               p.xdt, zv);
      pro_cvt_w(pp.w0, pp.w1, p.wdt, w);  // the same 8 weights for every head
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
          if ((tl & 7) == 0) o.ls[r * o.lng + ((k - kb) / 64) * o.lsb] = s;
        }
        if (o.emit) pro_emit<COH>(p, K, row0 + r, k, lo, hi, (tl & 7) == 0, s);
      }
    }
  }
  __syncthreads();
}

}  // namespace qlin
