// Skinny quantized GEMM for up to 16 activation rows per row tile (decode, best-of-N
// rows), gfx950: the kernel template and its launchers.  The instantiations are
// spread over skinny_f16.hip, skinny_i8w8.hip and skinny_i8w4.hip, which compile in
// parallel; skinny.hip routes a launch to them.
//
// Replaces the decode-shaped launches of gemm_i8 / gemm_w4 / proj3(_w4) /
// mlp_gate_up(_quant)(_w4) (kernels/gemm.py:20-312, kernels/w4.py:107-323).
//
// Work decomposition
//   * A wave owns a column tile of TN = 16*COLS output columns and a K range.  Lane
//     l = (g = l/16, j = l%16) loads, per 32-wide K step, COLS adjacent columns
//     (one 8- or 16-byte load per weight row) of the 8 K rows 8g..8g+7 (W8), or of
//     the 4 packed byte rows 4g..4g+3 (W4).  16 lanes x COLS bytes is a coalesced
//     run along N, the engine layout's contiguous axis.
//   * In registers the lane turns those rows into COLS MFMA B operands -- column
//     t of its COLS columns for instruction t -- by byte permutes (qlin_dev.h), and
//     issues COLS 16x16x32 MFMAs against the same A operand (activation rows
//     0..15 of the row tile, the lane's 8 K values).  MFMA row i = activation row;
//     MFMA column j = column j*COLS + t of the tile.  Rows >= M are zero.
//   * fp16 activations: v_mfma_f32_16x16x32_f16 on exactly converted weights, fp32
//     accumulation; W4 nibbles enter the MFMA with a constant offset that is
//     removed per group, where the group scales are applied in fp32.
//     int8 activations (engine signature): v_mfma_i32_16x16x32_i8, exact int32 per
//     64-wide activation group (W4 per weight sub-block), then the reference's fp32
//     epilogue `acc += float(i32) * a_s (* w_s)` (kernels/gemm.py:43-45,
//     kernels/w4.py:103-104).
//   * The K dimension is split over the `waves` of a workgroup (reduced in LDS in a
//     fixed order) and over `splits` workgroups (fp32 partials in the caller's
//     workspace, written and read as agent-scope atomics; the last workgroup to
//     arrive at a per-tile counter sums them in split order and resets the counter).
//     Split choices depend on K and N only, so each output row is computed
//     identically for every M <= 16.
//   * Every load of a 32-wide K step is issued D steps ahead from a register ring.
#pragma once

#include <algorithm>
#include <type_traits>

#include "producers.h"
#include "qlin_dev.h"
#include "qlin_internal.h"

namespace qlin {

template <int COLS>
struct Row {
  uint32_t d[COLS / 4];
};

// Weight rows, loaded non-temporally where that measured faster: W8 rows of 8 or 16
// columns (decode plans read each byte once; the 16-row prefill tiles of 8 columns lost
// nothing) and the wide W4 plan (16 columns, decode only).  W4 rows of 4 or 8 columns
// (decode and 16-row tiles: 5-14 % slower non-temporal), the 4-column W8 tiles (the
// 512-row o-projection's 16-row tiles: slower) and the zeros keep plain loads.
template <int COLS, bool NT>
__device__ __forceinline__ Row<COLS> ld_row(const uint8_t* p, bool valid) {
  Row<COLS> r;
  if constexpr (COLS == 16) {
    const u32x4 v = NT ? ld_global_nt<u32x4>(p) : ld_global<u32x4>(p);
    r.d[0] = valid ? v.x : 0u;
    r.d[1] = valid ? v.y : 0u;
    r.d[2] = valid ? v.z : 0u;
    r.d[3] = valid ? v.w : 0u;
  } else if constexpr (COLS == 8) {
    const u32x2 v = NT ? ld_global_nt<u32x2>(p) : ld_global<u32x2>(p);
    r.d[0] = valid ? v.x : 0u;
    r.d[1] = valid ? v.y : 0u;
  } else {
    const uint32_t v = NT ? ld_global_nt<uint32_t>(p) : ld_global<uint32_t>(p);
    r.d[0] = valid ? v : 0u;
  }
  return r;
}

__device__ __forceinline__ uint32_t byte_of(uint32_t d, int b) { return (d >> (8 * b)) & 0xFFu; }

// Raw dwords of COLS consecutive scale values (COLS/4 vectors for fp32, COLS/8 for
// 16-bit types, half a vector for 4 columns of 16-bit values); the conversion is
// deferred to cvt_scales so the load latency is not waited on where it is issued.
// The dtype branch is loop-invariant where this is used in a K loop.
template <int COLS>
__device__ __forceinline__ void ld_scales_raw(const void* p, int dt, long long idx, u32x4 raw[COLS / 4]) {
  if (dt == DT_F32) {
    const u32x4* q = (const u32x4*)((const float*)p + idx);
#pragma unroll
    for (int c = 0; c < COLS / 4; ++c) raw[c] = q[c];
  } else if constexpr (COLS == 4) {
    const u32x2 v = *(const u32x2*)((const uint16_t*)p + idx);
    raw[0] = u32x4{v.x, v.y, 0u, 0u};
  } else {
    const u32x4* q = (const u32x4*)((const uint16_t*)p + idx);
#pragma unroll
    for (int c = 0; c < COLS / 8; ++c) raw[c] = q[c];
  }
}

// The same without a branch, for loads issued ahead of a control-flow join: every
// dtype issues the fp32 count of loads (16-bit types re-read their last vector), so
// the compiler need not copy the results at the join and wait for them there.
template <int COLS>
__device__ __forceinline__ void ld_scales_raw_nb(const void* p, int dt, long long idx, u32x4 raw[COLS / 4]) {
  const bool f32 = dt == DT_F32;
  const uint8_t* base = (const uint8_t*)p + idx * (f32 ? 4 : 2);
  if constexpr (COLS == 4) {
    const u32x2 v0 = ld_global<u32x2>(base);
    const u32x2 v1 = ld_global<u32x2>(base + (f32 ? 8 : 0));
    raw[0] = u32x4{v0.x, v0.y, v1.x, v1.y};
  } else {
    const int last16 = COLS / 8 - 1;  // last vector of 16-bit scales
#pragma unroll
    for (int c = 0; c < COLS / 4; ++c) raw[c] = ld_global<u32x4>(base + 16 * (f32 ? c : min(c, last16)));
  }
}

template <int COLS>
__device__ __forceinline__ void cvt_scales(const u32x4 raw[COLS / 4], int dt, float out[COLS]) {
  if (dt == DT_F32) {
#pragma unroll
    for (int c = 0; c < COLS / 4; ++c) {
      out[4 * c] = bitcast<float>(raw[c].x);
      out[4 * c + 1] = bitcast<float>(raw[c].y);
      out[4 * c + 2] = bitcast<float>(raw[c].z);
      out[4 * c + 3] = bitcast<float>(raw[c].w);
    }
  } else if constexpr (COLS == 4) {
    const uint32_t w[2] = {raw[0].x, raw[0].y};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
      out[e] = (dt == DT_BF16) ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
    }
  } else {
#pragma unroll
    for (int c = 0; c < COLS / 8; ++c) {
      const uint32_t w[4] = {raw[c].x, raw[c].y, raw[c].z, raw[c].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        out[8 * c + e] = (dt == DT_BF16) ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
      }
    }
  }
}

// COLS consecutive 16-bit (fp16 / bf16) values -> fp32.
template <int COLS>
__device__ __forceinline__ void ld_act16(const void* p, int dt, long long idx, float out[COLS]) {
  const uint16_t* q = (const uint16_t*)p + idx;
  if constexpr (COLS == 4) {
    const u32x2 v = *(const u32x2*)q;
    const uint32_t w[2] = {v.x, v.y};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
      out[e] = (dt == DT_BF16) ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
    }
    return;
  }
#pragma unroll
  for (int c = 0; c < COLS; c += 8) {
    const u32x4 v = *(const u32x4*)(q + c);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
      out[c + e] = (dt == DT_BF16) ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
    }
  }
}

template <int COLS>
__device__ __forceinline__ void st_out16(void* p, int dt, long long idx, const float v[COLS]) {
  uint16_t* q = (uint16_t*)p + idx;
  if constexpr (COLS == 4) {
    u32x2 w;
    w.x = (uint32_t)to_out16(v[0], dt) | ((uint32_t)to_out16(v[1], dt) << 16);
    w.y = (uint32_t)to_out16(v[2], dt) | ((uint32_t)to_out16(v[3], dt) << 16);
    *(u32x2*)q = w;
    return;
  }
#pragma unroll
  for (int c = 0; c < COLS; c += 8) {
    u32x4 w;
    w.x = (uint32_t)to_out16(v[c + 0], dt) | ((uint32_t)to_out16(v[c + 1], dt) << 16);
    w.y = (uint32_t)to_out16(v[c + 2], dt) | ((uint32_t)to_out16(v[c + 3], dt) << 16);
    w.z = (uint32_t)to_out16(v[c + 4], dt) | ((uint32_t)to_out16(v[c + 5], dt) << 16);
    w.w = (uint32_t)to_out16(v[c + 6], dt) | ((uint32_t)to_out16(v[c + 7], dt) << 16);
    *(u32x4*)(q + c) = w;
  }
}

template <int COLS>
__device__ __forceinline__ void st_i8(int8_t* p, const int q[COLS]) {
  uint32_t w[COLS / 4];
#pragma unroll
  for (int c = 0; c < COLS / 4; ++c)
    w[c] = ((uint32_t)(q[4 * c] & 0xFF)) | ((uint32_t)(q[4 * c + 1] & 0xFF) << 8) |
           ((uint32_t)(q[4 * c + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * c + 3] & 0xFF) << 24);
  if constexpr (COLS == 16) {
    *(u32x4*)p = u32x4{w[0], w[1], w[2], w[3]};
  } else if constexpr (COLS == 8) {
    *(u32x2*)p = u32x2{w[0], w[1]};
  } else {
    *(uint32_t*)p = w[0];
  }
}

// SPLIT: whether workgroups split K (partials + arrival counters).  Wide launches
// (enough column or row tiles to fill the chip) use SPLIT = false.  MAXW: most waves
// per workgroup (4, or 8 for the decode variants that spread K over one workgroup's
// waves instead of over workgroups).
// Two waves per SIMD (at most 256 registers) except for the fp16-activation W4
// 16-column variant, which holds a deeper register ring and streams at one.
// KS: where the scale folds of the K loop fall.  KS_STEP4: every 4th 32-wide step
// (W4 group 128 with fp16 activations); KS_STEP2: every 2nd step (64-wide activation
// blocks / W4 sub-blocks with int8 activations); KS_ANY: tested per step at run
// time (other groups).  Static positions keep the accumulators in place across steps.
enum KStruct { KS_ANY = 0, KS_STEP2 = 2, KS_STEP4 = 4 };

// Waves per SIMD the register allocation must allow: 2 (at most 256 registers) for the
// 8-column int8-activation variants whose natural allocation lands just above 256,
// except the W4 gate/up ones, which need far more; 1 otherwise (no constraint).
template <int ACT, int WK, int EPI, int COLS>
struct SkOcc {
  static constexpr int value = (ACT == ACT_I8 && COLS == 8 && !(WK == WK_W4 && EPI != EPI_STORE)) ? 2 : 1;
};

// PRO: the launch makes its int8 activations itself (producers.h): a prologue writes the
// codes and scales of the workgroup's rows and K range into LDS, after the first weight
// loads are in flight, and the K loop reads them from there.
template <int ACT, int WK, bool HZ, int EPI, int COLS, bool SPLIT, int MAXW, int KS, bool PRO = false>
__global__ __launch_bounds__(64 * MAXW)
__attribute__((amdgpu_waves_per_eu(SkOcc<ACT, WK, EPI, COLS>::value))) void skinny_kernel(const SkArgs a) {
  static_assert(!PRO || ACT == ACT_I8, "the prologue makes int8 activations");
  constexpr int NS = (EPI == EPI_STORE) ? 1 : 2;  // weight sets feeding one output tile
  constexpr int TN = 16 * COLS;
  constexpr int NQ = COLS / 4;
  constexpr int NR = (WK == WK_W8) ? 8 : 4;  // weight rows per lane per 32-wide K step
  extern __shared__ float red[];

  const int nw = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int j = lane & 15;
  const int g = lane >> 4;
  // 4-column tiles are 64 weight columns: 64-byte (W8) or 32-byte (W4) row pieces, so
  // adjacent tiles share 128-byte lines.  Workgroups are dispatched to the 8 XCDs in
  // turn (workgroup b to XCD b % 8), and each XCD's L2 fetches a line on its own: the
  // tile order pairs adjacent tiles on one XCD (workgroups b and b + 8 of every 16)
  // so a line enters one L2 instead of two (measured: engine-signature W4 decode +2 %,
  // the others unchanged).  Any placement gives the same results.
  int tile = SPLIT ? blockIdx.x / a.splits : blockIdx.x;
  if constexpr (COLS == 4 && !SPLIT) {
    if (tile < (a.ntiles & ~15)) tile = ((tile >> 4) << 4) + 2 * (tile & 7) + ((tile >> 3) & 1);
  }
  const int split = SPLIT ? blockIdx.x - (blockIdx.x / a.splits) * a.splits : 0;
  const int rt = blockIdx.y;
  const int M = a.M;
  const int K = a.K;
  const int G = a.group;

  int si = 0;
  if constexpr (EPI == EPI_STORE) {
    if (a.nseg > 1 && tile >= a.seg[1].tile0) si = 1;
    if (a.nseg > 2 && tile >= a.seg[2].tile0) si = 2;
  }
  const Seg sg0 = a.seg[si];
  const uint8_t* wp[NS];
  const void* sp[NS];
  const uint8_t* zp[NS];
  wp[0] = sg0.w;
  sp[0] = sg0.s;
  zp[0] = sg0.z;
  if constexpr (NS == 2) {
    wp[1] = a.seg[1].w;
    sp[1] = a.seg[1].s;
    zp[1] = a.seg[1].z;
  }
  const int n = sg0.n;
  const int cseg = (tile - sg0.tile0) * TN + j * COLS;  // first column (within the matrix)
  const bool cvalid = cseg < n;
  const int ccl = cvalid ? cseg : 0;                     // in-bounds column for addressing

  const int arow = rt * 16 + j;  // activation row this lane feeds into the A operand
  const bool avalid = arow < M;
  // K range of this wave: contiguous kchunk-wide ranges (lanes == 0), or, for int8
  // activations with lanes == 2, the alternate 64-wide blocks of the split's range
  // (the K order of the tiled int8 kernel: see kof below)
  const bool inter = ACT == ACT_I8 && a.lanes == 2;
  const int kb = inter ? split * a.kchunk + 64 * wave : (split * nw + wave) * a.kchunk;
  const int ke = min(K, kb + a.kchunk);
  const int kst = inter ? 128 : 64;  // K distance between this wave's consecutive 64-wide blocks
  // K range of the workgroup (its waves' ranges together)
  const int kwb = inter ? split * a.kchunk : split * nw * a.kchunk;
  const int kwe = min(K, kwb + (inter ? a.kchunk : nw * a.kchunk));

  f32x4 acc[NS][COLS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int t = 0; t < COLS; ++t) acc[s][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---------------- epilogue prefetch ----------------
  // The finish runs from LDS on chunks of 8 output columns of one row, spread over
  // every thread of the workgroup (item = pass * blockDim + thread).  What it reads
  // from memory -- the tile's W8 column scales (staged into LDS before the finish) and
  // the residual chunk of the first pass -- is loaded here, with clamped addresses and
  // no branch (a dummy residual address when there is none): its latency then overlaps
  // the weight loads, where a branch would make the compiler wait for it at the join.
  const int tid = threadIdx.x;
  const int Mt = min(16, M - rt * 16);        // rows of this row tile
  const int R4 = ((Mt + 3) >> 2) * 4;          // rows of the finish layout
  const int tcol0 = (tile - sg0.tile0) * TN;   // tile's first column within the matrix
  constexpr int TNP = TN + 4;                  // padded row stride of the finish layout
  constexpr int CPR = TN / 8;                  // 8-column chunks per row
  constexpr int NSQ = NS * TN / 4;             // 4-column scale groups of the tile
  const int sq = min(tid, NSQ - 1);
  const int sq_s = sq / (TN / 4), sq_c = (sq % (TN / 4)) * 4;
  u32x4 sraw4[1] = {u32x4{0u, 0u, 0u, 0u}};
  if constexpr (WK == WK_W8) ld_scales_raw_nb<4>(sp[sq_s], a.sdt, min(tcol0 + sq_c, n - 4), sraw4);
  u32x4 rpre = u32x4{0u, 0u, 0u, 0u};
  if constexpr (EPI == EPI_STORE) {
    const int prow = min(tid / CPR, Mt - 1);
    const int pcol = min(tcol0 + (tid % CPR) * 8, n - 8);
    const uint16_t* rb = (const uint16_t*)(a.res ? a.res : a.out);
    const long long rld = a.res ? a.ldr : a.ldo;
    rpre = *(const u32x4*)(rb + (long long)(rt * 16 + prow) * rld + sg0.col0 + pcol);
  }

  // ---------------- software-pipelined K loop ----------------
  // Every load of one 32-wide K step (weights, activations, the step's group scales,
  // zeros and activation scales) goes into slot d of a D-deep register ring and is
  // issued D steps ahead, so D steps of HBM latency overlap.
  // Lanes past N or M read clamped in-bounds addresses; their MFMA columns / rows
  // are never stored.
  constexpr int D = (NS == 2) ? 2 : 4;
  constexpr bool F16 = ACT == ACT_F16;
  constexpr bool W4 = WK == WK_W4;
  using XV = typename std::conditional<F16, u32x4, u32x2>::type;
  struct Step {
    Row<COLS> w[NS][NR];
    XV xv;                            // fp16: 8 halves; int8: 8 bytes
    u32x4 sraw[W4 ? NS : 1][COLS / 4];  // W4: raw scales of the step's group
    Row<COLS> z[(W4 && HZ) ? NS : 1];   // W4: zeros of the step's group
    float as_[F16 ? 1 : 4];           // int8: activation scales, rows 4g..4g+3
  };
  const long long xrow = (long long)(avalid ? arow : 0);
  const _Float16* xpf = (const _Float16*)a.x + xrow * a.ldx + 8 * g;
  const int8_t* xpi = (const int8_t*)a.x + xrow * K + 8 * g;
  const int NG = K / 64;
  long long asrow[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int orow = rt * 16 + 4 * g + r;
    asrow[r] = (long long)(orow < M ? orow : 0) * NG;
  }
  auto load_step = [&](Step& st, int k) {
    if constexpr (F16) {
      st.xv = *(const u32x4*)(xpf + k);
    } else if constexpr (!PRO) {
      st.xv = *(const u32x2*)(xpi + k);
#pragma unroll
      for (int r = 0; r < 4; ++r) st.as_[r] = a.xs[asrow[r] + k / 64];
    }
    const long long r0 = W4 ? (long long)(k / 2 + 4 * g) : (long long)(k + 8 * g);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint8_t* base = wp[s] + r0 * n + ccl;
#pragma unroll
      for (int r = 0; r < NR; ++r) st.w[s][r] = ld_row<COLS, (!W4 && COLS >= 8) || COLS == 16>(base + (long long)r * n, true);
      if constexpr (W4) {
        const long long gi = (long long)(k / G) * n + ccl;
        // measured: the fp16-activation loops run best with the dtype branch (the
        // compiler unswitches them), the int8-activation ones without it
        if constexpr (F16) ld_scales_raw<COLS>(sp[s], a.sdt, gi, st.sraw[s]);
        else ld_scales_raw_nb<COLS>(sp[s], a.sdt, gi, st.sraw[s]);
        if constexpr (HZ) st.z[s] = ld_row<COLS, false>(zp[s] + gi, true);
      }
    }
  };
  const int nsteps = inter ? 2 * (((a.kchunk >> 6) - wave + 1) >> 1) : (ke > kb ? (ke - kb) >> 5 : 0);
  // K of step i: 32-wide steps, two per 64-wide block, blocks kst apart
  auto kof = [&](int i) {
    if constexpr (ACT == ACT_F16) return kb + 32 * i;
    else return kb + kst * (i >> 1) + 32 * (i & 1);
  };
  Step buf[D];
  // The loop is unrolled by U = 4 steps, and compute() receives the step's position
  // u = i % 4 as a compile-time constant.  Every wave's K range starts at a multiple
  // of its K granule (64 for int8 activations, whole W4 groups), so the group and
  // activation-block ends that are multiples of 4 steps apart are known statically
  // and the accumulators stay in place across steps.
  // fp16-activation W8 waves load no step twice: a wave64 memory instruction costs its
  // CU about 16 cycles of address processing, and the decode split-K waves are 2-4
  // steps long, so loads re-issued for a clamped step index (the pipeline's last D)
  // doubled the issue time before the first weights could arrive.  Long ranges run a
  // straight-line main loop (every load valid); the last steps, and short ranges, test
  // each load.  The other variants keep the clamped, branch-free form (measured
  // faster for them: their waves are longer and hold more registers).
  constexpr int U = 4;
  constexpr bool kExactLoads = F16 && !W4;
  // PRO: the workgroup's codes, [Mt][ldq] bytes over [kwb, kwe), then scales [Mt][lng]
  uint8_t* const plq = (uint8_t*)red + a.pro.lds_off;
  const int plng = (kwe - kwb) >> 6;
  float* const pls = (float*)(plq + (long long)Mt * a.pro.ldq);
  float* const plr = pls + Mt * plng;
  ProGeo pgeo;
  ProPre ppre;
  auto prologue = [&]() {
    if constexpr (PRO) {
      ProOut o;
      o.lq = plq;
      o.ls = pls;
      o.ldq = a.pro.ldq;
      o.lng = plng;
      o.lsb = 1;
      o.emit = a.pro.q != nullptr && tile == 0;
      pro_block(a.pro, K, pgeo, ppre, o, plr);
    }
  };
  auto run_pipeline = [&](auto&& compute) {
    if (!PRO && nsteps <= 0) return;
    if constexpr (kExactLoads) {
      // steps [base0, nsteps): fewer than U + D, in at most two static chunks of U
      auto tail = [&](int base0) {
        static_for<0, 2>([&](auto cc) {
          constexpr int c = decltype(cc)::value;
          static_for<0, U>([&](auto uc) {
            constexpr int u = decltype(uc)::value;
            const int i = base0 + c * U + u;
            if (i < nsteps) {
              compute(buf[u % D], kof(i), uc);
              if (i + D < nsteps) load_step(buf[u % D], kof(i + D));
            }
          });
        });
      };
      int base0 = 0;
      if (nsteps >= U + D) {
#pragma unroll
        for (int d = 0; d < D; ++d) load_step(buf[d], kof(d));
        base0 = ((nsteps - U - D) / U + 1) * U;  // chunks whose loads are all in range
        for (int base = 0; base < base0; base += U) {
          static_for<0, U>([&](auto uc) {
            constexpr int u = decltype(uc)::value;
            const int i = base + u;
            compute(buf[u % D], kof(i), uc);
            load_step(buf[u % D], kof(i + D));
          });
        }
      } else {
#pragma unroll
        for (int d = 0; d < D; ++d)
          if (d < nsteps) load_step(buf[d], kof(d));
      }
      tail(base0);
    } else {
      // every load issued unconditionally, the step index clamped to the last step
      if constexpr (PRO) {
        // the prologue's loads go out first (a wave's loads complete in issue order),
        // then the first weight loads -- unconditionally, so that no control-flow join
        // lies between them and the prologue's waits (waves without steps load the
        // workgroup's first K rows and drop them)
        pgeo = pro_geo(a.pro, rt * 16, Mt, kwb, kwe);
        pro_issue(a.pro, K, pgeo, ppre);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int d = 0; d < D; ++d) load_step(buf[d], nsteps > 0 ? kof(d < nsteps ? d : nsteps - 1) : kwb);
        prologue();  // every wave, with its first loads in flight
        if (nsteps <= 0) return;
      } else {
#pragma unroll
        for (int d = 0; d < D; ++d) load_step(buf[d], kof(d < nsteps ? d : nsteps - 1));
      }
      const int nfull = nsteps - nsteps % U;
      for (int base = 0; base < nfull; base += U) {
        static_for<0, U>([&](auto uc) {
          constexpr int u = decltype(uc)::value;
          const int i = base + u;
          compute(buf[u % D], kof(i), uc);
          const int nx = i + D < nsteps ? i + D : nsteps - 1;
          load_step(buf[u % D], kof(nx));
        });
      }
      static_for<0, U - 1>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        const int i = nfull + u;
        if (i < nsteps) {
          compute(buf[u % D], kof(i), uc);
          if constexpr (U > D) {
            const int nx = i + D < nsteps ? i + D : nsteps - 1;
            load_step(buf[u % D], kof(nx));
          }
        }
      });
    }
  };

  if constexpr (F16) {
    // ---------------- fp16 activations, fp16 MFMA ----------------
    // W4: the B operand holds each packed byte as (1024 + lo, 64 + hi) (two
    // instructions, w4_pair_offset).  Per group, two extra MFMAs of the activations
    // against constant operands give c1 = sum(1024 x_even + 64 x_odd) and
    // c2 = sum(x_even + x_odd) for every row; at the group end each column folds in
    // scale * (acc - (c1 + z c2)), with z = 8 when the layout has no zeros, so an
    // explicit all-8 zero tensor gives bit-identical results.
    f32x4 tot[NS][COLS];
    f32x4 c1 = f32x4{0.f, 0.f, 0.f, 0.f}, c2 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int t = 0; t < COLS; ++t) tot[s][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const f16x2 o12 = f16x2{(_Float16)1024.0f, (_Float16)64.0f};
    const f16x2 one2 = f16x2{(_Float16)1.0f, (_Float16)1.0f};
    const f16x8 boff = f16x8{o12[0], o12[1], o12[0], o12[1], o12[0], o12[1], o12[0], o12[1]};
    const f16x8 bone = f16x8{one2[0], one2[1], one2[0], one2[1], one2[0], one2[1], one2[0], one2[1]};
    run_pipeline([&](const Step& st, int k, auto uc) {
      constexpr int u = decltype(uc)::value;
      const f16x8 av = bitcast<f16x8>(st.xv);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
#pragma unroll
        for (int t = 0; t < COLS; ++t) {
          const int q = t >> 2, b = t & 3;
          u32x4 bw;
          if constexpr (W4) {
            bw.x = w4_pair_offset(st.w[s][0].d[q], b);
            bw.y = w4_pair_offset(st.w[s][1].d[q], b);
            bw.z = w4_pair_offset(st.w[s][2].d[q], b);
            bw.w = w4_pair_offset(st.w[s][3].d[q], b);
          } else {
            bw.x = w8_pair_f16(st.w[s][0].d[q], st.w[s][1].d[q], b);
            bw.y = w8_pair_f16(st.w[s][2].d[q], st.w[s][3].d[q], b);
            bw.z = w8_pair_f16(st.w[s][4].d[q], st.w[s][5].d[q], b);
            bw.w = w8_pair_f16(st.w[s][6].d[q], st.w[s][7].d[q], b);
          }
          acc[s][t] = mfma_f16(av, bitcast<f16x8>(bw), acc[s][t]);
        }
      }
      if constexpr (W4) {
        c1 = mfma_f16(av, boff, c1);
        c2 = mfma_f16(av, bone, c2);
        // group end
        if (KS == KS_STEP4 ? (u == 3) : ((k + 32) % G == 0)) {
          f32x4 corr8;
#pragma unroll
          for (int r = 0; r < 4; ++r) corr8[r] = fmaf(8.0f, c2[r], c1[r]);
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            float sc[COLS];
            cvt_scales<COLS>(st.sraw[s], a.sdt, sc);
#pragma unroll
            for (int t = 0; t < COLS; ++t) {
              f32x4 corr = corr8;
              if constexpr (HZ) {
                const float z = (float)byte_of(st.z[s].d[t >> 2], t & 3);
#pragma unroll
                for (int r = 0; r < 4; ++r) corr[r] = fmaf(z, c2[r], c1[r]);
              }
#pragma unroll
              for (int r = 0; r < 4; ++r) tot[s][t][r] = fmaf(sc[t], acc[s][t][r] - corr[r], tot[s][t][r]);
              acc[s][t] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
          }
          c1 = f32x4{0.f, 0.f, 0.f, 0.f};
          c2 = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    });
    if constexpr (W4) {
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int t = 0; t < COLS; ++t) acc[s][t] = tot[s][t];
    }
  } else {
    // ---------------- int8 activations (engine signature), int8 MFMA ----------------
    const int SUB = W4 ? (G < 64 ? G : 64) : 64;
    i32x4 iacc[NS][COLS];
    i32x4 sx = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int t = 0; t < COLS; ++t) iacc[s][t] = i32x4{0, 0, 0, 0};
    // PRO: rows of this lane's A operand and of its activation scales within the row
    // tile (rows past Mt read the last real row; their results are never stored)
    const int parow = min(j, Mt - 1);
    int psrow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) psrow[r] = min(4 * g + r, Mt - 1);
    run_pipeline([&](const Step& st, int k, auto uc) {
      constexpr int u = decltype(uc)::value;
      u32x2 xv;
      float as_[4];
      if constexpr (PRO) {
        xv = *(const u32x2*)(plq + (long long)parow * a.pro.ldq + (k - kwb) + 8 * g);
#pragma unroll
        for (int r = 0; r < 4; ++r) as_[r] = pls[psrow[r] * plng + ((k - kwb) >> 6)];
      } else {
        xv = st.xv;
#pragma unroll
        for (int r = 0; r < 4; ++r) as_[r] = st.as_[r];
      }
      uint64_t ap = (uint64_t)xv.x | ((uint64_t)xv.y << 32);
      if constexpr (W4) {
        // k slots: even K values first, then odd (the nibble split order below)
        ap = (uint64_t)perm(xv.y, xv.x, 0x06040200u) | ((uint64_t)perm(xv.y, xv.x, 0x07050301u) << 32);
      }
#pragma unroll
      for (int s = 0; s < NS; ++s) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          uint32_t lo4[4], hi4[4];
          if constexpr (W4) {
            uint32_t L[4], H[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) w4_split_i8x16(st.w[s][r].d[q], L[r], H[r]);
            tr4(L[0], L[1], L[2], L[3], lo4);
            tr4(H[0], H[1], H[2], H[3], hi4);
          } else {
            tr4(st.w[s][0].d[q], st.w[s][1].d[q], st.w[s][2].d[q], st.w[s][3].d[q], lo4);
            tr4(st.w[s][4].d[q], st.w[s][5].d[q], st.w[s][6].d[q], st.w[s][7].d[q], hi4);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const uint64_t bv = (uint64_t)lo4[u] | ((uint64_t)hi4[u] << 32);
            iacc[s][4 * q + u] = mfma_i8(ap, bv, iacc[s][4 * q + u]);
          }
        }
      }
      if constexpr (W4 && HZ) sx = mfma_i8(ap, 0x0101010101010101ull, sx);
      // end of an activation block / weight sub-block
      if (KS == KS_STEP2 ? (u & 1) == 1 : ((k + 32) % SUB == 0)) {
        if constexpr (!W4) {
#pragma unroll
          for (int s = 0; s < NS; ++s)
#pragma unroll
            for (int t = 0; t < COLS; ++t) {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                acc[s][t][r] = fmaf((float)iacc[s][t][r], as_[r], acc[s][t][r]);
              iacc[s][t] = i32x4{0, 0, 0, 0};
            }
        } else {
#pragma unroll
          for (int s = 0; s < NS; ++s) {
            // The MFMA summed 16 * (nibble - 8) * a: float(16 * dot) (exact, |.| < 2^24)
            // against the scale product divided by 16 (exact) is fma(float(dot), a_s *
            // b_s, acc) bit for bit, without a shift per output.
            float ws[COLS];
            cvt_scales<COLS>(st.sraw[s], a.sdt, ws);
#pragma unroll
            for (int t = 0; t < COLS; ++t) ws[t] *= 0.0625f;
#pragma unroll
            for (int t = 0; t < COLS; ++t) {
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                int v = iacc[s][t][r];  // 16 * the dot
                if constexpr (HZ) v += (8 - (int)byte_of(st.z[s].d[t >> 2], t & 3)) * 16 * sx[r];
                acc[s][t][r] = fmaf((float)v, as_[r] * ws[t], acc[s][t][r]);
              }
              iacc[s][t] = i32x4{0, 0, 0, 0};
            }
          }
          if constexpr (HZ) sx = i32x4{0, 0, 0, 0};
        }
      }
    });
  }


  // ---------------- finish layout: workgroup sums in LDS ----------------
  // Every wave writes its accumulators (the row groups that hold real rows) as
  // [set][row][column] (row stride TNP) into its own slot; the slots are summed in wave
  // order (0, 1, ..., nw-1) into slot 0.  The W8 column scales follow the slots as fp32
  // [set][column].  `red` holds nw slots of NS*R4*TNP floats plus NS*TN floats.
  const int per = NS * R4 * TNP;
  float* const scl = red + nw * per;
  if (g < R4 / 4) {
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
      for (int t = 0; t < COLS; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave * per + (s * R4 + 4 * g + r) * TNP + j * COLS + t] = acc[s][t][r];
  }
  if constexpr (WK == WK_W8) {
    if (tid < NSQ) {
      float c4[4];
      cvt_scales<4>(sraw4, a.sdt, c4);
#pragma unroll
      for (int e = 0; e < 4; ++e) scl[sq_s * TN + sq_c + e] = c4[e];
    }
  }
  __syncthreads();
  if (nw > 1) {
    // every slot's value is read before the first add (a loop over the run-time wave
    // count would wait out one LDS latency per wave); slots past nw re-read the last
    for (int e = tid; e < per; e += blockDim.x) {
      float p[MAXW];
#pragma unroll
      for (int w = 0; w < MAXW; ++w) p[w] = red[min(w, nw - 1) * per + e];
      float v = p[0];
#pragma unroll
      for (int w = 1; w < MAXW; ++w)
        if (w < nw) v += p[w];
      red[e] = v;
    }
    __syncthreads();
  }

  // ---------------- reduction over workgroups (split-K) ----------------
  // Partials travel as 16-byte device-coherent (SC1) stores and loads, readable from
  // every XCD without a whole-L2 writeback or invalidate.  Every thread stores its
  // (set, row, 4-column) groups of the workgroup's sums and waits for its stores;
  // after a barrier one thread increments the tile's arrival counter, and the
  // workgroup that sees the final count sums every split's partial in split order
  // (8 splits' loads in flight at a time) back into the finish layout.
  if constexpr (SPLIT) {
    __shared__ int s_last;
    const long long MN = (long long)M * a.ncols;
    const __amdgpu_buffer_rsrc_t rs = part_rsrc(a.part, (unsigned)((long long)a.splits * NS * MN * 4));
    constexpr int TN4 = TN / 4;
    const int nel4 = NS * Mt * TN4;
    const unsigned sstride = (unsigned)(NS * MN * 4);
    for (int e = tid; e < nel4; e += blockDim.x) {
      const int s = e / (Mt * TN4);
      const int rem = e - s * (Mt * TN4);
      const int row = rem / TN4;
      const int col = (rem - row * TN4) * 4;
      if (tcol0 + col < n) {
        const unsigned off = (unsigned)((((long long)split * NS + s) * MN + (long long)(rt * 16 + row) * a.ncols +
                                         sg0.col0 + tcol0 + col) * 4);
        st_coherent(*(const f32x4*)&red[(s * R4 + row) * TNP + col], rs, off);
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // every partial store of this thread has completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) {
      unsigned* cp = a.cnt + (long long)rt * a.ntiles + tile;
      const unsigned prev = __hip_atomic_fetch_add(cp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == (unsigned)(a.splits - 1);
      if (last) __hip_atomic_store(cp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;  // uniform over the workgroup
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    for (int e = tid; e < nel4; e += blockDim.x) {
      const int s = e / (Mt * TN4);
      const int rem = e - s * (Mt * TN4);
      const int row = rem / TN4;
      const int col = (rem - row * TN4) * 4;
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      if (tcol0 + col < n) {
        const unsigned off =
            (unsigned)(((long long)s * MN + (long long)(rt * 16 + row) * a.ncols + sg0.col0 + tcol0 + col) * 4);
        for (int p0 = 0; p0 < a.splits; p0 += 8) {
          f32x4 part[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) part[q] = ld_coherent(rs, off + (unsigned)min(p0 + q, a.splits - 1) * sstride);
#pragma unroll
          for (int q = 0; q < 8; ++q)
            if (p0 + q < a.splits) v = (p0 + q == 0) ? part[q] : v + part[q];
        }
      }
      *(f32x4*)&red[(s * R4 + row) * TNP + col] = v;
    }
    __syncthreads();
  }

  // ---------------- epilogue: every thread, 8-column chunks of one row ----------------
  // The pass count is uniform, so every lane of a wave reaches the amax shuffles;
  // items past the tile compute on clamped rows and store nothing.
  const int nitems = Mt * CPR;
  for (int base = 0; base < nitems; base += blockDim.x) {
    const int it = base + tid;
    const int row = min(it / CPR, Mt - 1);
    const int c = (it % CPR) * 8;                // chunk's first column within the tile
    const bool cval = it < nitems && tcol0 + c < n;
    const int orow = rt * 16 + row;
    const long long oc = (long long)sg0.col0 + tcol0 + c;  // first output column
    // W8 column scale, then the residual: one rounding (fmaf) with a residual, the
    // product alone without; the tiled int8 kernel rounds the same way, so both
    // families give the same bits for the same K order.
    float v[NS][8], cs[NS][8];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const f32x4 lo = *(const f32x4*)&red[(s * R4 + row) * TNP + c];
      const f32x4 hi = *(const f32x4*)&red[(s * R4 + row) * TNP + c + 4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[s][e] = lo[e], v[s][4 + e] = hi[e];
#pragma unroll
      for (int e = 0; e < 8; ++e) cs[s][e] = (WK == WK_W8) ? scl[s * TN + c + e] : 1.0f;
    }
    if constexpr (EPI == EPI_STORE) {
      if (a.res != nullptr) {
        // items past the row or the tile read a clamped, in-bounds chunk and store nothing
        const long long rc = (long long)sg0.col0 + min(tcol0 + c, n - 8);
        const u32x4 rr = (base == 0) ? rpre : *(const u32x4*)((const uint16_t*)a.res + (long long)orow * a.ldr + rc);
        const uint32_t rw[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint16_t h = (uint16_t)(rw[e >> 1] >> (16 * (e & 1)));
          v[0][e] = fmaf(v[0][e], cs[0][e], (a.odt == DT_BF16) ? bf16_to_f32(h) : (float)bitcast<_Float16>(h));
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[0][e] *= cs[0][e];
      }
      if (cval) st_out16<8>(a.out, a.odt, (long long)orow * a.ldo + oc, v[0]);
    } else {
      float h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = silu(v[0][e] * cs[0][e]) * (v[1][e] * cs[1][e]);
      if constexpr (EPI == EPI_GATEUP) {
        if (cval) st_out16<8>(a.out, DT_BF16, (long long)orow * a.ncols + oc, h);
      } else {
        // bf16 round trip (kernels/gemm.py:198-200), then the amax of the 64-column
        // group over its 8 chunks (8 consecutive lanes)
        float am = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          h[e] = bf16_to_f32(f32_to_bf16(h[e]));
          am = fmaxf(am, fabsf(h[e]));
        }
        if (!cval) am = 0.0f;
#pragma unroll
        for (int m = 1; m < 8; m <<= 1) am = fmaxf(am, __shfl_xor(am, m));
        const float sc = fmaxf(am / 127.0f, 1e-8f);
        int q[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = round_i8(h[e] / sc);
        if (cval) {
          st_i8<8>(a.oq + (long long)orow * a.ncols + oc, q);
          if ((c & 63) == 0) a.os[(long long)orow * (a.ncols / 64) + oc / 64] = sc;
        }
      }
    }
  }
}

template <int ACT, int WK, bool HZ, int EPI, int COLS, bool SPLIT, int MAXW, int KS, bool PRO = false>
hipError_t launch_v(const SkLaunch& L, const SkArgs& a, hipStream_t st) {
  auto* k = skinny_kernel<ACT, WK, HZ, EPI, COLS, SPLIT, MAXW, KS, PRO>;
  // Largest dynamic LDS of this variant (MAXW finish slots of 16 rows, the column
  // scales, the prologue's code block); the kernel's static LDS comes on top, so the
  // limit is raised to exactly this, not to the whole 160 KB.
  constexpr int NS = (EPI == EPI_STORE) ? 1 : 2;
  constexpr size_t kFinLds = ((size_t)MAXW * NS * 16 * (16 * COLS + 4) + (size_t)NS * 16 * COLS) * sizeof(float);
  constexpr size_t kMaxLds = PRO ? std::min<size_t>(kFinLds + kProLdsBytes, 160 * 1024 - 256) : kFinLds;
  if (L.lds > kMaxLds) return hipErrorInvalidValue;
  if constexpr (kMaxLds > 65536) {
    static bool attr_set = false;  // benign race: every caller sets the same value
    if (!attr_set) {
      const hipError_t e =
          hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMaxLds);
      if (e != hipSuccess) return e;
      attr_set = true;
    }
  }
  hipLaunchKernelGGL(k, L.grid, dim3(64 * L.waves), L.lds, st, a);
  return hipGetLastError();
}

// BIG: the variant also exists with up to 8 waves per workgroup.  COLS = 4: the
// one-pass variants (K over up to 8 waves of one workgroup, no split).
template <int ACT, int WK, bool HZ, int EPI, int COLS, bool BIG, int KS, bool PRO = false>
hipError_t launch_t(const SkLaunch& L, const SkArgs& a, hipStream_t st) {
  if constexpr (COLS == 4) {
    if (a.splits > 1 || L.waves > 8) return hipErrorInvalidValue;
    return launch_v<ACT, WK, HZ, EPI, 4, false, 8, KS, PRO>(L, a, st);
  } else {
    if (L.waves > 4) {
      if constexpr (BIG) {
        if (a.splits > 1) return launch_v<ACT, WK, HZ, EPI, COLS, true, 8, KS, PRO>(L, a, st);
        return launch_v<ACT, WK, HZ, EPI, COLS, false, 8, KS, PRO>(L, a, st);
      }
      return hipErrorInvalidValue;
    }
    if (a.splits > 1) return launch_v<ACT, WK, HZ, EPI, COLS, true, 4, KS, PRO>(L, a, st);
    return launch_v<ACT, WK, HZ, EPI, COLS, false, 4, KS, PRO>(L, a, st);
  }
}

#define QL_CASE(A, W, Z, E, C, B, KSV)                                                          \
  if (L.act == A && L.wk == W && (L.hz != 0) == Z && L.epi == E && L.cols == C && L.ks == KSV) \
    return launch_t<A, W, Z, E, C, B, KSV>(L, a, st);
// the fused-prologue variant of a case
#define QL_CASE_PRO(W, Z, E, C, B)                                                         \
  if (L.wk == W && (L.hz != 0) == Z && L.epi == E && L.cols == C && L.ks == KS_STEP2) \
    return launch_t<ACT_I8, W, Z, E, C, B, KS_STEP2, true>(L, a, st);

}  // namespace qlin
