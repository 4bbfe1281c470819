// Tiled int8-activation GEMM for the engine-signature calls with more than 16 rows
// (prefill chunks), gfx950: int8 or W4 weights; the store epilogue and the fused
// gate/up epilogues (silu(g) * u, optionally requantized per 64 columns).
//
// Replaces the prefill-sized launches of gemm_i8, gemm_w4, proj3(_w4) and
// mlp_gate_up(_quant)(_w4) (kernels/gemm.py:20-312; kernels/w4.py:64-323) with the
// reference's arithmetic: an exact int32 dot per 64-wide activation block, then
// `acc += float(dot) * a_s[m, block]` in fp32 (W4: per 64-wide weight sub-block,
// `acc += float(dot) * (a_s * b_s[group, n])`, w4.py:103-104), then the column scale
// (W8) and either the residual and a 16-bit store (gemm.py:43-57) or, for gate/up
// (two weight sets feeding one tile), h = silu(g) * u, stored as bf16 or rounded
// through bf16 and quantized per 64 columns with max(amax / 127, 1e-8) and round
// half away from zero (gemm.py:195-211).
//
//   * Workgroup tile 128 x 128, 8 waves: 2 x 2 wave tiles of 64 x 64, times two K
//     groups.  A stage of the LDS ring holds two activation blocks (128 K); group kg
//     computes block 2 * stage + kg, and at the end group 1's accumulators are added
//     to group 0's through LDS (fixed order).
//   * MFMA: v_mfma_i32_16x16x64_i8, one instruction per 64-wide block, started from
//     an inline zero.  Lane (g, j) holds K bytes 16g..16g+15 of activation row j and
//     of weight column 4j + t for instruction t.  Weight bytes are N-contiguous in
//     LDS (as in HBM, rows padded per lane group); each lane reads 4 adjacent columns
//     of its 16 K rows (one dword per row) and 4x4 byte transposes turn them into the
//     4 B operands.  W4: the
//     nibbles become int8 16 * (n - 8) (even K then odd K), the activation operand
//     is permuted to the same order, and the dot is shifted right by 4 (exact);
//     explicit zeros add (8 - z) * sum(a) from one more MFMA against all-ones.
//   * Copies: global -> registers (three stages ahead, two for gate/up) -> LDS (one
//     stage ahead), one barrier per stage.
//   * Split-K: `splits` workgroups per tile over equal ranges of 64-wide blocks; each
//     stores its fp32 partial tile (both weight sets for gate/up; device-coherent) and
//     counts its arrival, and the last to arrive sums the partials in split order and
//     runs the epilogue.
//   * The K order of every output element is fixed (blocks in order within each K
//     group, then group 0 + group 1, then splits in order), so rows do not depend on M
//     or on the chunking for a given split count.
#include <stdlib.h>

#include <algorithm>

#include "qlin_dev.h"
#include "qlin_internal.h"

namespace qlin {

namespace {

constexpr int BM = 128;
constexpr int GROUP_M = 8;  // tile order: 8 row tiles per group share weight column tiles in L2

// WNW: 64-column wave tiles per workgroup row.  2: the 128 x 128 tile of 8 waves with
// copies through registers; 1: the 128 x 64 tile of 4 waves with LDS DMA copies (W8 store
// calls), small enough in registers and LDS for three workgroups per CU.
template <int WK, int NS, int WNW = 2>
struct Gi8 {
  static constexpr int BN = 64 * WNW;
  static constexpr int WAVES = 4 * WNW;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr bool W4 = WK == WK_W4;
  static constexpr int A_BLK = BM * 64;                 // activation bytes of one block
  static constexpr int B_ROWS = W4 ? 32 : 64;           // weight rows of one block
  // Weight rows are N-contiguous (128 bytes), with 64 bytes of padding after every
  // group of RG rows, RG = the rows of one MFMA lane group (16 int8, 8 packed).  The
  // four lane groups of a ds_read_b32 then start 16 dwords apart modulo the 64 banks
  // and read without bank conflicts (unpadded they all hit the same 16 banks).
  static constexpr int RG = W4 ? 8 : 16;
  static constexpr int B_PAD = 64;
  static constexpr int B_BLK = B_ROWS * BN + (B_ROWS / RG) * B_PAD;  // one block of one set
  static __device__ __forceinline__ int b_row(int r) { return r * BN + (r / RG) * B_PAD; }
  static constexpr int B_OFF = 2 * A_BLK;               // weights: [set][2 blocks]
  static constexpr int AS_OFF = B_OFF + NS * 2 * B_BLK;  // activation scales: [2][128] fp32
  static constexpr int BS_OFF = AS_OFF + 2 * BM * 4;    // W4 group scales: [set][2][128] fp32
  static constexpr int BZ_OFF = BS_OFF + (W4 ? NS * 2 * BN * 4 : 0);  // W4 zeros: [set][2][128] bytes
  static constexpr int STAGE = BZ_OFF + (W4 ? NS * 2 * BN : 0);
  static constexpr int RED = 2 * WNW * 64 * 64 * 4;  // one set of group 1's accumulators at the end
  static constexpr int LDS = (2 * STAGE > RED) ? 2 * STAGE : RED;
};

__device__ __forceinline__ uint32_t rfl(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// activation row r's 16-byte chunk c within a block: rows of 64 bytes, chunks swizzled
// so the 8-lane phases of ds_read_b128 hit distinct banks
__device__ __forceinline__ int a_off(int r, int c) { return r * 64 + 16 * (c ^ ((r >> 2) & 3)); }

}  // namespace

// 16-byte / 4-byte LDS DMA: lane i copies from vaddr to LDS m0 + 16 i (4 i).  Issued from
// inline assembly; the loop waits for them explicitly (vmcnt) before its barrier.
__device__ __forceinline__ void i8_dma16(const void* vaddr, uint32_t m0) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(vaddr), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void i8_dma4(const void* vaddr, uint32_t m0) {
  asm volatile("global_load_lds_dword %0, off" ::"v"(vaddr), "{m0}"(m0) : "memory");
}
constexpr int kWaitVm0 = 0x0F70;  // s_waitcnt vmcnt(0) (expcnt, lgkmcnt at their maxima)

template <int WK, bool HZ, int EPI, int WNW>
__global__ __launch_bounds__(256 * WNW) __attribute__((amdgpu_waves_per_eu(WNW == 1 ? 3 : 2)))
void prefill_i8_kernel(const SkArgs a) {
  constexpr int NS = (EPI == EPI_STORE) ? 1 : 2;  // weight sets feeding one tile
  using G = Gi8<WK, NS, WNW>;
  constexpr int BN = G::BN, THREADS = G::THREADS;
  static_assert(WNW == 2 || (WK == WK_W8 && NS == 1), "the DMA tile serves W8 store calls");
  constexpr bool W4 = G::W4;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int tid = threadIdx.x;
  const int wave = (int)rfl((uint32_t)tid >> 6), lane = tid & 63;
  const int j = lane & 15, g = lane >> 4;
  const int kg = wave / (2 * WNW), wm = (wave / WNW) & 1, wn = wave % WNW;
  const int M = a.M, K = a.K;
  // split-K: `S` workgroups per output tile, each over nk consecutive 64-wide blocks
  // from kb0
  // Workgroups go to the 8 XCDs in turn; with a.gm set, XCD x's workgroups (b = x,
  // x + 8, ...) take one contiguous run of the tile order (a tile's splits included).
  const int S = a.splits;
  const int b = (int)blockIdx.x, W = (int)gridDim.x;
  const int v = a.gm > 0 ? (b & 7) * (W >> 3) + min(b & 7, W & 7) + (b >> 3) : b;
  const int tile = v / S, split = v % S;
  const int nk = K / 64 / S;
  const int kb0 = split * nk;

  // grouped tile order: runs of consecutive tiles cover gm row tiles x a few column
  // tiles, so the workgroups of one XCD share activation and weight tiles in its L2
  const int tiles_m = (M + BM - 1) / BM, tiles_n = a.ntiles;
  const int gm = a.gm > 0 ? a.gm : GROUP_M;
  const int per_group = gm * tiles_n;
  const int grp = tile / per_group;
  const int first_m = grp * gm;
  const int gsize = min(tiles_m - first_m, gm);
  const int tm = first_m + (tile % per_group) % gsize;
  const int tn = (tile % per_group) / gsize;
  int si = 0;
  if constexpr (EPI == EPI_STORE) {
    if (a.nseg > 1 && tn >= a.seg[1].tile0) si = 1;
    if (a.nseg > 2 && tn >= a.seg[2].tile0) si = 2;
  }
  const Seg sg = a.seg[si];
  const uint8_t* wset[NS];
  const void* sset[NS];
  const uint8_t* zset[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    wset[s] = a.seg[si + s].w;
    sset[s] = a.seg[si + s].s;
    zset[s] = a.seg[si + s].z;
  }
  const int n = sg.n;
  const int ncol0 = (tn - sg.tile0) * BN;  // tile's first column within its matrix
  const int m0 = tm * BM;

  // ---------------- copies: global -> registers -> LDS ----------------
  // A: 1024 16-byte chunks per stage (2 per thread); B: W8 1024, W4 512; scales and
  // zeros: one value per thread.  Rows past M and blocks past the last read
  // clamped, in-bounds addresses and are never used.
  const int8_t* xq = (const int8_t*)a.x;
  const int NG = K / 64;
  struct Regs {
    u32x4 av[2];
    u32x4 bv[NS][W4 ? 1 : 2];
    float as_;
    uint32_t bs;  // W4: raw dword of one group scale of set tid / 256
    uint32_t bz;  // W4 with zeros: the matching zero
  };
  // The block of every load below is uniform over a wave (its K group k2 is a function of
  // the wave), so each address is a per-thread offset fixed for the whole loop plus the
  // block's offset in a scalar register: buffer loads over the activations, weights and
  // activation scales (the host keeps each under 2^31 bytes), no per-stage address
  // arithmetic on the vector ALU.
  const __amdgpu_buffer_rsrc_t xr = part_rsrc(xq, (unsigned)((long long)M * K));
  const __amdgpu_buffer_rsrc_t sr = part_rsrc(a.xs, (unsigned)((long long)M * NG * 4));
  __amdgpu_buffer_rsrc_t wr[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) wr[s] = part_rsrc(wset[s], (unsigned)((long long)(W4 ? K / 2 : K) * n));
  unsigned xoff[2], woff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = tid + THREADS * i;
    const int r = (q & 511) >> 2, c = q & 3;
    xoff[i] = (unsigned)(min(m0 + r, M - 1) * K + 16 * c);
    const int rw = W4 ? (tid & 255) >> 3 : (q & 511) >> 3, cw = W4 ? tid & 7 : q & 7;
    woff[i] = (unsigned)(rw * n + ncol0 + 16 * cw);
  }
  const unsigned soff = (unsigned)(min(m0 + (tid & 127), M - 1) * NG * 4);
  auto fetch = [&](Regs& rg, int st) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int blk = kb0 + min(2 * st + i, nk - 1);  // K group i (q >> 9 = i)
      rg.av[i] = bitcast<u32x4>(__builtin_amdgcn_raw_buffer_load_b128(xr, xoff[i], blk * 64, 0));
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if constexpr (W4) {
        const int blk = kb0 + min(2 * st + (tid >> 8), nk - 1);
        rg.bv[s][0] = bitcast<u32x4>(__builtin_amdgcn_raw_buffer_load_b128(wr[s], woff[0], blk * 32 * n, 0));
      } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int blk = kb0 + min(2 * st + i, nk - 1);
          rg.bv[s][i] = bitcast<u32x4>(__builtin_amdgcn_raw_buffer_load_b128(wr[s], woff[i], blk * 64 * n, 0));
        }
      }
    }
    if (tid < 256) {
      const int blk = kb0 + min(2 * st + (tid >> 7), nk - 1);
      rg.as_ = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, soff, blk * 4, 0));
    }
    if constexpr (W4) {
      // group scales (and zeros) of both blocks: 256 per set, thread tid takes one of
      // set tid / 256
      const int s = tid >> 8;
      if (s < NS) {
        const int t2 = tid & 255, k2 = t2 >> 7, c = t2 & 127;
        const int blk = kb0 + min(2 * st + k2, nk - 1);
        const long long gi = (long long)(blk * 64 / a.group) * n + ncol0 + c;
        rg.bs = ld_scale1_raw(sset[s], a.sdt, gi);  // converted at the LDS store
        if constexpr (HZ) rg.bz = ld_global<uint8_t>(zset[s] + gi);
      }
    }
  };
  auto store = [&](const Regs& rg, int buf) {
    uint8_t* base = lds + buf * G::STAGE;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = tid + THREADS * i;
      const int k2 = q >> 9, r = (q & 511) >> 2, c = q & 3;
      *(u32x4*)(base + k2 * G::A_BLK + a_off(r, c)) = rg.av[i];
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint8_t* sb = base + G::B_OFF + s * 2 * G::B_BLK;
      if constexpr (W4) {
        const int k2 = tid >> 8, r = (tid & 255) >> 3, c = tid & 7;
        *(u32x4*)(sb + k2 * G::B_BLK + G::b_row(r) + 16 * c) = rg.bv[s][0];
      } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int q = tid + THREADS * i;
          const int k2 = q >> 9, r = (q & 511) >> 3, c = q & 7;
          *(u32x4*)(sb + k2 * G::B_BLK + G::b_row(r) + 16 * c) = rg.bv[s][i];
        }
      }
    }
    if (tid < 256) ((float*)(base + G::AS_OFF))[tid] = rg.as_;
    if constexpr (W4) {
      if ((tid >> 8) < NS) {
        // gi of the fetch has the parity of tid (n and ncol0 are even)
        ((float*)(base + G::BS_OFF))[tid] = cvt_scale1(rg.bs, a.sdt, tid);
        if constexpr (HZ) base[G::BZ_OFF + tid] = (uint8_t)rg.bz;
      }
    }
  };

  f32x4 acc[NS][4][4];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[s][rb][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const i32x4 izero = i32x4{0, 0, 0, 0};
  const int cb = wn * 64 + 4 * j;  // lane's first column within the tile
  // W8 column scales of the epilogue, loaded now (no branch) so their latency hides
  // behind the K loop
  u32x4 csraw[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    csraw[s] = W4 ? u32x4{0u, 0u, 0u, 0u} : ld_scale4_raw(sset[s], a.sdt, min(ncol0 + cb, n - 4));

  // one 64-wide block of this wave's K group from LDS stage `buf`
  auto compute = [&](int buf) {
    const uint8_t* base = lds + buf * G::STAGE;
    const uint8_t* sa = base + kg * G::A_BLK;
    i32x4 av[4];
    f32x4 asv[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const int r = wm * 64 + rb * 16 + j;
      av[rb] = *(const i32x4*)(sa + a_off(r, g));
      asv[rb] = *(const f32x4*)(base + G::AS_OFF + (kg * BM + wm * 64 + rb * 16 + 4 * g) * 4);
    }
    if constexpr (W4) {
      // activation slots in the order of the nibble split: even K of the 16, then odd K
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const u32x4 x = bitcast<u32x4>(av[rb]);
        av[rb] = bitcast<i32x4>(u32x4{perm(x.y, x.x, 0x06040200u), perm(x.w, x.z, 0x06040200u),
                                      perm(x.y, x.x, 0x07050301u), perm(x.w, x.z, 0x07050301u)});
      }
    }
    i32x4 sx[4];
    if constexpr (W4 && HZ) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
        sx[rb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
            av[rb], bitcast<i32x4>(u32x4{0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u}), izero, 0, 0, 0);
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint8_t* sb = base + G::B_OFF + (s * 2 + kg) * G::B_BLK;
      u32x4 bv[4];
      if constexpr (W4) {
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w4_split_i8x16(*(const uint32_t*)(sb + G::b_row(8 * g + i) + cb), lo[i], hi[i]);
        uint32_t e0[4], e1[4], o0[4], o1[4];
        tr4(lo[0], lo[1], lo[2], lo[3], e0);
        tr4(lo[4], lo[5], lo[6], lo[7], e1);
        tr4(hi[0], hi[1], hi[2], hi[3], o0);
        tr4(hi[4], hi[5], hi[6], hi[7], o1);
#pragma unroll
        for (int t = 0; t < 4; ++t) bv[t] = u32x4{e0[t], e1[t], o0[t], o1[t]};
        // The MFMA sums 16 * (nibble - 8) * a: the dot is p / 16, exactly.  Rather than
        // shifting every p, the fold takes float(p) (exact: |p| < 2^24) against the scale
        // product divided by 16 (exact): fma(float(p), fl(a_s * b_s) / 16, acc) is
        // fma(float(p / 16), fl(a_s * b_s), acc) bit for bit, one instruction less.
        const f32x4 bsv = *(const f32x4*)(base + G::BS_OFF + (s * 256 + kg * BN + cb) * 4) * 0.0625f;
        int zc[4] = {0, 0, 0, 0};  // 16 * (8 - z): explicit zeros add (8 - z) * sum(a), times 16
        if constexpr (HZ) {
          const uint32_t zw = *(const uint32_t*)(base + G::BZ_OFF + s * 256 + kg * BN + cb);
#pragma unroll
          for (int t = 0; t < 4; ++t) zc[t] = (8 - (int)((zw >> (8 * t)) & 0xFFu)) * 16;
        }
        auto fold4 = [&](const i32x4& p, int rb, int t) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            int v = p[r];  // 16 * the dot
            if constexpr (HZ) v += zc[t] * sx[rb][r];
            acc[s][rb][t][r] = fmaf((float)v, asv[rb][r] * bsv[t], acc[s][rb][t][r]);
          }
        };
        if constexpr (NS == 1) {
          // all 16 dots first, then their folds (as for W8 below)
          i32x4 p[4][4];
#pragma unroll
          for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int t = 0; t < 4; ++t)
              p[rb][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[rb], bitcast<i32x4>(bv[t]), izero, 0, 0, 0);
#pragma unroll
          for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int t = 0; t < 4; ++t) fold4(p[rb][t], rb, t);
        } else {
#pragma unroll
          for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int t = 0; t < 4; ++t)
              fold4(__builtin_amdgcn_mfma_i32_16x16x64_i8(av[rb], bitcast<i32x4>(bv[t]), izero, 0, 0, 0), rb, t);
        }
      } else {
        uint32_t d[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) d[i] = *(const uint32_t*)(sb + G::b_row(16 * g + i) + cb);
        uint32_t x0[4], x1[4], x2[4], x3[4];
        tr4(d[0], d[1], d[2], d[3], x0);
        tr4(d[4], d[5], d[6], d[7], x1);
        tr4(d[8], d[9], d[10], d[11], x2);
        tr4(d[12], d[13], d[14], d[15], x3);
#pragma unroll
        for (int t = 0; t < 4; ++t) bv[t] = u32x4{x0[t], x1[t], x2[t], x3[t]};
        if constexpr (NS == 1 && WNW == 2) {
          // all 16 dots first, then their folds: the folds run back to back instead of each
          // waiting on its MFMA (a block's compute measured 1029 instead of 1397 cycles for a
          // wave alone, 650 instead of 789 per block with two waves on a SIMD)
          i32x4 p[4][4];
#pragma unroll
          for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int t = 0; t < 4; ++t)
              p[rb][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[rb], bitcast<i32x4>(bv[t]), izero, 0, 0, 0);
#pragma unroll
          for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[s][rb][t][r] = fmaf((float)p[rb][t][r], asv[rb][r], acc[s][rb][t][r]);
        } else {
#pragma unroll
          for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const i32x4 p = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[rb], bitcast<i32x4>(bv[t]), izero, 0, 0, 0);
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[s][rb][t][r] = fmaf((float)p[r], asv[rb][r], acc[s][rb][t][r]);
            }
        }
      }
    }
  };

  // ---------------- K loop: stage st holds blocks 2st and 2st+1 ----------------
  // Stage s is stored to LDS buffer s & 1 one iteration ahead (after the barrier that
  // ended the last read of that buffer) and computed in iteration s.  Its copy into
  // registers is issued three iterations ahead with one weight set (two register
  // sets, the loop written for even and odd st so their indices are static) and two
  // iterations ahead with two (one register set: the gate/up accumulators need the
  // registers).  The copy goes out right after the registers' LDS store, before the
  // barrier, so its issue overlaps the wait there (gate/up 47 us instead of 51 at
  // M = 512; issuing the store and copy before the MFMAs instead measured 49).
  // Every copy and LDS store is issued unconditionally: stages past the last one read
  // the last block again (fetch clamps the block index) and are stored to the buffer
  // no one reads any more.  A copy issued under a condition made the wait insertion
  // assume, at the join, that its registers were the most recent loads: it waited for
  // every copy in flight (vmcnt(0)) before each stage's LDS stores and again before
  // the next copy, so a stage waited a whole memory round trip.
  const int nst = (nk + 1) / 2;
  if constexpr (WNW == 1) {
    // Two LDS stages; the copy of stage st+1 goes out (LDS DMA, no registers) while stage st
    // is computed, into the buffer the barrier that ended stage st-1 freed.  Stages past the
    // last read the last block again (the index is clamped) into a buffer no one reads.
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
    auto dma_stage = [&](int st, int buf) {
      const uint32_t sbase = lds0 + (uint32_t)(buf * G::STAGE);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {  // activations: 16 x 1 KB per stage, 4 per wave
        const int q = wave * 4 + q4, k2 = q >> 3;
        const int r = (q & 7) * 16 + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 2) & 3);  // the chunk a_off(r, c) places at this slot
        const int blk = kb0 + min(2 * st + k2, nk - 1);
        const int row = min(m0 + r, M - 1);
        i8_dma16(xq + (long long)row * K + blk * 64 + 16 * c, sbase + (uint32_t)(k2 * G::A_BLK + (q & 7) * 1024));
      }
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) {  // weights: 8 groups of 16 rows x 64 bytes, 2 per wave
        const int q = wave * 2 + q2, k2 = q >> 2, grp = q & 3;
        const int blk = kb0 + min(2 * st + k2, nk - 1);
        const uint8_t* src = wset[0] + (long long)(blk * 64 + 16 * grp + (lane >> 2)) * n + ncol0 + 16 * (lane & 3);
        i8_dma16(src, sbase + (uint32_t)(G::B_OFF + k2 * G::B_BLK + G::b_row(16 * grp)));
      }
      {  // activation scales: [2 blocks][128 rows] fp32, 64 per wave
        const int k2 = wave >> 1, r = (wave & 1) * 64 + lane;
        const int blk = kb0 + min(2 * st + k2, nk - 1);
        i8_dma4(a.xs + (long long)min(m0 + r, M - 1) * NG + blk,
                sbase + (uint32_t)(G::AS_OFF + (k2 * BM + (wave & 1) * 64) * 4));
      }
    };
    dma_stage(0, 0);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
      dma_stage(st + 1, (st + 1) & 1);
      if (2 * st + kg < nk) compute(st & 1);
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      __syncthreads();
    }
  } else if constexpr (NS == 1) {
    Regs rg0, rg1;
    fetch(rg0, 0);
    store(rg0, 0);
    fetch(rg1, 1);
    fetch(rg0, 2);
    __syncthreads();
    // next: the registers holding stage st+1, stored now and refilled with stage st+3
    auto iter = [&](int st, Regs& next) {
      if (2 * st + kg < nk) compute(st & 1);
      store(next, (st + 1) & 1);
      fetch(next, st + 3);
      __syncthreads();
    };
    int st = 0;
    for (; st + 1 < nst; st += 2) {
      iter(st, rg1);
      iter(st + 1, rg0);
    }
    if (st < nst) iter(st, rg1);
  } else {
    Regs rg;
    fetch(rg, 0);
    store(rg, 0);
    fetch(rg, 1);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
      if (2 * st + kg < nk) compute(st & 1);
      store(rg, (st + 1) & 1);
      fetch(rg, st + 2);
      __syncthreads();
    }
  }

  // ---------------- K groups: group 0 + group 1 (fixed order), one set at a time ----------------
  constexpr int WT = 2 * WNW;  // wave tiles (wm, wn) of one K group
  const int wt = wave % WT;
  float* red = (float*)lds + wt * (64 * 64) + lane;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if (s > 0) __syncthreads();  // group 0 has read the previous set
    if (kg == 1) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) red[((rb * 4 + t) * 4 + r) * 64] = acc[s][rb][t][r];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[s][rb][t][r] += red[((rb * 4 + t) * 4 + r) * 64];
    }
  }
  if (S > 1) {
    // Split-K: group 0's partial tile of each weight set (wave w: the float4 (rb, t) of
    // every lane at byte ((rb * 4 + t) * 64 + lane) * 16 of its 16 KB slot, slots
    // [split][set][wave]) goes out through device-coherent stores; each workgroup's
    // stores complete before it counts its arrival, and the last to arrive sums the
    // partials in split order.
    __shared__ int s_last;
    constexpr unsigned kSlot = 64u * 64u * 4u;
    const __amdgpu_buffer_rsrc_t rs =
        part_rsrc(a.part + (long long)tile * S * NS * WT * (64 * 64), (unsigned)(S * NS * WT) * kSlot);
    const unsigned lane_off = (unsigned)lane * 16u;
    if (kg == 0) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const unsigned base = (unsigned)((split * NS + s) * WT + wt) * kSlot + lane_off;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
          for (int t = 0; t < 4; ++t) st_coherent(acc[s][rb][t], rs, base + (unsigned)(rb * 4 + t) * 1024u);
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // every partial store of this wave has completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(a.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == (unsigned)(S - 1);
      if (last) __hip_atomic_store(a.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last || kg != 0) return;  // uniform over each wave
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    for (int sp = 0; sp < S; ++sp) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const unsigned base = (unsigned)((sp * NS + s) * WT + wt) * kSlot + lane_off;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const f32x4 v = ld_coherent(rs, base + (unsigned)(rb * 4 + t) * 1024u);
            acc[s][rb][t] = (sp == 0) ? v : acc[s][rb][t] + v;
          }
      }
    }
  }
  if (kg != 0) return;

  // ---------------- epilogue ----------------
  const int col = ncol0 + cb;  // within the matrix
  if (col >= n) return;
  float cs[NS][4];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if constexpr (W4) {
      cs[s][0] = cs[s][1] = cs[s][2] = cs[s][3] = 1.0f;
    } else {
      cvt_scale4(csraw[s], a.sdt, cs[s]);
    }
  }
  if constexpr (EPI == EPI_STORE) {
    // column scale (W8), residual, 16-bit store.  The output type and the residual
    // are uniform: branch once, outside the per-value code.  Row addresses: uniform
    // base of the wave's first row, per-lane offset, uniform multiple of the stride.
    const int ocol = sg.col0 + col;
    const int r0 = m0 + wm * 64;
    const int nrows = M - r0;
    uint16_t* const obase = (uint16_t*)a.out + (long long)r0 * a.ldo;
    const uint16_t* const rbase = a.res ? (const uint16_t*)a.res + (long long)r0 * a.ldr : nullptr;
    const long long oofs = (long long)(4 * g) * a.ldo + ocol, rofs = (long long)(4 * g) * a.ldr + ocol;
    auto store_all = [&](auto bf16, auto with_res) {
      constexpr bool BF = decltype(bf16)::value, RES = decltype(with_res)::value;
      auto cvt2 = [](float v0, float v1) -> uint32_t {
        if constexpr (BF) return (uint32_t)f32_to_bf16(v0) | ((uint32_t)f32_to_bf16(v1) << 16);
        else return bitcast<uint32_t>(__builtin_convertvector((float __attribute__((ext_vector_type(2)))){v0, v1}, f16x2));
      };
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (rb * 16 + 4 * g + r >= nrows) continue;
          const int ur = rb * 16 + r;
          // column scale and residual in one rounding (fmaf), the product alone
          // without a residual: the skinny kernel's epilogue rounds the same way
          float y[4];
          if constexpr (RES) {
            const u32x2 rv = *(const u32x2*)(rbase + (long long)ur * a.ldr + rofs);
            const uint32_t rw[2] = {rv.x, rv.y};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const uint16_t hh = (uint16_t)(rw[t >> 1] >> (16 * (t & 1)));
              y[t] = fmaf(acc[0][rb][t][r], cs[0][t], BF ? bf16_to_f32(hh) : (float)bitcast<_Float16>(hh));
            }
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) y[t] = acc[0][rb][t][r] * cs[0][t];
          }
          u32x2 o;
          o.x = cvt2(y[0], y[1]);
          o.y = cvt2(y[2], y[3]);
          *(u32x2*)(obase + (long long)ur * a.ldo + oofs) = o;
        }
    };
    using T = std::true_type;
    using F = std::false_type;
    if (a.odt == DT_BF16) {
      if (a.res) store_all(T{}, T{});
      else store_all(T{}, F{});
    } else {
      if (a.res) store_all(F{}, T{});
      else store_all(F{}, F{});
    }
  } else {
    // h = silu(g) * u; bf16 store, or bf16 round trip and per-64-column int8 quant.
    // A row's 64 columns of this wave tile are the 16 lanes of its row group (4
    // columns each): the amax reduces over those lanes.
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + rb * 16 + 4 * g + r;
        float h[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) h[t] = silu(acc[0][rb][t][r] * cs[0][t]) * (acc[1][rb][t][r] * cs[1][t]);
        if constexpr (EPI == EPI_GATEUP) {
          if (row < M) {
            u32x2 o;
            o.x = (uint32_t)f32_to_bf16(h[0]) | ((uint32_t)f32_to_bf16(h[1]) << 16);
            o.y = (uint32_t)f32_to_bf16(h[2]) | ((uint32_t)f32_to_bf16(h[3]) << 16);
            *(u32x2*)((uint16_t*)a.out + (long long)row * a.ncols + col) = o;
          }
        } else {
          float am = 0.0f;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            h[t] = bf16_to_f32(f32_to_bf16(h[t]));  // bf16 round trip (kernels/gemm.py:198-200)
            am = fmaxf(am, fabsf(h[t]));
          }
#pragma unroll
          for (int m = 1; m < 16; m <<= 1) am = fmaxf(am, __shfl_xor(am, m));
          const float sc = fmaxf(am / 127.0f, 1e-8f);
          if (row < M) {
            uint32_t qw = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) qw |= ((uint32_t)(round_i8(h[t] / sc) & 0xFF)) << (8 * t);
            *(uint32_t*)(a.oq + (long long)row * a.ncols + col) = qw;
            if (j == 0) a.os[(long long)row * (a.ncols / 64) + col / 64] = sc;
          }
        }
      }
  }
}

template <int WK, bool HZ, int EPI, int WNW>
static hipError_t launch_i8_t(const SkArgs& a, int tiles, hipStream_t st) {
  using G = Gi8<WK, (EPI == EPI_STORE) ? 1 : 2, WNW>;
  static bool attr_set = false;  // benign race: every caller sets the same value
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute((const void*)prefill_i8_kernel<WK, HZ, EPI, WNW>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((prefill_i8_kernel<WK, HZ, EPI, WNW>), dim3(tiles), dim3(G::THREADS), (size_t)G::LDS, st, a);
  return hipGetLastError();
}

template <int EPI>
static hipError_t launch_i8_e(const SkArgs& a, int wk, bool hz, int tiles, hipStream_t st) {
  if (wk == WK_W8) return launch_i8_t<WK_W8, false, EPI, 2>(a, tiles, st);
  if (hz) return launch_i8_t<WK_W4, true, EPI, 2>(a, tiles, st);
  return launch_i8_t<WK_W4, false, EPI, 2>(a, tiles, st);
}

// Column tile of a call: 128, or 64 (the 4-wave DMA tile, three workgroups per CU) for
// W8 store calls with QLIN_I8_DMA=1 (same bits).  The DMA tile is not the default: timed
// alone, the 6144-deep down projection at M = 512 over 4 splits ran 28.8 us on it against
// 30.5, but inside a layer's sequence of calls 32.7 against about 31, and proj3 (one
// split) was slower on it either way.
static int i8_bn(int wk, int epi, int splits) {
  (void)splits;
  if (wk != WK_W8 || epi != EPI_STORE) return 128;
  const char* e = getenv("QLIN_I8_DMA");
  return (e && atoi(e) == 1) ? 64 : 128;
}

// Whether the tiled kernel covers a call; the 128-column condition holds for both tiles
// (the DMA tile is only forced where it covers the call).
bool prefill_i8_ok(const SkArgs& a, int wk, int epi) {
  if (a.M <= 16 || a.K % 64 != 0 || ((uintptr_t)a.x & 15) != 0) return false;
  // the copies address activations, their scales and each weight matrix with buffer
  // offsets computed in 31 bits
  if ((long long)a.M * a.K >= (1LL << 31) || (long long)a.M * (a.K / 64) * 4 >= (1LL << 31)) return false;
  for (int s = 0; s < a.nseg; ++s)
    if ((long long)a.K * a.seg[s].n >= (1LL << 31)) return false;
  if (wk == WK_W4 && a.group < 64) return false;
  const char* e = getenv("QLIN_I8_DMA");
  const int bn = (e && atoi(e) == 1 && wk == WK_W8 && epi == EPI_STORE) ? 64 : 128;
  const int nsets = (epi == EPI_STORE) ? a.nseg : 1;  // gate/up: one column range, two weight sets
  for (int s = 0; s < nsets; ++s)
    if (a.seg[s].n % bn != 0) return false;
  return true;
}

hipError_t launch_prefill_i8(SkArgs a, int wk, bool hz, int epi, hipStream_t st) {
  const int bn = i8_bn(wk, epi, a.splits);
  int tn = 0;
  if (epi == EPI_STORE) {
    for (int s = 0; s < a.nseg; ++s) {
      a.seg[s].tile0 = tn;
      tn += a.seg[s].n / bn;
    }
  } else {
    a.seg[0].tile0 = a.seg[1].tile0 = 0;
    tn = a.seg[0].n / bn;
  }
  a.ntiles = tn;
  if (a.splits < 1) a.splits = 1;
  const int tiles = ((a.M + BM - 1) / BM) * tn * a.splits;
  // Tile order: each XCD runs one contiguous eighth of it, going down gm row tiles
  // before the next column tile; gm minimises what a run reads into its XCD's L2: rows
  // x (128 x K int8 activations) + columns x (the weights of 128 columns, every set).
  // QLIN_I8_GM overrides it (0: groups of 8 row tiles, workgroups in launch order).
  const char* eg = getenv("QLIN_I8_GM");
  if (eg && *eg) {
    a.gm = atoi(eg) > 0 ? atoi(eg) : 0;
  } else {
    const long long tm = (a.M + BM - 1) / BM;
    const long long run = std::max<long long>(1, (tm * tn + 7) / 8);
    const double arow = (double)BM * a.K, wcol = (double)a.K * bn * (wk == WK_W4 ? 0.5 : 1.0) * (epi == EPI_STORE ? 1 : 2);
    double best_c = 0.0;
    for (int gm = 1; gm <= 64; gm *= 2) {
      const long long h = std::min<long long>(gm, tm);
      const long long rows = std::min(h, run), cols = (run + h - 1) / h;
      const double c = (double)rows * arow + (double)cols * wcol;
      if (gm == 1 || c < best_c) best_c = c, a.gm = gm;
      if (gm >= tm) break;
    }
  }
  switch (epi) {
    case EPI_STORE:
      if (bn == 64) return launch_i8_t<WK_W8, false, EPI_STORE, 1>(a, tiles, st);
      return launch_i8_e<EPI_STORE>(a, wk, hz, tiles, st);
    case EPI_GATEUP: return launch_i8_e<EPI_GATEUP>(a, wk, hz, tiles, st);
    default: return launch_i8_e<EPI_GATEUP_Q>(a, wk, hz, tiles, st);
  }
}

}  // namespace qlin
