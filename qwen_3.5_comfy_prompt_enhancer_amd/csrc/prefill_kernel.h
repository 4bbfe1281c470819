// Prefill GEMM for fp16 activations with more than 16 rows, gfx950: the kernel
// template, included by prefill.hip (W8 and the dispatch) and by one source per W4
// scale dtype (prefill_w4_f16.hip, prefill_w4_bf16.hip, prefill_w4_f32.hip).
//
// out[M,N] = x[M,K] . dequant(W)[K,N] (+ residual), W in the engine layouts (int8
// [K,N] with per-column scales, or packed nibbles [K/2,N] with per-group scales and
// optional zeros).
//
//   * Workgroup tile BM x BN = (128 WM) x (64 WN) computed by WM x WN waves, each
//     owning a 128 x 64 output tile = 8 x 4 blocks of v_mfma_f32_16x16x32_f16 with
//     fp32 accumulation.  Tall wave tiles make every dequantized weight operand feed
//     8 MFMAs.  With 8 waves (256 x 256) two waves share each SIMD, so one wave's
//     dequantization and LDS traffic issue while the other's MFMAs run.  With KG = 2
//     wave groups, each group computes one of the two 32-wide substeps of every K
//     tile and the groups' accumulators are added through LDS at the end: twice the
//     waves for the same tile, for shapes with few tiles.
//   * Global -> LDS copies are 16-byte LDS DMA (global_load_lds_dwordx4): no VGPR
//     staging.  Activation tiles land as 128-byte rows of 64 halves with the 16-byte
//     chunk c of row r stored at position c ^ ((r >> 1) & 7), which makes the MFMA
//     operand reads (ds_read_b128, rows j of 16, K chunks by lane group) free of bank
//     conflicts for gfx950's read phases (lane blocks 0/3, 1/2, 4/7, 5/6 of 8 lanes
//     share a cycle).  Weight tiles land as raw bytes, in blocks of 8 rows of 128
//     bytes padded to 1088 bytes, so the four lane groups of a ds_read_b32 hit four
//     disjoint bank quarters.
//   * Weights are dequantized per MFMA operand in registers (v_perm_b32 exponent
//     trick): lane (g, j) reads 4 adjacent columns of its 8 K rows and builds the B
//     operands of 4 MFMAs; MFMA column j of instruction t is output column 4j + t.
//     W8 values are exact integers in fp16 and the column scale multiplies the fp32
//     result; W4 (nibble - z) is exact and the group scale (times 2^8) is folded into the fp16
//     weight (one fp16 rounding per weight).  W4 kernels are built per scale dtype SD,
//     so the scale conversion in the MFMA loop is one or two instructions with no
//     branch.
//   * NSTAGE K tiles of 64 in an LDS ring with one barrier per tile.  Before it, a
//     wave waits (vmcnt) for the copy of the next tile it needs; after it, the stage
//     every wave has finished reading receives the copy of the tile NSTAGE ahead.
//     The DMA is issued from inline assembly so the compiler's wait insertion, which
//     would otherwise drain every in-flight copy before each LDS read, leaves the
//     ring alone; the waits are explicit and count this kernel's own copies only.
//   * Split-K: `splits` workgroups share an output tile, each over a contiguous
//     range of K tiles.  Each stores its fp32 partial tile (16-byte device-coherent
//     stores, readable from every XCD), waits for the stores, and bumps the tile's
//     arrival counter; the last to arrive sums the partials in split order (all
//     loads of one split in flight together), resets the counter and runs the
//     epilogue.  The sum order is fixed, so results are deterministic.
//   * Balanced schedule (its own instantiation): when the tiles would leave CUs idle
//     for a whole round, each workgroup takes the same run of (tile, K tile) units,
//     crossing tile boundaries; a tile shared by two workgroups is finished by one of
//     them, which adds the other's fp32 partial (one flag bit per piece, no waiting).
//   * The K order of every output element is fixed (tiles in order, two 32-wide
//     substeps each, partials summed in split order), so a row's result depends on
//     the split count and the number of wave groups but not on M or the tile size.
#pragma once

#include "qlin_dev.h"
#include "qlin_internal.h"

namespace qlin {

namespace {

constexpr int BK = 64;           // K per stage
constexpr int GROUP_M = 8;       // tile order: 8 row tiles per group

template <int WK, int WM, int WN, int KG, int NS = 3>
struct Geo {
  static constexpr int NSTAGE = NS;  // K tiles in the LDS ring
  static constexpr int BM = 128 * WM;
  static constexpr int BN = 64 * WN;  // WN even: the weight tile is stored in 128-column halves
  static constexpr int WAVES = WM * WN * KG;  // KG wave groups split each K tile's substeps
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int A_BYTES = BM * 128;
  static constexpr int HB_BLOCKS = (WK == WK_W8) ? 8 : 4;  // 64 int8 rows or 32 packed rows per half
  static constexpr int B_BLOCKS = HB_BLOCKS * (BN / 128);
  // LDS bytes of one 8-row weight block: rows of 128 B + pad.  A lane group g of a
  // wave reads block g (W8) or row pair g & 1 of block g >> 1 (W4); the pads put the
  // four lane groups on four different 16-bank quarters of the 64 banks, and the
  // two groups of each half-wave on different halves of 32 banks.
  static constexpr int WB = (WK == WK_W8) ? 1024 + 64 : 1024 + 128;
  static constexpr int B_BYTES = B_BLOCKS * WB;
  static constexpr int SC_BYTES = (WK == WK_W8) ? 0 : WAVES * 1024;  // W4 scales + zeros
  static constexpr int STAGE = A_BYTES + B_BYTES + SC_BYTES;
  static constexpr int A_DMA = (BM / 8) / WAVES;  // 1 KB activation blocks per wave
  static constexpr int B_DMA = B_BLOCKS / WAVES;  // weight blocks per wave
  static constexpr int DMA = A_DMA + B_DMA + (WK == WK_W4 ? 1 : 0);  // copies per wave per stage
  static constexpr int OCC = (WAVES >= 8) ? 2 : 1;                    // waves per SIMD
  static_assert(WN % 2 == 0 && (BM / 8) % WAVES == 0 && B_BLOCKS % WAVES == 0, "tile geometry");
  static_assert(KG == 1 || KG == 2, "one or two K groups");
  static_assert(KG == 1 || NSTAGE * STAGE >= WM * WN * 128 * 64 * 4, "LDS for the K-group reduction");
  static_assert(WK == WK_W8 || 10 * BN <= SC_BYTES, "W4 scale region");
};

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4
// left at its maximum, lgkmcnt 11:8 = 0).
constexpr int wait_vm_lgkm0(int n) { return (n & 15) | (((n >> 4) & 3) << 14) | 0x70; }

__device__ __forceinline__ uint32_t rfl(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ const void* rfl_ptr(const void* p) {
  const uint64_t v = (uint64_t)p;
  const uint64_t lo = rfl((uint32_t)v), hi = rfl((uint32_t)(v >> 32));
  return (const void*)((hi << 32) | lo);
}

// 16-byte LDS DMA: lane i copies 16 bytes from sbase + voff to LDS m0 + 16 i.
__device__ __forceinline__ void dma_s(const void* sbase, uint32_t voff, uint32_t m0) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

// Same with a full 64-bit address per lane.
__device__ __forceinline__ void dma_v(const void* vaddr, uint32_t m0) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(vaddr), "{m0}"(m0) : "memory");
}

// W4 group scales enter the fp16 weight values multiplied by 2^8 (exact), and the
// epilogue multiplies the fp32 result by 2^-8 (exact): the products (nibble - z) * s * 2^8
// are normal fp16 numbers for scales in [2^-22, 17] (|nibble - z| <= 15), where an
// unshifted scale below 2^-14 would lose precision as a subnormal.
constexpr float kW4ScaleShift = 256.0f;

// Group scale t of a lane's 4 columns -> fp16 scale * 2^8.  w holds the raw scales:
// 4 fp32 words, or 2 words of two 16-bit scales (column 2i in the low half).  Every
// form is exact up to the one rounding to fp16 (the fp16 product by 2^8 is exact
// unless it overflows, which rounds as the fp32 route would).
template <int SD>
__device__ __forceinline__ _Float16 scale_f16(const uint32_t (&w)[4], int t) {
  if constexpr (SD == DT_F32) {
    return (_Float16)(bitcast<float>(w[t]) * kW4ScaleShift);
  } else if constexpr (SD == DT_BF16) {
    const uint32_t v = w[t >> 1];
    return (_Float16)(bitcast<float>((t & 1) ? (v & 0xFFFF0000u) : (v << 16)) * kW4ScaleShift);
  } else {
    const f16x2 p = bitcast<f16x2>(w[t >> 1]) * f16x2{(_Float16)kW4ScaleShift, (_Float16)kW4ScaleShift};
    return p[t & 1];
  }
}

}  // namespace

// SD: the W4 scale dtype (DT_F16, DT_BF16 or DT_F32); 0 for W8, whose column scales
// are read once per tile, in the epilogue, in any dtype.
template <int WK, bool HZ, int SD, int WM, int WN, int KG, int NS, bool BAL>
__global__ __launch_bounds__(64 * WM * WN * KG)
__attribute__((amdgpu_waves_per_eu(Geo<WK, WM, WN, KG, NS>::OCC, Geo<WK, WM, WN, KG, NS>::OCC)))
void prefill_kernel(const TlArgs a) {
  using G = Geo<WK, WM, WN, KG, NS>;
  constexpr int NSTAGE = G::NSTAGE;
  constexpr int BN = G::BN;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;

  const int M = a.M, N = a.N, K = a.K;
  const int tiles_m = (M + G::BM - 1) / G::BM, tiles_n = (N + BN - 1) / BN;
  __shared__ int s_last;

  // One piece of work: K tiles kb .. kb + nk - 1 of output tile `tile`, shared by xs
  // workgroups (1: no exchange).  Split-K (pair = false): xs splits, partial slot
  // xslot, the last to arrive sums every slot in split order.  Balanced schedule
  // (pair = true): xs <= 2, slot 0 holds the piece that starts at K = 0, and one of
  // the two pieces finishes the tile, adding the other's partial to its own
  // accumulators.
  auto run = [&](const int tile, const int kb, const int nk, const int xs, const int xslot, const bool pair) {
  // In the balanced schedule (BAL) the thread index goes through an empty asm so that
  // nothing derived from it is hoisted out of the loop over pieces (which would keep
  // those values live across every piece and spill).
  int tid = (int)threadIdx.x;
  if constexpr (BAL) asm volatile("" : "+v"(tid));
  const int wave = (int)rfl((uint32_t)tid >> 6), lane = tid & 63;  // wave index in an SGPR
  const int j = lane & 15, g = lane >> 4;
  const int kg = wave / (WM * WN);  // K group: with KG = 2, group kg computes substep kg
  const int wl = wave % (WM * WN);  // wave within its group
  const int wm = wl / WN, wn = wl % WN;
  // grouped tile order: runs of consecutive tiles cover gm row tiles x a few column
  // tiles, so the workgroups of one XCD share activation and weight tiles in its L2
  // (the balanced schedule numbers tiles row by row: its workgroups already run
  // consecutive tiles on one XCD)
  const int pid = tile;
  const int gm = a.gm > 0 ? a.gm : GROUP_M;
  const int per_group = gm * tiles_n;
  const int first_m = (pid / per_group) * gm;
  const int gsize = min(tiles_m - first_m, gm);
  const int tm = pair ? pid / tiles_n : first_m + (pid % per_group) % gsize;
  const int tn = pair ? pid % tiles_n : (pid % per_group) / gsize;
  const int m0 = tm * G::BM, n0 = tn * BN;

  // activation copies: block q of this wave = rows 8 * blk .. +7; lane -> row
  // 8 blk + lane / 8, LDS position lane % 8 holding K chunk (position ^ swizzle)
  uint32_t offA[G::A_DMA];
#pragma unroll
  for (int q = 0; q < G::A_DMA; ++q) {
    const int r = 8 * (wave * G::A_DMA + q) + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int row = min(m0 + r, M - 1);  // rows past M read row M-1 and are never stored
    offA[q] = (uint32_t)(((long long)row * a.ldx + 8 * c) * 2);
  }
  // weight copies: block = 8 (packed) rows of 128 bytes of one 128-column half;
  // lane -> row, 16-byte chunk
  uint32_t offB[G::B_DMA];
#pragma unroll
  for (int q = 0; q < G::B_DMA; ++q) {
    const int blk = wave * G::B_DMA + q;
    const int half = blk / G::HB_BLOCKS, b = blk % G::HB_BLOCKS;
    const int s = lane >> 3;
    // W4 stores packed row 4h + i of a block at slot 2i + h, and the 16-byte chunks of
    // odd slots with their 64-byte halves swapped (chunk c at position c ^ 4), so the
    // two row pairs of a block sit 16 banks apart
    const int r = 8 * b + ((WK == WK_W8) ? s : 4 * (s & 1) + (s >> 1));
    const int chunk = (WK == WK_W8) ? (lane & 7) : (lane & 7) ^ ((s & 1) << 2);
    int col = n0 + 128 * half + 16 * chunk;
    col = (col < N) ? col : n0;  // chunks past N (N % 16 == 0) re-read a valid chunk
    offB[q] = (uint32_t)(r * N + col);
  }
  constexpr int ssz = (SD == DT_F32) ? 4 : 2;
  constexpr int SB = BN * ssz;  // bytes of one scale row of the tile
  // W4: this lane's 16 bytes of the scale/zero region, the same for every K tile:
  // kind 1 = scale row (sc_hi: of substep 1) at byte sc_in, kind 2 = zero row, 0 = none
  // (columns past N included)
  int sc_kind = 0, sc_hi = 0, sc_in = 0;
  // the group (a power of two in practice) as a shift, so the scale rows of a K tile
  // cost no division
  const bool g_pow2 = (a.group & (a.group - 1)) == 0;
  const int g_shift = __builtin_ctz((unsigned)a.group);
  if constexpr (WK == WK_W4) {
    const int o = wave * 1024 + 16 * lane;
    if (o < 2 * SB) {
      sc_hi = o >= SB;
      sc_in = o - sc_hi * SB;
      sc_kind = (n0 + sc_in / ssz < N) ? 1 : 0;
    } else if (HZ && o < 2 * SB + 2 * BN) {
      sc_hi = o - 2 * SB >= BN;
      sc_in = o - 2 * SB - sc_hi * BN;
      sc_kind = (n0 + sc_in < N) ? 2 : 0;
    }
  }

  auto issue = [&](int kt, int st) {
    const int k0 = kt * BK;
    const uint32_t base = lds0 + (uint32_t)(st * G::STAGE);
    const void* xa = rfl_ptr(a.x + k0);
#pragma unroll
    for (int q = 0; q < G::A_DMA; ++q) dma_s(xa, offA[q], rfl(base + (uint32_t)((wave * G::A_DMA + q) * 1024)));
    const void* wb = rfl_ptr(a.w + (long long)((WK == WK_W8) ? k0 : k0 / 2) * N);
#pragma unroll
    for (int q = 0; q < G::B_DMA; ++q)
      dma_s(wb, offB[q], rfl(base + (uint32_t)(G::A_BYTES + (wave * G::B_DMA + q) * G::WB)));
    if constexpr (WK == WK_W4) {
      // scale rows of K substeps 0 and 1 (the same row when the group spans the
      // tile), then zero rows; remaining lanes re-read a valid address.  Both
      // candidate addresses are formed and one is selected, with no branch.
      // (row bases and the substep-1 row step are uniform, kept in scalar registers)
      int gr0, gr1;
      if (g_pow2) {  // uniform
        gr0 = k0 >> g_shift, gr1 = (k0 + 32) >> g_shift;
      } else {
        gr0 = k0 / a.group, gr1 = (k0 + 32) / a.group;
      }
      const uint8_t* s0 = (const uint8_t*)rfl_ptr((const uint8_t*)a.s + ((long long)gr0 * N + n0) * ssz);
      const uint32_t dr = rfl((uint32_t)(gr1 - gr0) * (uint32_t)N);
      const void* p = sc_kind == 1 ? (const void*)(s0 + (sc_hi ? dr * ssz : 0u) + sc_in) : a.s;
      if constexpr (HZ) {
        const uint8_t* z0 = (const uint8_t*)rfl_ptr(a.z + (long long)gr0 * N + n0);
        p = sc_kind == 2 ? (const void*)(z0 + (sc_hi ? dr : 0u) + sc_in) : p;
      }
      dma_v(p, rfl(base + (uint32_t)(G::A_BYTES + G::B_BYTES + wave * 1024)));
    }
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int rb = 0; rb < 8; ++rb)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[rb][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Operands of one 32-wide K substep: 8 activation blocks, the raw weight dwords
  // (8 int8 rows or 4 packed rows of 4 columns) and, for W4, 4 scales and 4 zeros.
  struct Ops {
    f16x8 av[8];
    uint32_t d[8];
    uint32_t sv[4];
    uint32_t zv;
  };
  const int cc = wn * 64 + 4 * j;  // first of this lane's 4 columns within the tile
  // W8 column scales of the epilogue, loaded now (every wave, no branch) so their
  // latency hides behind the K loop; issued before the first copy, they only make
  // the first copy wait count cover one more (older) load
  u32x4 csraw = u32x4{0u, 0u, 0u, 0u};
  if constexpr (WK == WK_W8) csraw = ld_scale4_raw(a.s, a.sdt, min(n0 + cc, N - 4));
  // this lane's first weight byte in the tile's LDS blocks: W8 reads row i of block
  // 4 ks + g, W4 packed rows 4 (g & 1) + i (slot 2 i + (g & 1), halves swapped in odd
  // slots) of block 2 ks + (g >> 1)
  const int cb = (WK == WK_W8)
                     ? (wn >> 1) * G::HB_BLOCKS * G::WB + g * G::WB + (wn & 1) * 64 + 4 * j
                     : (wn >> 1) * G::HB_BLOCKS * G::WB + (g >> 1) * G::WB + (g & 1) * 128 +
                           (((wn & 1) ^ (g & 1)) * 64) + 4 * j;

  auto load_ops = [&](int st, int ks, Ops& o) {
    const uint8_t* sA = lds + st * G::STAGE;
    const uint8_t* sB = sA + G::A_BYTES;
    const uint8_t* sS = sB + G::B_BYTES;
#pragma unroll
    for (int rb = 0; rb < 8; ++rb) {
      const int row = wm * 128 + rb * 16 + j;
      o.av[rb] = *(const f16x8*)(sA + row * 128 + 16 * ((4 * ks + g) ^ (j >> 1)));
    }
    if constexpr (WK == WK_W8) {
#pragma unroll
      for (int i = 0; i < 8; ++i) o.d[i] = *(const uint32_t*)(sB + 4 * ks * G::WB + i * 128 + cb);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) o.d[i] = *(const uint32_t*)(sB + 2 * ks * G::WB + i * 256 + cb);
      // the raw scales of columns cc .. cc + 3
      if constexpr (SD == DT_F32) {
        const u32x4 v = *(const u32x4*)(sS + ks * SB + cc * 4);
        o.sv[0] = v.x, o.sv[1] = v.y, o.sv[2] = v.z, o.sv[3] = v.w;
      } else {
        const u32x2 v = *(const u32x2*)(sS + ks * SB + cc * 2);
        o.sv[0] = v.x, o.sv[1] = v.y, o.sv[2] = 0u, o.sv[3] = 0u;
      }
      o.zv = 0x08080808u;
      if constexpr (HZ) o.zv = *(const uint32_t*)(sS + 2 * SB + ks * BN + cc);
    }
  };

  // B operand of MFMA column t (output column 4j + t) from the raw weight dwords
  auto dequant = [&](const Ops& o, int t) -> f16x8 {
    u32x4 h;
    if constexpr (WK == WK_W8) {
      h = u32x4{w8_pair_f16(o.d[0], o.d[1], t), w8_pair_f16(o.d[2], o.d[3], t), w8_pair_f16(o.d[4], o.d[5], t),
                w8_pair_f16(o.d[6], o.d[7], t)};
    } else {
      const f16x2 bias = w4_bias((o.zv >> (8 * t)) & 0xFFu);
      const _Float16 sc = scale_f16<SD>(o.sv, t);
      const f16x2 s2 = f16x2{sc, sc};
      h.x = bitcast<uint32_t>(bitcast<f16x2>(w4_pair_f16(o.d[0], t, bias)) * s2);
      h.y = bitcast<uint32_t>(bitcast<f16x2>(w4_pair_f16(o.d[1], t, bias)) * s2);
      h.z = bitcast<uint32_t>(bitcast<f16x2>(w4_pair_f16(o.d[2], t, bias)) * s2);
      h.w = bitcast<uint32_t>(bitcast<f16x2>(w4_pair_f16(o.d[3], t, bias)) * s2);
    }
    return bitcast<f16x8>(h);
  };

  // column-outer order: the dequantization of column t + 1 overlaps the 8 MFMAs of
  // column t
  auto mma = [&](const Ops& o) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const f16x8 bv = dequant(o, t);
#pragma unroll
      for (int rb = 0; rb < 8; ++rb) acc[rb][t] = mfma_f16(o.av[rb], bv, acc[rb][t]);
    }
  };

  // Software pipeline, one barrier per K tile, placed between the two substeps:
  //   load substep-1 operands of tile kt  | MFMAs of tile kt substep 0
  //   wait: this wave's LDS reads returned, tile kt+1 copied; barrier
  //   DMA tile kt + NSTAGE into tile kt's stage (every wave has read it)
  //   load substep-0 operands of tile kt+1 | MFMAs of tile kt substep 1
  // LDS reads always overlap MFMAs, and a wave waiting at the barrier still has
  // its substep-0 MFMAs executing.
  auto schedule = [&]() {
    // dequantization of the first weight operand, then each MFMA with one LDS read
    // and two VALU slots
    __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);  // VALU
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
    }
  };

  // this piece's K tiles: kb .. kb + nk - 1
#pragma unroll
  for (int u = 0; u < NSTAGE - 1; ++u) issue(kb + min(u, nk - 1), u);
  // With one wave per SIMD (registers to spare) the loops below are unrolled by
  // NSTAGE so that every LDS stage index is a compile-time constant in the main
  // loop (no per-iteration address arithmetic); a runtime-indexed copy of the body
  // finishes the last nk % NSTAGE tiles.  Two waves per SIMD keep the rolled loop
  // (its 256 registers would not hold the unrolled one).
  constexpr int UNROLL = (G::OCC == 1) ? NSTAGE : 1;
  if constexpr (KG == 2) {
    // each wave computes one substep per tile: wait for the tile, barrier (which also
    // frees the stage computed in the previous iteration), copy ahead, compute
    auto body = [&](int kt, int st) {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0((NSTAGE - 2) * G::DMA));
      asm volatile("s_barrier" ::: "memory");
      issue(kb + min(kt + NSTAGE - 1, nk - 1), (st + NSTAGE - 1) % NSTAGE);
      __builtin_amdgcn_sched_barrier(0);
      Ops o;
      load_ops(st, kg, o);
      mma(o);
      __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // DS reads
      __builtin_amdgcn_sched_group_barrier(0x002, 12, 0);  // VALU
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
      }
    };
    int kt = 0;
    if constexpr (UNROLL > 1) {
      for (; kt + NSTAGE <= nk; kt += NSTAGE) {
#pragma unroll
        for (int u = 0; u < NSTAGE; ++u) body(kt + u, u);
      }
    }
    for (; kt < nk; ++kt) body(kt, kt % NSTAGE);
  } else {
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0((NSTAGE - 2) * G::DMA));  // first tile copied
    asm volatile("s_barrier" ::: "memory");
    issue(kb + min(NSTAGE - 1, nk - 1), NSTAGE - 1);
    Ops o0, o1;
    load_ops(0, 0, o0);
    auto body = [&](int kt, int st) {
      __builtin_amdgcn_sched_barrier(0);
      load_ops(st, 1, o1);
      mma(o0);
      schedule();
      __builtin_amdgcn_sched_barrier(0);
      // outstanding copies: tiles kt+1 .. kt+NSTAGE-1; wait for kt+1 (and for every
      // LDS read of stage st), then hand stage st to the copy of tile kt + NSTAGE
      // (past the last tile it re-reads tile nk-1 into a stage never read again)
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0((NSTAGE - 2) * G::DMA));
      asm volatile("s_barrier" ::: "memory");
      issue(kb + min(kt + NSTAGE, nk - 1), st);
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 1 < nk) load_ops((st + 1) % NSTAGE, 0, o0);
      mma(o1);
      schedule();
    };
    int kt = 0;
    if constexpr (UNROLL > 1) {
      for (; kt + NSTAGE <= nk; kt += NSTAGE) {
#pragma unroll
        for (int u = 0; u < NSTAGE; ++u) body(kt + u, u);
      }
    }
    for (; kt < nk; ++kt) body(kt, kt % NSTAGE);
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));  // no copy may outlive the workgroup

  if constexpr (KG == 2) {
    // K-group reduction through the (now idle) LDS stages: group 1 writes its
    // accumulators, group 0 adds them (fixed order: group 0 + group 1)
    float* red = (float*)lds + (long long)wl * (128 * 64) + lane;
    asm volatile("s_barrier" ::: "memory");  // every wave's last LDS read has returned
    if (kg == 1) {
#pragma unroll
      for (int rb = 0; rb < 8; ++rb)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) red[((rb * 4 + t) * 4 + r) * 64] = acc[rb][t][r];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int rb = 0; rb < 8; ++rb)
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[rb][t][r] += red[((rb * 4 + t) * 4 + r) * 64];
    }
  }

  if (xs > 1) {
    // Partial tile of this wave: the float4 (rb, t) of every lane at byte
    // ((rb * 4 + t) * 64 + lane) * 16 of the wave's slot, so each store or load
    // instruction moves 1 KiB contiguous.  Device-coherent (SC1) stores and loads;
    // each workgroup's stores complete before it signals.
    constexpr unsigned kSlot = 128u * 64u * 4u;  // bytes of one wave's partial tile
    const __amdgpu_buffer_rsrc_t rs =
        part_rsrc(a.part + (long long)tile * xs * G::WAVES * (128 * 64), (unsigned)(xs * G::WAVES) * kSlot);
    const unsigned lane_off = (unsigned)lane * 16u;
    auto store_partial = [&]() {
      if (kg == 0) {
        const unsigned base = (unsigned)(xslot * G::WAVES + wl) * kSlot + lane_off;
#pragma unroll
        for (int rb = 0; rb < 8; ++rb)
#pragma unroll
          for (int t = 0; t < 4; ++t) st_coherent(acc[rb][t], rs, base + (unsigned)(rb * 4 + t) * 1024u);
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0);  // every partial store of this wave has completed
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __syncthreads();
    };
    if (!pair) {
      store_partial();
      if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(a.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == (unsigned)(xs - 1);
        if (last) __hip_atomic_store(a.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = last;
      }
      __syncthreads();
      if (!s_last || kg != 0) return;  // uniform over each wave
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      // the last workgroup sums the partials in split order: 32 independent loads per split
      for (int sp = 0; sp < xs; ++sp) {
        const unsigned base = (unsigned)(sp * G::WAVES + wl) * kSlot + lane_off;
#pragma unroll
        for (int rb = 0; rb < 8; ++rb)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const f32x4 v = ld_coherent(rs, base + (unsigned)(rb * 4 + t) * 1024u);
            acc[rb][t] = (sp == 0) ? v : acc[rb][t] + v;
          }
      }
    } else {
      // Two pieces, one bit each in the tile's word: bit p = piece p's partial is
      // stored.  A piece that finds the other's bit set finishes the tile at once,
      // with no store of its own; otherwise it stores its partial, sets its bit and
      // finishes the tile only if the other's bit was set meanwhile.  The atomics on
      // the word are ordered, so exactly one piece finishes, and nothing waits.  The
      // finisher adds the other's partial to its own accumulators (the fp32 sum of
      // two values does not depend on their order, so neither does the result on
      // which piece finishes) and clears the word.
      const unsigned mine = 1u << xslot, other = 1u << (1 - xslot);
      if (tid == 0)
        s_last = (__hip_atomic_fetch_or(a.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & other) ? 1 : 0;
      __syncthreads();
      if (!s_last) {  // uniform
        store_partial();
        if (tid == 0)
          s_last =
              (__hip_atomic_fetch_or(a.cnt + tile, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & other) ? 1 : 0;
        __syncthreads();
        if (!s_last) return;
      }
      if (tid == 0) __hip_atomic_store(a.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (kg != 0) return;
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      const unsigned base = (unsigned)((1 - xslot) * G::WAVES + wl) * kSlot + lane_off;
#pragma unroll
      for (int rb = 0; rb < 8; ++rb)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[rb][t] = acc[rb][t] + ld_coherent(rs, base + (unsigned)(rb * 4 + t) * 1024u);
    }
  }

  // epilogue: lane holds rows 4g..4g+3 of each 16-row block, columns 4j..4j+3 of the
  // wave's 64 (MFMA t = column 4j + t)
  const int colb = n0 + wn * 64 + 4 * j;
  if (kg != 0 || colb >= N) return;
  float cs[4] = {1.f / kW4ScaleShift, 1.f / kW4ScaleShift, 1.f / kW4ScaleShift, 1.f / kW4ScaleShift};
  if constexpr (WK == WK_W8) cvt_scale4(csraw, a.sdt, cs);
  // The output type and the residual are uniform: branch once here, so each of the
  // 128 values of a lane costs a multiply, a conversion and (with a residual) an add.
  // Row addresses are a uniform base (the wave's first row) plus a per-lane offset
  // computed once, plus a uniform multiple of the row stride.
  const int r0 = m0 + wm * 128;       // first row of the wave
  const int nrows = M - r0;           // rows of the wave below M (may exceed 128)
  uint16_t* const obase = (uint16_t*)a.out + (long long)r0 * a.ldo;
  const uint16_t* const rbase = a.res ? (const uint16_t*)a.res + (long long)r0 * a.ldr : nullptr;
  const long long oofs = (long long)(4 * g) * a.ldo + colb, rofs = (long long)(4 * g) * a.ldr + colb;
  auto store_all = [&](auto bf16, auto with_res) {
    constexpr bool BF = decltype(bf16)::value, RES = decltype(with_res)::value;
    // two values -> one dword of 16-bit outputs (fp16: one packed RNE conversion)
    auto cvt2 = [](float v0, float v1) -> uint32_t {
      if constexpr (BF) return (uint32_t)f32_to_bf16(v0) | ((uint32_t)f32_to_bf16(v1) << 16);
      else return bitcast<uint32_t>(__builtin_convertvector((float __attribute__((ext_vector_type(2)))){v0, v1}, f16x2));
    };
#pragma unroll
    for (int rb = 0; rb < 8; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (rb * 16 + 4 * g + r >= nrows) continue;
        const int ur = rb * 16 + r;  // uniform part of the row
        float y[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) y[t] = acc[rb][t][r] * cs[t];
        if constexpr (RES) {
          const u32x2 rv = *(const u32x2*)(rbase + (long long)ur * a.ldr + rofs);
          const uint32_t rw[2] = {rv.x, rv.y};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint16_t h = (uint16_t)(rw[t >> 1] >> (16 * (t & 1)));
            y[t] += BF ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
          }
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
  };

  const int nkt = K / BK;  // K tiles of one output tile
  if constexpr (!BAL) {
    // one tile per workgroup, or `splits` workgroups per tile over equal K ranges.
    // Workgroups go to the 8 XCDs in turn; with a.gm set, XCD x's workgroups (b = x,
    // x + 8, ...) take one contiguous run of the order (a tile's splits included).
    const int S = a.splits;
    const int nk = nkt / S;
    const int b = (int)blockIdx.x, W = (int)gridDim.x;
    const int v = a.gm > 0 ? (b & 7) * (W >> 3) + min(b & 7, W & 7) + (b >> 3) : b;
    run(v / S, (v % S) * nk, nk, S, v % S, false);
    return;
  }
  // Balanced schedule: the (tile, K tile) units in order, a.sk consecutive units per
  // workgroup, so every workgroup does the same work when the tiles alone would leave
  // CUs idle.  The host only picks it when no tile spans more than two workgroups.
  // Workgroups go to the 8 XCDs in turn; with a multiple of 8 of them, workgroup b
  // takes range (b % 8) * (W / 8) + b / 8, so each XCD runs one contiguous eighth of
  // the units (whole rows of tiles when there are 8 row tiles: one activation block
  // per XCD L2), and the two pieces of a tile run on the same XCD.
  const int total = tiles_m * tiles_n * nkt;
  const int W = (int)gridDim.x;
  const int v = (W % 8 == 0) ? ((int)blockIdx.x % 8) * (W / 8) + (int)blockIdx.x / 8 : (int)blockIdx.x;
  const int beg = v * a.sk, end = min(beg + a.sk, total);
  for (int pos = beg; pos < end;) {
    const int tile = pos / nkt, kb = pos - tile * nkt;
    const int ke = min(nkt, end - tile * nkt);
    const int c0 = tile * nkt / a.sk, c1 = (tile * nkt + nkt - 1) / a.sk;  // workgroups on the tile
    if (pos != beg) __syncthreads();  // the previous piece's LDS reads are done before new copies
    run(tile, kb, ke - kb, c1 - c0 + 1, kb == 0 ? 0 : 1, true);
    pos = tile * nkt + ke;
  }
}

template <int WK, bool HZ, int SD, int WM, int WN, int KG, int NS, bool BAL>
static hipError_t launch_prefill_t(const TlArgs& a, hipStream_t st) {
  using G = Geo<WK, WM, WN, KG, NS>;
  const long long tiles = (long long)((a.M + G::BM - 1) / G::BM) * ((a.N + G::BN - 1) / G::BN);
  const long long units = tiles * (a.K / BK);
  const int wgs = (int)(a.sk > 0 ? (units + a.sk - 1) / a.sk : tiles * a.splits);
  const size_t lds = (size_t)G::NSTAGE * G::STAGE;
  static bool attr_set = false;  // benign race: every caller sets the same value
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute((const void*)prefill_kernel<WK, HZ, SD, WM, WN, KG, NS, BAL>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((prefill_kernel<WK, HZ, SD, WM, WN, KG, NS, BAL>), dim3(wgs), dim3(G::THREADS), lds, st, a);
  return hipGetLastError();
}


// One plan shape of one weight kind / zeros / scale dtype; the balanced schedule is
// its own instantiation, so the other plans compile as they would without it.
template <int WK, bool HZ, int SD>
static hipError_t launch_prefill_kind(const TlArgs& a, int shape, hipStream_t st) {
  const bool bal = a.sk > 0;
  switch (shape) {
    case PF_128x128:
      return bal ? launch_prefill_t<WK, HZ, SD, 1, 2, 1, 3, true>(a, st) : launch_prefill_t<WK, HZ, SD, 1, 2, 1, 3, false>(a, st);
    case PF_128x128_K2:
      return bal ? launch_prefill_t<WK, HZ, SD, 1, 2, 2, 3, true>(a, st) : launch_prefill_t<WK, HZ, SD, 1, 2, 2, 3, false>(a, st);
    case PF_256x256:
      return bal ? launch_prefill_t<WK, HZ, SD, 2, 4, 1, 3, true>(a, st) : launch_prefill_t<WK, HZ, SD, 2, 4, 1, 3, false>(a, st);
    default:
      return hipErrorInvalidValue;
  }
}

// W4 launchers, one source file each (scale dtype fp16, bf16, fp32)
hipError_t launch_prefill_w4_f16(const TlArgs& a, bool hz, int shape, hipStream_t st);
hipError_t launch_prefill_w4_bf16(const TlArgs& a, bool hz, int shape, hipStream_t st);
hipError_t launch_prefill_w4_f32(const TlArgs& a, bool hz, int shape, hipStream_t st);

}  // namespace qlin
