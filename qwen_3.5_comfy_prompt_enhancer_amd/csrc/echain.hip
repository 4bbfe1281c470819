// Engine decode chain, gfx950: the engine-signature linears of a decode step (int8
// activations with one fp32 scale per 64 columns, W8 or W4 weights) and the activation
// producers between them, as work units of ONE persistent launch with dependency
// levels -- or the units of a single call as a plain grid.
//
// The reference's decode step launches a producer (kernels/norm.py) and a linear
// (kernels/gemm.py, kernels/w4.py) per projection, about a hundred launches per token,
// and names whole-step capture or a decode megakernel as its next step
// (ENGINEERING.md:383-399).  Between two mixer kernels (attention / delta rule) the
// engine's calls form a dependent sequence (engine.py:236-279, 265-268, 272-279,
// 218-226):
//   norm_gated_quant | gate_mul_quant -> o-projection gemm_i8 (+ hidden, in place)
//   -> rmsnorm_quant -> mlp_gate_up_quant -> down gemm_i8 (+ hidden, in place)
//   -> rmsnorm_quant (next layer) -> proj3
// A chain runs that sequence as jobs: a linear job reads int8 codes + scales from
// memory, or makes them with its producer in each unit's prologue (the producer's
// inputs may be written by an earlier level of the same launch: the row statistics of
// rmsnorm are computed by every unit that needs them, so a producer never costs a
// level of its own).
//
//   * Work unit = (job, 128-column tile, weight set, K split): 4 waves, each folding
//     `wblk` consecutive 64-wide blocks.  The unit length depends on (K, N, sets) only,
//     never on M, on the level sizes or on the chain around the job, so a job gives the
//     same bits in every chain and as a single call (the engine-signature entry points
//     with at most 8 rows run their units through this same kernel), and row m of an
//     M-row call equals an M = 1 call bit for bit.
//   * Per 64-wide block one v_mfma_i32_16x16x64_i8 per output column gives the exact
//     int32 dot, started from an inline zero, then `acc = fma(float(dot), a_s, acc)`
//     in fp32 (kernels/gemm.py:43-45); W4 nibbles enter as int8 16 * (n - 8) and fold
//     against a_s * b_s[group] / 16, explicit zeros add (8 - z) * sum(a)
//     (kernels/w4.py:64-104).  Waves are summed in LDS in wave order, K splits in
//     split order (device-coherent partials), then the W8 column scale and the
//     residual in one fmaf, or the gate/up epilogue silu(g) * u -> bf16 -> per-64
//     max(amax / 127, 1e-8) -> round half away from zero (gemm.py:195-211).  gate and
//     up are separate units of one tile.  In a single call the tile's last arrival at
//     a counter runs the epilogue; in the chain the tile's last unit does, polling its
//     partners' slots (unit_finish).
//   * Activations: each unit stages its rows' codes and scales of its K range in LDS
//     (device-coherent loads, or the producer, producers.h pro_block<true>), after its
//     dependency wait; its weights come through a register ring of 2 blocks per wave
//     issued before the wait (in the chain: right after the previous unit's exchange
//     and epilogue, so that they stream while the workgroup waits).
//   * Scheduling (persistent form): 64 queues hand out units in increasing order, and a
//     unit waits only for units of lower levels, through a flag per level that the
//     level's last tile sets (bounded polls; a wait that gives up sets an error word),
//     so every wait ends whether or not all workgroups are resident.  The last
//     workgroup to leave resets the queues, counts and flags.
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/qlin.h"
#include "producers.h"
#include "qlin_dev.h"
#include "qlin_internal.h"

#define QL_TRY_E(expr)          \
  do {                          \
    const int rc_ = (expr);     \
    if (rc_ != QLIN_OK) return rc_; \
  } while (0)

namespace qlin {
namespace {

constexpr int EW = 4;                // waves per unit
constexpr int ET = 64 * EW;
constexpr int TNC = 128;             // columns per tile: 16 lanes x 8 columns
constexpr int TNP = TNC + 4;         // padded LDS row of the wave sums
constexpr int EMAXM = 8;             // rows (the engine's decode batch limit, engine.py:392)
constexpr int RB = 2;                // 64-wide blocks a wave has in flight (register ring)
constexpr int KU_MAX = 2048;         // longest unit K range (its codes are staged in LDS)
constexpr int LDQ = KU_MAX + 16;     // LDS code row stride (16 bytes stagger the rows over banks)
constexpr int kSpinLimit = 1 << 22;  // polls of a dependency before giving up
constexpr int kWaitVm0 = 0x0F70;     // s_waitcnt vmcnt(0)
constexpr int kQueues = 64;             // unit queues, one counter per 128-byte line
constexpr int kLevel0 = 32 * (kQueues + 1);
constexpr int kPlanSlots = 768;      // workgroups the unit plan is sized for (3 per CU x 256 CUs; a fixed
                                     // constant, so a job's K order never depends on the launch)
constexpr int kLongFactor = 2;
constexpr int kEPre = 4;             // producer: row chunks a lane loads ahead (all of a 2048-wide row)

enum EEpi { EE_STORE = 0, EE_GATEUP = 1, EE_GATEUP_Q = 2 };

// Device descriptor of one job.
struct alignas(16) EJob {
  const int8_t* aq;      // codes [M][K] (no producer)
  const float* as;       // scales [M][K/64]
  const uint8_t* w[2];   // weight sets (set 1: gate/up's up)
  const void* s[2];
  const uint8_t* z[2];   // W4 zeros or nullptr
  void* out;             // 16-bit [M][ldo] (EE_STORE, EE_GATEUP)
  const void* res;       // EE_STORE residual or nullptr (may alias out)
  int8_t* oq;            // EE_GATEUP_Q codes [M][N]
  float* os;             //   and scales [M][N/64]
  long long ldo, ldr;
  long long part;        // first float of the job's partials (plan or workspace)
  ProArgs pro;           // kind PRO_NONE: activations from aq / as
  int K, N, group, sdt, odt, epi, nsets, hz;
  int ntiles, splits, wblk, unit0, cnt0, level, emit, xch;
};

// Header of a chain plan (device memory).
struct alignas(16) EHdr {
  int magic, nunits, njobs, nlevels;
  int M, err, w4, err_run;   // err: the last finished launch (0 / 1); err_run: the running one
  long long jobs_off, unit_off, need_off, cnt_off, flag_off, part_off, bytes;
};
constexpr int kMagic = 0x71656331;  // "qec1"

// Arguments of the single-call form: the jobs by value, split-K scratch in the workspace.
struct ECallArgs {
  EJob jobs[3];
  int njobs, M, nunits, pad;
  float* part;
  unsigned* cnt;
};

struct ESh {
  float red[EW * EMAXM * TNP];         // per-wave sums [wave][row][column]
  uint8_t q[EMAXM * LDQ];              // the unit's codes [row][K range]
  float s[(KU_MAX / 64) * 16];         // the unit's activation scales [block][row (16)]
  float lr[EMAXM];                     // producer: per-row inverse RMS
  float cs[2 * TNC];                   // the tile's W8 column scales [set][column]
  u32x2 rv[ET];                        // thread t's residual chunk
  int unit, unit2, flag;
};

// Register ring of one wave: RB blocks of weights (W8: 16 K rows x 8 columns; W4: 8
// packed rows), W4 group scales and zeros per block.
template <bool W4>
struct ERing {
  static constexpr int NR = W4 ? 8 : 16;
  uint32_t w[RB][NR][2];
  u32x4 sraw[W4 ? RB : 1][2];
  uint32_t zr[W4 ? RB : 1][2];
};

struct EPos {
  int job, tile, set, split;
};

// The thread index as a value the compiler cannot treat as loop-invariant: every use
// recomputes what it derives from it, where hoisting those values out of the
// persistent loop would keep dozens of registers live across it (and spill them).
__device__ __forceinline__ int etid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

__device__ __forceinline__ EPos unit_pos(const EJob& J, int jn, int u) {
  EPos p;
  p.job = jn;
  const int local = u - J.unit0;
  const int per = J.nsets * J.splits;
  p.tile = local / per;
  const int rem = local - p.tile * per;
  p.set = rem / J.splits;
  p.split = rem - p.set * J.splits;
  return p;
}

// The wave's first K row and its 64-wide blocks within the unit.
__device__ __forceinline__ void wave_blocks(const EJob& J, const EPos& P, int* k0, int* nblk) {
  const int wave = etid() >> 6;
  *k0 = (P.split * EW + wave) * J.wblk * 64;
  *nblk = max(0, min(J.wblk, (J.K - *k0) / 64));
}

template <bool W4>
__device__ __forceinline__ const uint8_t* set_w(const EJob& J, int set) {
  return set ? J.w[1] : J.w[0];
}

// What the ring loads of a unit need: its weight set and the wave's K range.  The
// persistent form computes it for the next unit while the current one runs.
struct ELoad {
  const uint8_t* w;
  const void* s;
  const uint8_t* z;
  int N, group, sdt, col0, k0, nblk;
};

__device__ __forceinline__ ELoad make_load(const EJob& J, const EPos& P) {
  ELoad L;
  L.w = P.set ? J.w[1] : J.w[0];
  L.s = P.set ? J.s[1] : J.s[0];
  L.z = P.set ? J.z[1] : J.z[0];
  L.N = J.N;
  L.group = J.group;
  L.sdt = J.sdt;
  L.col0 = P.tile * TNC;
  wave_blocks(J, P, &L.k0, &L.nblk);
  return L;
}

// Issues the loads of block b of the wave's range into ring slot `slot`.  Blocks past
// the range load the range's last block again (or block 0 of the matrix when the wave
// has none): every register of the slot is written.
template <bool W4>
__device__ __forceinline__ void load_block(const ELoad& L, int b, ERing<W4>& R, int slot) {
  constexpr int NR = ERing<W4>::NR;
  const int lane = etid() & 63, j = lane & 15, g = lane >> 4;
  const int N = L.N;
  const int col = L.col0 + j * 8;
  const int ccl = col < N ? col : 0;
  const int kb = L.nblk > 0 ? L.k0 + 64 * min(b, L.nblk - 1) : 0;
  const long long r0 = W4 ? (long long)(kb / 2 + 8 * g) : (long long)(kb + 16 * g);
  const uint8_t* base = L.w + r0 * N + ccl;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const u32x2 v = ld_global_nt<u32x2>(base + (long long)r * N);
    R.w[slot][r][0] = v.x;
    R.w[slot][r][1] = v.y;
  }
  if constexpr (W4) {
    const long long idx = (long long)(kb / L.group) * N + ccl;
    const bool f32 = L.sdt == DT_F32;
    const uint8_t* sb = (const uint8_t*)L.s + idx * (f32 ? 4 : 2);
    R.sraw[slot][0] = ld_global<u32x4>(sb);
    R.sraw[slot][1] = ld_global<u32x4>(sb + (f32 ? 16 : 0));
    const u32x2 zv = ld_global<u32x2>(L.z ? L.z + idx : sb);
    R.zr[slot][0] = zv.x;
    R.zr[slot][1] = zv.y;
  }
}

// Activation codes and scales of a unit (no producer), loaded device-coherently into
// registers: up to 4 16-byte pieces of codes and one scale per thread (M <= 8 rows,
// K range <= 2048).  Pieces past the range read zeros at an out-of-range offset.
struct EStage {
  u32x4 q[4];
  float s;
};

__device__ __forceinline__ void stage_issue(const EJob& J, int M, int kbase, int kuu, EStage& st) {
  const int tid = etid();
  const int K = J.K;
  const int per = kuu >> 4;  // 16-byte pieces per row
  const __amdgpu_buffer_rsrc_t qr = part_rsrc(J.aq, (unsigned)((long long)M * K));
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int i = tid + ET * c;
    const int row = i / per, pc = i - row * per;
    const unsigned off = (i < M * per) ? (unsigned)((long long)row * K + kbase + 16 * pc) : 0xFFFFFFF0u;
    st.q[c] = __builtin_amdgcn_raw_buffer_load_b128(qr, off, 0, kCpolSc1);
  }
  const int nb = kuu >> 6, ng = K >> 6;
  const __amdgpu_buffer_rsrc_t sr = part_rsrc(J.as, (unsigned)((long long)M * ng * 4));
  const int row = tid / max(nb, 1), b = tid - row * max(nb, 1);
  const unsigned soff = (tid < M * nb) ? (unsigned)(((long long)row * ng + (kbase >> 6) + b) * 4) : 0xFFFFFFF0u;
  st.s = bitcast<float>(__builtin_amdgcn_raw_buffer_load_b32(sr, soff, 0, kCpolSc1));
}

__device__ __forceinline__ void stage_store(int M, int kuu, const EStage& st, ESh& sh) {
  const int tid = etid();
  const int per = kuu >> 4;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int i = tid + ET * c;
    if (i < M * per) {
      const int row = i / per, pc = i - row * per;
      *(u32x4*)&sh.q[row * LDQ + 16 * pc] = st.q[c];
    }
  }
  const int nb = kuu >> 6;
  if (tid < M * nb) {
    const int row = tid / nb, b = tid - row * nb;
    sh.s[b * 16 + row] = st.s;
  }
}

// The A operand of block b (lane (j, g): row j, K bytes 16 g .. 16 g + 15 of the
// block; rows past M read row M - 1, whose MFMA rows are never used) and the
// activation scales of rows 4 g .. 4 g + 3 (zero past the wave's range: the fold then
// adds exactly 0).
__device__ __forceinline__ u32x4 a_operand(const ESh& sh, int M, int wave, int wblk, int nblk, int b) {
  const int lane = etid() & 63, j = lane & 15, g = lane >> 4;
  const int bb = nblk > 0 ? min(b, nblk - 1) : 0;
  return *(const u32x4*)&sh.q[min(j, M - 1) * LDQ + (wave * wblk + bb) * 64 + 16 * g];
}

__device__ __forceinline__ f32x4 a_scales(const ESh& sh, int wave, int wblk, int nblk, int b) {
  const int g = (etid() & 63) >> 4;
  const f32x4 v = *(const f32x4*)&sh.s[(wave * wblk + min(b, max(nblk - 1, 0))) * 16 + 4 * g];
  return b < nblk ? v : f32x4{0.f, 0.f, 0.f, 0.f};
}

// 4 scale values of type dt from their raw bits (ld_scale4_raw / a 16-byte load: 16-bit
// types in the first two dwords), without a branch on the dtype: a branch inside the
// K loop makes the compiler copy the live accumulators and ring at the join.
__device__ __forceinline__ void cvt_scale4_nb(const u32x4 raw, int dt, float out[4]) {
  const bool f32 = dt == DT_F32, bf = dt == DT_BF16;
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    const float v16 = bf ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
    out[e] = f32 ? bitcast<float>(w[e]) : v16;
  }
}

__device__ __forceinline__ i32x4 mfma64(u32x4 a, u32x4 b) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(bitcast<i32x4>(a), bitcast<i32x4>(b), i32x4{0, 0, 0, 0}, 0, 0, 0);
}

// One 64-wide W8 block of the lane's 8 columns, folded into acc.
// multi: the unit has more than one activation row.  With one, rows 1-3 of a lane's
// accumulators are never read and their fold (three quarters of it) is skipped.
__device__ __forceinline__ void w8_block(const uint32_t (&w)[16][2], u32x4 a, f32x4 as, f32x4 (&acc)[8],
                                         bool multi) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    uint32_t x0[4], x1[4], x2[4], x3[4];
    tr4(w[0][q], w[1][q], w[2][q], w[3][q], x0);
    tr4(w[4][q], w[5][q], w[6][q], w[7][q], x1);
    tr4(w[8][q], w[9][q], w[10][q], w[11][q], x2);
    tr4(w[12][q], w[13][q], w[14][q], w[15][q], x3);
    i32x4 p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) p[u] = mfma64(a, u32x4{x0[u], x1[u], x2[u], x3[u]});
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[4 * q + u][0] = fmaf((float)p[u][0], as[0], acc[4 * q + u][0]);
    if (multi) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 1; r < 4; ++r) acc[4 * q + u][r] = fmaf((float)p[u][r], as[r], acc[4 * q + u][r]);
    }
  }
}

// One 64-wide W4 block: nibbles as int8 16 (n - 8), even K then odd K (the activation
// operand permuted to match), folded against a_s * b_s / 16; explicit zeros add
// 16 (8 - z) sum(a) (z = 8 when the job has none: no correction).
__device__ __forceinline__ void w4_block(const uint32_t (&w)[8][2], const u32x4 (&sraw)[2], const uint32_t (&zr)[2],
                                         int sdt, bool hz, u32x4 a, f32x4 as, f32x4 (&acc)[8], bool multi) {
  const u32x4 ap = u32x4{perm(a.y, a.x, 0x06040200u), perm(a.w, a.z, 0x06040200u), perm(a.y, a.x, 0x07050301u),
                         perm(a.w, a.z, 0x07050301u)};
  const i32x4 sx = mfma64(ap, u32x4{0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u});
  float ws[8];
  cvt_scale4_nb(sraw[0], sdt, ws);
  const bool f32 = sdt == DT_F32;
  cvt_scale4_nb(u32x4{f32 ? sraw[1].x : sraw[0].z, f32 ? sraw[1].y : sraw[0].w, sraw[1].z, sraw[1].w}, sdt, ws + 4);
#pragma unroll
  for (int t = 0; t < 8; ++t) ws[t] *= 0.0625f;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) w4_split_i8x16(w[i][q], lo[i], hi[i]);
    uint32_t e0[4], e1[4], o0[4], o1[4];
    tr4(lo[0], lo[1], lo[2], lo[3], e0);
    tr4(lo[4], lo[5], lo[6], lo[7], e1);
    tr4(hi[0], hi[1], hi[2], hi[3], o0);
    tr4(hi[4], hi[5], hi[6], hi[7], o1);
    i32x4 p[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) p[u] = mfma64(ap, u32x4{e0[u], e1[u], o0[u], o1[u]});
    int zc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) zc[u] = hz ? (8 - (int)((zr[q] >> (8 * u)) & 0xFFu)) * 16 : 0;
#pragma unroll
    for (int u = 0; u < 4; ++u)
      acc[4 * q + u][0] = fmaf((float)(p[u][0] + zc[u] * sx[0]), as[0] * ws[4 * q + u], acc[4 * q + u][0]);
    if (multi) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 1; r < 4; ++r)
          acc[4 * q + u][r] = fmaf((float)(p[u][r] + zc[u] * sx[r]), as[r] * ws[4 * q + u], acc[4 * q + u][r]);
    }
  }
}

__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Level l's flag, set by its last tile.  (Waiting units poll this word, not the level's
// count: polls of the word that the tiles' atomics update slow those atomics down.)
__device__ __forceinline__ unsigned* level_flag(uint8_t* plan, const EHdr& H, int l) {
  return (unsigned*)(plan + H.flag_off) + 32 * l;
}


// What the epilogue of a single call reads from memory, loaded ahead so that it is not
// on the critical path after the split-K exchange: the W8 column scale of thread t
// (set t / 128, column t % 128) and the residual of thread c's chunk (row c / 32,
// columns 4 (c % 32) of the tile).  (The chain's finisher loads them with its partial
// reads instead.)
struct EEpiPre {
  uint32_t csr;  // raw bits of thread t's column scale: set t / 128, column t % 128
  u32x2 rv;
};

__device__ __forceinline__ void epi_chunk(const EJob& J, const EPos& P, int M, int* row, int* gc, bool* valid) {
  const int nch = M * (TNC / 4);
  const int c = etid();
  const int cc = c < nch ? c : nch - 1;
  *row = cc >> 5;
  *gc = P.tile * TNC + (cc & 31) * 4;
  *valid = c < nch && *gc < J.N;
}

template <bool W4>
__device__ __forceinline__ void epi_prefetch_scales(const EJob& J, const EPos& P, EEpiPre& e) {
  e.csr = 0u;
  if constexpr (!W4) {
    const int t = etid();
    const int set = (t >> 7) < J.nsets ? (t >> 7) : 0;
    const int col = min(P.tile * TNC + (t & (TNC - 1)), J.N - 1);
    e.csr = ld_scale1_raw(set ? J.s[1] : J.s[0], J.sdt, col);
  }
}

// The column scales and the residual into LDS (before a barrier that precedes the
// epilogue): held in registers through the K loop, they would be spilled.
template <bool W4>
__device__ __forceinline__ void epi_pre_to_lds(const EJob& J, const EPos& P, const EEpiPre& e, ESh& sh) {
  const int t = etid();
  if constexpr (!W4) {
    const int col = min(P.tile * TNC + (t & (TNC - 1)), J.N - 1);
    sh.cs[t] = cvt_scale1(e.csr, J.sdt, col);
  }
  sh.rv[t] = e.rv;
}

__device__ __forceinline__ void epi_prefetch_res(const EJob& J, const EPos& P, int M, EEpiPre& e) {
  int row, gc;
  bool valid;
  epi_chunk(J, P, M, &row, &gc, &valid);
  const __amdgpu_buffer_rsrc_t rr =
      part_rsrc(J.res ? J.res : J.out, (unsigned)(((long long)(M - 1) * (J.res ? J.ldr : J.ldo) + J.N) * 2));
  e.rv = bitcast<u32x2>(__builtin_amdgcn_raw_buffer_load_b64(
      rr, (valid && J.res) ? (unsigned)(((long long)row * J.ldr + gc) * 2) : 0xFFFFFFF0u, 0, kCpolSc1));
}

// The unit of a tile that runs its epilogue in the persistent chain: the tile's last
// (set, split), whose unit number is the tile's largest.
__device__ __forceinline__ bool unit_is_finisher(const EJob& J, const EPos& P) {
  return P.set == J.nsets - 1 && P.split == J.splits - 1;
}

// A polling finisher empties its partners' slots for the next use (in the chain after
// its level count, off the tile's path).
template <bool FLIP>
__device__ __forceinline__ void empty_parts(const EJob& J, const EPos& P, int M, float* part_base) {
  const int c = etid();
  const long long MT = (long long)M * TNC;
  if (!J.xch || c >= M * (TNC / 4)) return;
  const int S = J.splits, NSx = J.nsets;
  const __amdgpu_buffer_rsrc_t pr =
      part_rsrc(part_base + J.part, (unsigned)((long long)J.ntiles * NSx * S * MT * 4));
  const f32x4 empty = part_mark<FLIP>();
  for (int s = 0; s < NSx; ++s)
    for (int p = 0; p < S; ++p)
      if (!(s == NSx - 1 && p == S - 1))
        st_coherent(empty, pr, (unsigned)(((((long long)P.tile * NSx + s) * S + p) * MT + c * 4) * 4));
}

// The part of a unit after its K loop: wave sums, K-split / weight-set exchange,
// epilogue.  Returns whether this unit finished its tile (it ran the epilogue).
//
// Two exchanges give the same sums in the same order (per set, split 0 + split 1 + ...):
//  * counter (POLL false; a single call with more units than the chip holds at once):
//    every part is stored, the stores are waited for, an arrival counter per tile picks
//    the last arrival, which reads and sums the parts;
//  * polling (POLL true; the persistent chain, and single calls whose units are all
//    resident at once): the tile's finisher unit (unit_is_finisher) polls its partners'
//    slots until none is empty (part_flip encoding, qlin_dev.h) and sums them with its
//    own part (kept in registers); empty_parts() zeroes them again.  The others store
//    their part and go on without waiting.  One memory round trip on the tile's path
//    instead of three (store completion, counter, reads).  In the chain the finisher's
//    partners have smaller unit numbers, so the smallest unfinished unit never polls
//    for a part that no workgroup holds; in a single call every unit is resident.
// PRE_LDS: the unit's residual and column scales were loaded ahead into LDS
// (epi_pre_to_lds); the polling finisher of a split tile loads its own with its polls.
// FLIP: the slots' encoding (part_code, qlin_dev.h).
template <bool W4, bool POLL = false, bool PRE_LDS = !POLL, bool FLIP = false>
__device__ __forceinline__ bool unit_finish(const EJob& J, const EPos& P, int M, f32x4 (&acc)[8], ESh& sh,
                                            float* part_base, unsigned* cnt_base, int* err_run = nullptr) {
  const int tid = etid(), wave = tid >> 6, lane = tid & 63, j = lane & 15, g = lane >> 4;
  const int nch = M * (TNC / 4);
  const long long MT = (long long)M * TNC;
  if (4 * g < M) {
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (4 * g + r < M) sh.red[(wave * EMAXM + 4 * g + r) * TNP + j * 8 + t] = acc[t][r];
  }
  __syncthreads();
  f32x4 v[2];  // the tile's sums: [set 0, set 1] of chunk tid (row tid / 32, columns 4 (tid % 32))
  v[0] = v[1] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int c = tid;  // nch <= 256
  // the thread's epilogue chunk (row, 4 columns)
  const int N = J.N;
  const int cc = c < nch ? c : nch - 1;  // every thread takes part in the amax shuffles
  const int row = cc >> 5, gc = P.tile * TNC + (cc & 31) * 4;
  const bool valid = c < nch && gc < N;
  const int gcl = gc < N ? gc : N - 4;
  // The chain's finisher loads its epilogue inputs (residual, W8 column scales) with
  // its first reads of the partners' parts, in the same round trip; single calls load
  // them ahead, into LDS.
  u32x2 rvv = u32x2{0u, 0u};
  u32x4 csr[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
  const auto load_epi_in = [&]() {
    const __amdgpu_buffer_rsrc_t rr =
        part_rsrc(J.res ? J.res : J.out, (unsigned)(((long long)(M - 1) * (J.res ? J.ldr : J.ldo) + N) * 2));
    rvv = bitcast<u32x2>(__builtin_amdgcn_raw_buffer_load_b64(
        rr, (valid && J.res) ? (unsigned)(((long long)row * J.ldr + gc) * 2) : 0xFFFFFFF0u, 0, kCpolSc1));
    if constexpr (!W4) {
      csr[0] = ld_scale4_raw(J.s[0], J.sdt, gcl);
      csr[1] = ld_scale4_raw(J.nsets > 1 ? J.s[1] : J.s[0], J.sdt, gcl);
    }
  };
  if (c < nch) {
    const int row = c >> 5, cc = (c & 31) * 4;
    f32x4 sum = *(const f32x4*)&sh.red[row * TNP + cc];
#pragma unroll
    for (int wv = 1; wv < EW; ++wv) sum = sum + *(const f32x4*)&sh.red[(wv * EMAXM + row) * TNP + cc];
    v[0] = sum;
  }
  bool finish = true;
  if (POLL && J.xch) {
    const int S = J.splits, NSx = J.nsets;
    float* const part = part_base + J.part;
    const __amdgpu_buffer_rsrc_t pr = part_rsrc(part, (unsigned)((long long)J.ntiles * NSx * S * MT * 4));
    const auto slot = [&](int s, int p) {
      return (unsigned)(((((long long)P.tile * NSx + s) * S + p) * MT + c * 4) * 4);
    };
    if (!unit_is_finisher(J, P)) {
      if (c < nch) st_coherent(part_code<FLIP>(v[0]), pr, slot(P.set, P.split));
      return false;
    }
    load_epi_in();
    if (c < nch) {
      const f32x4 mine = v[0];
      bool late = false;
      for (int s = 0; s < NSx; ++s) {
        f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int p0 = 0; p0 < S; p0 += 8) {
          f32x4 pp[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) pp[q] = ld_coherent(pr, slot(s, min(p0 + q, S - 1)));
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int p = p0 + q;
            if (p < S) {
              if (s == NSx - 1 && p == S - 1) {
                pp[q] = mine;
              } else {
                int spins = 0;
                while (part_empty<FLIP>(pp[q])) {
                  if (++spins > kSpinLimit) {
                    late = true;
                    break;
                  }
                  __builtin_amdgcn_s_sleep(1);
                  pp[q] = ld_coherent(pr, slot(s, p));
                }
              }
              const f32x4 x = (s == NSx - 1 && p == S - 1) ? pp[q] : part_code<FLIP>(pp[q]);
              sum = (p == 0) ? x : sum + x;
            }
          }
        }
        v[s] = sum;
      }
      if (late && err_run) __hip_atomic_store(err_run, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else if (POLL && !PRE_LDS) {
    load_epi_in();
  } else if (J.xch) {
    // every (set, split) of the tile stores its sums; the last to arrive sums them in
    // split order per set
    const int S = J.splits, NSx = J.nsets;
    float* const part = part_base + J.part;
    const __amdgpu_buffer_rsrc_t pr = part_rsrc(part, (unsigned)((long long)J.ntiles * NSx * S * MT * 4));
    if (c < nch)
      st_coherent(v[0], pr, (unsigned)(((((long long)P.tile * NSx + P.set) * S + P.split) * MT + c * 4) * 4));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) {
      unsigned* cp = cnt_base + J.cnt0 + P.tile;
      const unsigned prev = __hip_atomic_fetch_add(cp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev == (unsigned)(NSx * S - 1);
      if (last) __hip_atomic_store(cp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh.flag = last;
    }
    __syncthreads();
    finish = sh.flag != 0;
    if (finish) {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (c < nch) {
        for (int s = 0; s < NSx; ++s) {
          const unsigned off = (unsigned)((((long long)P.tile * NSx + s) * S * MT + c * 4) * 4);
          f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
          for (int p0 = 0; p0 < S; p0 += 8) {
            f32x4 pp[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) pp[q] = ld_coherent(pr, off + (unsigned)(min(p0 + q, S - 1) * MT * 4));
#pragma unroll
            for (int q = 0; q < 8; ++q)
              if (p0 + q < S) sum = (p0 + q == 0) ? pp[q] : sum + pp[q];
          }
          v[s] = sum;
        }
      }
    }
  }
  if (!finish) return false;

  // ---------------- epilogue ----------------
  float cs[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) cs[s][e] = 1.0f;
  if constexpr (!W4) {
    if (POLL && (J.xch || !PRE_LDS)) {
      cvt_scale4_nb(csr[0], J.sdt, cs[0]);
      cvt_scale4_nb(csr[1], J.sdt, cs[1]);
    } else {
      const int lc = (cc & 31) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        cs[0][e] = sh.cs[lc + e];
        cs[1][e] = sh.cs[TNC + lc + e];
      }
    }
  }
  if (J.epi == EE_STORE) {
    float y[4];
    const __amdgpu_buffer_rsrc_t orr = part_rsrc(J.out, (unsigned)(((long long)(M - 1) * J.ldo + N) * 2));
    if (J.res) {
      const u32x2 rv = (POLL && (J.xch || !PRE_LDS)) ? rvv : sh.rv[c];
      const uint32_t rw[2] = {rv.x, rv.y};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t h = (uint16_t)(rw[e >> 1] >> (16 * (e & 1)));
        y[e] = fmaf(v[0][e], cs[0][e], J.odt == DT_BF16 ? bf16_to_f32(h) : (float)bitcast<_Float16>(h));
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = v[0][e] * cs[0][e];
    }
    if (valid) {
      u32x2 o;
      o.x = (uint32_t)to_out16(y[0], J.odt) | ((uint32_t)to_out16(y[1], J.odt) << 16);
      o.y = (uint32_t)to_out16(y[2], J.odt) | ((uint32_t)to_out16(y[3], J.odt) << 16);
      __builtin_amdgcn_raw_buffer_store_b64(o, orr, (unsigned)(((long long)row * J.ldo + gc) * 2), 0, kCpolSc1);
    }
  } else {
    float h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = silu(v[0][e] * cs[0][e]) * (v[1][e] * cs[1][e]);
    if (J.epi == EE_GATEUP) {
      if (valid) {
        const __amdgpu_buffer_rsrc_t orr = part_rsrc(J.out, (unsigned)(((long long)(M - 1) * J.ldo + N) * 2));
        u32x2 o;
        o.x = (uint32_t)f32_to_bf16(h[0]) | ((uint32_t)f32_to_bf16(h[1]) << 16);
        o.y = (uint32_t)f32_to_bf16(h[2]) | ((uint32_t)f32_to_bf16(h[3]) << 16);
        __builtin_amdgcn_raw_buffer_store_b64(o, orr, (unsigned)(((long long)row * J.ldo + gc) * 2), 0, kCpolSc1);
      }
    } else {
      // bf16 round trip (kernels/gemm.py:198-200), amax of the 64-column group over
      // its 16 chunks (16 consecutive threads), scale and codes (gemm.py:201-211)
      float am = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        h[e] = bf16_to_f32(f32_to_bf16(h[e]));
        am = fmaxf(am, fabsf(h[e]));
      }
      if (!valid) am = 0.0f;
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) am = fmaxf(am, __shfl_xor(am, m));
      const float sc = fmaxf(am / 127.0f, 1e-8f);
      uint32_t qw = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) qw |= ((uint32_t)round_i8(h[e] / sc) & 0xFFu) << (8 * e);
      if (valid) {
        const __amdgpu_buffer_rsrc_t qr = part_rsrc(J.oq, (unsigned)((long long)M * N));
        __builtin_amdgcn_raw_buffer_store_b32(qw, qr, (unsigned)((long long)row * N + gc), 0, kCpolSc1);
        if ((gc & 63) == 0) {
          const __amdgpu_buffer_rsrc_t sr = part_rsrc(J.os, (unsigned)((long long)M * (N / 64) * 4));
          __builtin_amdgcn_raw_buffer_store_b32(bitcast<uint32_t>(sc), sr,
                                                (unsigned)(((long long)row * (N / 64) + gc / 64) * 4), 0, kCpolSc1);
        }
      }
    }
  }
  return true;
}

// Activations of a unit into LDS: the producer (which ends with a barrier), or the
// staged codes (issued by stage_issue) and a barrier.
__device__ __forceinline__ void stage_producer(const EJob& J, const EPos& P, int M, int kbase, int kuu, ESh& sh) {
  const ProGeo G = pro_geo(J.pro, 0, M, kbase, kbase + kuu);
  ProPreN<kEPre> pp;
  pro_issue<true>(J.pro, J.K, G, pp);
  ProOut o;
  o.lq = sh.q;
  o.ls = sh.s;
  o.ldq = LDQ;
  o.lng = 1;
  o.lsb = 16;
  o.emit = J.emit && J.pro.q != nullptr && P.tile == 0 && P.set == 0;
  pro_block<true>(J.pro, J.K, G, pp, o, sh.lr);
}

// Pins the accumulators: the fold of a block is computed here, not sunk below a later
// barrier (the compiler would otherwise hold the block's MFMA results across it).
__device__ __forceinline__ void pin_acc(f32x4 (&acc)[8]) {
#pragma unroll
  for (int t = 0; t < 8; ++t) asm volatile("" : "+v"(acc[t]));
}

// The K loop of one unit over its ring cycles.  `before_last()` runs before the last
// cycle (the persistent form learns the next unit there), and `refill_next(slot)`
// refills a slot in the last cycle (the next unit's first blocks; nothing in the
// single-call form).
template <bool W4, typename Before, typename Next>
__device__ __forceinline__ void unit_loop(const EJob& J, const EPos& P, int M, ERing<W4>& R, const ESh& sh,
                                          f32x4 (&acc)[8], Before&& before_last, Next&& refill_next) {
  const int wave = etid() >> 6;
  const ELoad Ld = make_load(J, P);
  const int nblk = Ld.nblk;
  const int ncyc = J.wblk / RB;
  const bool hz = J.hz != 0;
  const bool multi = M > 1;
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto block = [&](int b, int s) {
    const u32x4 a = a_operand(sh, M, wave, J.wblk, nblk, b);
    const f32x4 as = a_scales(sh, wave, J.wblk, nblk, b);
    if constexpr (W4) w4_block(R.w[s], R.sraw[s], R.zr[s], J.sdt, hz, a, as, acc, multi);
    else w8_block(R.w[s], a, as, acc, multi);
  };
  for (int cyc = 0; cyc + 1 < ncyc; ++cyc) {
#pragma unroll
    for (int s = 0; s < RB; ++s) {
      block(RB * cyc + s, s);
      __builtin_amdgcn_sched_barrier(0);
      load_block<W4>(Ld, RB * (cyc + 1) + s, R, s);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  pin_acc(acc);
  before_last();
#pragma unroll
  for (int s = 0; s < RB; ++s) {
    block(RB * (ncyc - 1) + s, s);
    pin_acc(acc);
    __builtin_amdgcn_sched_barrier(0);
    refill_next(s);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ------------------------------------------------------------------ kernels

// Single call: unit u = blockIdx.x of up to 3 jobs (proj3 segments; one job otherwise).
// POLL: every unit of the grid is resident at once, and split tiles use the polling
// exchange on slots that start zero and are left zero.
template <bool W4, bool POLL>
__global__ __launch_bounds__(ET) __attribute__((amdgpu_waves_per_eu(3))) void ecall_kernel(const ECallArgs a) {
  __shared__ ESh sh;
  const int u = blockIdx.x;
  const int jn = (a.njobs > 1 && u >= a.jobs[1].unit0) + (a.njobs > 2 && u >= a.jobs[2].unit0);
  const EJob& J = a.jobs[jn];
  const EPos P = unit_pos(J, jn, u);
  const int M = a.M;
  const int ku = EW * J.wblk * 64;
  const int kbase = P.split * ku;
  const int kuu = min(ku, J.K - kbase);
  ERing<W4> R;
  const ELoad Ld = make_load(J, P);
  EEpiPre pre;
  if (J.pro.kind != PRO_NONE) {
#pragma unroll
    for (int s = 0; s < RB; ++s) load_block<W4>(Ld, s, R, s);
    epi_prefetch_scales<W4>(J, P, pre);
    epi_prefetch_res(J, P, M, pre);
    stage_producer(J, P, M, kbase, kuu, sh);
  } else {
    EStage st;
    stage_issue(J, M, kbase, kuu, st);
#pragma unroll
    for (int s = 0; s < RB; ++s) load_block<W4>(Ld, s, R, s);
    epi_prefetch_scales<W4>(J, P, pre);
    epi_prefetch_res(J, P, M, pre);
    stage_store(M, kuu, st, sh);
    __syncthreads();
  }
  epi_pre_to_lds<W4>(J, P, pre, sh);  // read after the wave-sum barrier
  f32x4 acc[8];
  unit_loop<W4>(J, P, M, R, sh, acc, []() {}, [](int) {});
  if (unit_finish<W4, POLL, true, true>(J, P, M, acc, sh, a.part, a.cnt) && POLL) empty_parts<true>(J, P, M, a.part);
}

// Persistent chain: workgroup b takes units from queue b % 64 until the plan runs out.
template <bool W4>
__global__ __launch_bounds__(ET) __attribute__((amdgpu_waves_per_eu(3))) void echain_kernel(
    uint8_t* plan, const EJob* __restrict__ jobs, const int* __restrict__ unit_job, const unsigned* __restrict__ need) {
  __shared__ ESh sh;
  const EHdr H = *(const EHdr*)plan;
  unsigned* const cnt = (unsigned*)(plan + H.cnt_off);
  float* const part = (float*)(plan + H.part_off);
  const int tid = etid();
  const int M = H.M;
  const int q = (int)(blockIdx.x % kQueues);
  unsigned* const queue = cnt + 32 * q;
  auto take = [&]() {
    return (int)__hip_atomic_fetch_add(queue, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * kQueues + q;
  };
  // A workgroup holds two units from its queue: the one it runs and the next, whose
  // descriptor is then read before the current unit's dependency wait.  Queues hand
  // their units out in increasing order, so the smallest unfinished unit is always
  // some workgroup's current unit and never waits.
  if (tid == 0) {
    sh.unit = take();
    sh.unit2 = take();
  }
  __syncthreads();
  int u = sh.unit;
  int un = sh.unit2;
  ERing<W4> R;
  int jn = 0;
  EPos P;
  if (u < H.nunits) {
    jn = __builtin_amdgcn_readfirstlane(unit_job[u]);
    P = unit_pos(jobs[jn], jn, u);
    const ELoad L0 = make_load(jobs[jn], P);
#pragma unroll
    for (int s = 0; s < RB; ++s) load_block<W4>(L0, s, R, s);
  }
  while (u < H.nunits) {
    // the unit after the next one: taken now, read at the next unit's start
    int nn = 0;
    if (tid == 0) nn = take();
    const EJob& J = jobs[jn];
    const int ku = EW * J.wblk * 64;
    const int kbase = P.split * ku;
    const int kuu = min(ku, J.K - kbase);

    // ---- the next unit's descriptor (past the last unit: any valid descriptor; the
    // workgroup leaves before loading anything for it) ----
    const bool more = un < H.nunits;
    const int jnn = more ? __builtin_amdgcn_readfirstlane(unit_job[un]) : jn;
    const EPos Pn = unit_pos(jobs[jnn], jnn, more ? un : jobs[jnn].unit0);
    const ELoad Ln = make_load(jobs[jnn], Pn);

    // ---- dependency: level L waits for every tile of level L - 1 ----
    if (J.level > 0) {
      if (tid == 0) {
        const unsigned* f = level_flag(plan, H, J.level - 1);
        int spins = 0, nap = 1;
        while (ld_agent(f) == 0u) {
          if (++spins > kSpinLimit) {
            __hip_atomic_store((int*)(plan + offsetof(EHdr, err_run)), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          if (nap == 1) __builtin_amdgcn_s_sleep(1);
          else if (nap == 2) __builtin_amdgcn_s_sleep(2);
          else __builtin_amdgcn_s_sleep(6);
          nap = nap < 3 ? nap + 1 : 3;
        }
      }
      __syncthreads();
    }
    // ---- activations into LDS ----
    if (J.pro.kind != PRO_NONE) {
      stage_producer(J, P, M, kbase, kuu, sh);
    } else {
      EStage st;
      stage_issue(J, M, kbase, kuu, st);
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      stage_store(M, kuu, st, sh);
      __syncthreads();
    }
    // ---- K loop ----
    f32x4 acc[8];
    unit_loop<W4>(J, P, M, R, sh, acc, []() {}, [](int) {});
    const bool fin = unit_finish<W4, true>(J, P, M, acc, sh, part, cnt + kLevel0 + 32 * H.nlevels,
                                           (int*)(plan + offsetof(EHdr, err_run)));

    // ---- the tile counts for its level (its outputs written first); the level's last
    // tile sets the flag ----
    if (fin && J.level + 1 < H.nlevels) {
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __syncthreads();
      if (tid == 0) {
        const unsigned pl = __hip_atomic_fetch_add(cnt + kLevel0 + 32 * J.level, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
        if (pl + 1 == need[J.level])
          __hip_atomic_store(level_flag(plan, H, J.level), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (fin) empty_parts<false>(J, P, M, part);
    // ---- the next unit's first blocks.  Issued only now: gfx950 counts loads and
    // stores on one in-order counter, so weight loads issued before this unit's
    // partial and output stores would make every wait for those stores (on the path
    // to the next level) wait for the weights as well.  A workgroup with no next unit
    // leaves here: loads for nothing would queue in front of the memory operations on
    // other units' dependency paths. ----
    if (!more) break;
#pragma unroll
    for (int s = 0; s < RB; ++s) load_block<W4>(Ln, s, R, s);
    if (tid == 0) sh.unit2 = nn;
    __syncthreads();
    jn = jnn;
    P = Pn;
    u = un;
    un = (int)__builtin_amdgcn_readfirstlane((uint32_t)sh.unit2);
  }
  // the last workgroup to leave resets the queues, level counters and flags, and
  // publishes this launch's error word
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(cnt + 32 * kQueues, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == gridDim.x - 1) {
      for (int l = 0; l < H.nlevels; ++l) {
        __hip_atomic_store(cnt + kLevel0 + 32 * l, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(level_flag(plan, H, l), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      for (int qq = 0; qq < kQueues; ++qq) __hip_atomic_store(cnt + 32 * qq, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(cnt + 32 * kQueues, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int* const er = (int*)(plan + offsetof(EHdr, err_run));
      const int e = __hip_atomic_load(er, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store((int*)(plan + offsetof(EHdr, err)), e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(er, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace

// ------------------------------------------------------------------ host side

// Blocks per wave of a job's units: RB (K ranges of 512 per unit), or more for jobs
// whose shortest units outnumber the workgroups that fit the chip kLongFactor times
// over (fewer split-K exchanges at the same parallelism), up to KU_MAX per unit.  A
// function of (K, N, sets) only.
int echain_wblk(int K, int N, int nsets) {
  const long long kun = (K + 511) / 512;
  const long long units = (long long)((N + TNC - 1) / TNC) * nsets * kun;
  const long long r = std::max<long long>(1, std::min<long long>(units / ((long long)kLongFactor * kPlanSlots),
                                                                 std::min<long long>(kun, KU_MAX / 512)));
  return RB * (int)r;
}

// One job of a call or chain, as the host validates and lays it out.
struct EHost {
  EJob d;
  long long units, parts;  // work units; partial floats per row (0: no exchange)
};

bool ealigned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int efail(const char* fn, int code, const char* what, int i) {
  char msg[256];
  snprintf(msg, sizeof(msg), "%s: job %d: %s", fn, i, what);
  return set_error(code, msg);
}

// Completes a job descriptor (tiles, splits, unit length, exchange) and validates it.
int echain_layout_job(const char* fn, int i, int M, EJob& d, long long* units, long long* parts_per_row) {
  if (M < 1 || M > EMAXM) return efail(fn, QLIN_ERR_UNSUPPORTED, "1-8 rows", i);
  if (d.K <= 0 || d.N <= 0) return efail(fn, QLIN_ERR_INVALID, "bad sizes", i);
  if (d.K % 64 != 0) return efail(fn, QLIN_ERR_UNSUPPORTED, "K must be a multiple of 64", i);
  if (d.N % 16 != 0) return efail(fn, QLIN_ERR_UNSUPPORTED, "N must be a multiple of 16", i);
  const bool w4 = d.group != 0;
  if (w4 && (d.group % 64 != 0 || d.K % d.group != 0))
    return efail(fn, QLIN_ERR_UNSUPPORTED, "W4 group must be a multiple of 64 dividing K", i);
  if (d.nsets != 1 && d.nsets != 2) return efail(fn, QLIN_ERR_INVALID, "weight sets", i);
  for (int s = 0; s < d.nsets; ++s) {
    if (!d.w[s] || !d.s[s]) return efail(fn, QLIN_ERR_INVALID, "null weight or scale", i);
    if (!ealigned(d.w[s], 16) || !ealigned(d.s[s], 16) || (d.z[s] && !ealigned(d.z[s], 16)))
      return efail(fn, QLIN_ERR_UNSUPPORTED, "weight/scale/zero pointers must be 16-byte aligned", i);
    if (!w4 && d.z[s]) return efail(fn, QLIN_ERR_INVALID, "zeros given for W8 weights", i);
  }
  if (d.nsets == 2 && (d.z[0] == nullptr) != (d.z[1] == nullptr))
    return efail(fn, QLIN_ERR_INVALID, "zeros for gate and up, or for neither", i);
  if (d.sdt != DT_F16 && d.sdt != DT_BF16 && d.sdt != DT_F32) return efail(fn, QLIN_ERR_UNSUPPORTED, "scale dtype", i);
  d.hz = (d.z[0] != nullptr) ? 1 : 0;
  if (d.pro.kind == PRO_NONE) {
    if (!d.aq || !d.as) return efail(fn, QLIN_ERR_INVALID, "null activations", i);
    if (!ealigned(d.aq, 16) || !ealigned(d.as, 4))
      return efail(fn, QLIN_ERR_UNSUPPORTED, "activation codes must be 16-byte aligned", i);
  }
  if (d.epi == EE_STORE || d.epi == EE_GATEUP) {
    if (!d.out) return efail(fn, QLIN_ERR_INVALID, "null output", i);
    if (d.ldo < d.N || d.ldo % 4 != 0 || !ealigned(d.out, 8))
      return efail(fn, QLIN_ERR_UNSUPPORTED, "output must be 8-byte aligned with a row stride >= N, multiple of 4", i);
    if (d.res && (d.ldr < d.N || d.ldr % 4 != 0 || !ealigned(d.res, 8)))
      return efail(fn, QLIN_ERR_UNSUPPORTED, "residual must be 8-byte aligned with a row stride >= N, multiple of 4", i);
    if (d.odt != DT_F16 && d.odt != DT_BF16) return efail(fn, QLIN_ERR_UNSUPPORTED, "output dtype", i);
  } else {
    if (!d.oq || !d.os) return efail(fn, QLIN_ERR_INVALID, "null out_q / out_s", i);
    if (d.N % 64 != 0) return efail(fn, QLIN_ERR_UNSUPPORTED, "gate/up + quant needs N % 64 == 0", i);
    if (!ealigned(d.oq, 4) || !ealigned(d.os, 4)) return efail(fn, QLIN_ERR_UNSUPPORTED, "out_q alignment", i);
  }
  if ((d.epi == EE_STORE) != (d.nsets == 1)) return efail(fn, QLIN_ERR_INVALID, "epilogue / weight sets", i);
  if (((long long)(M - 1) * d.ldo + d.N) * 2 >= (1LL << 31) || (long long)M * d.K >= (1LL << 31))
    return efail(fn, QLIN_ERR_UNSUPPORTED, "activation or output too large", i);
  d.wblk = echain_wblk(d.K, d.N, d.nsets);
  const int ku = EW * d.wblk * 64;
  d.splits = (d.K + ku - 1) / ku;
  d.ntiles = (d.N + TNC - 1) / TNC;
  d.xch = (d.splits > 1 || d.nsets == 2) ? 1 : 0;
  *units = (long long)d.ntiles * d.nsets * d.splits;
  *parts_per_row = d.xch ? (long long)d.ntiles * d.nsets * d.splits * TNC : 0;
  if ((long long)d.ntiles * d.nsets * d.splits * M * TNC * 4 >= (1LL << 31))
    return efail(fn, QLIN_ERR_UNSUPPORTED, "partials too large", i);
  return QLIN_OK;
}

namespace {

std::mutex g_emu;
int g_egrid[64][2];

// Workgroups of an engine-chain launch: 2 per CU, though 3 fit.  A chain's levels wait
// on one another, and with fewer workgroups per CU each unit's K loop, sum and exchange
// run sooner: W8 47.1-47.4 vs 49.0-49.1 us per layer at M = 4 (44.7 vs 44.8 at M = 1),
// W4 43.9-44.0 vs 45.4-45.6 at M = 1 and 47.9 vs 51.3-51.6 at M = 4 (alternated twice).
// One per CU leaves too few units in flight on the wide levels: W8 64.6 / 69.4 us.
int egrid(bool w4, int* grid) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) return set_error(QLIN_ERR_HIP, "qlin_echain_run: hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_emu);
  if (g_egrid[dev][w4] == 0) {
    int cus = 0, per = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
      e = w4 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, echain_kernel<true>, ET, 0)
             : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, echain_kernel<false>, ET, 0);
    if (e != hipSuccess || cus <= 0 || per <= 0) return set_error(QLIN_ERR_HIP, "qlin_echain_run: occupancy query failed");
    g_egrid[dev][w4] = cus * std::min(per, 2);
  }
  *grid = g_egrid[dev][w4];
  return QLIN_OK;
}

struct EPlanInfo {
  const void* plan;
  int w4;
  long long jobs_off, unit_off, need_off;
};
std::vector<EPlanInfo> g_eplans;

}  // namespace

// The single-call form: up to 3 jobs (same K, activations, weight format) at level 0,
// split-K scratch from the caller's workspace ([counters | partials]).  `clear` zeroes
// the counters first (a scratch not known to be zero).
// Workgroups of a single call's grid that are resident on the device at once.
int g_cres[64][2];
int ecall_resident(bool w4, int* n) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) return set_error(QLIN_ERR_HIP, "echain_call: hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_emu);
  if (g_cres[dev][w4] == 0) {
    int cus = 0, per = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
      e = w4 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, ecall_kernel<true, true>, ET, 0)
             : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, ecall_kernel<false, true>, ET, 0);
    if (e != hipSuccess || cus <= 0 || per <= 0) return set_error(QLIN_ERR_HIP, "echain_call: occupancy query failed");
    g_cres[dev][w4] = cus * per;
  }
  *n = g_cres[dev][w4];
  return QLIN_OK;
}

// The workspace (or a scratch laid out like it): `counter_bytes` of arrival counters,
// `poll_bytes` of polling-exchange slots (zero between calls), then split-K partials.
// A call whose units are all resident at once takes the polling exchange
// (QLIN_ECALL_POLL=0 turns it off); a larger one the arrival counters.
int echain_call(const char* fn, EJob* jobs, int njobs, int M, void* ws, size_t wsb, size_t counter_bytes,
                size_t poll_bytes, hipStream_t stream, bool clear) {
  if (njobs < 1 || njobs > 3) return set_error(QLIN_ERR_INVALID, "echain_call: 1-3 jobs");
  ECallArgs a;
  memset(&a, 0, sizeof(a));
  long long units = 0, parts = 0, cnts = 0;
  const bool w4 = jobs[0].group != 0;
  for (int i = 0; i < njobs; ++i) {
    EJob d = jobs[i];
    long long u = 0, ppr = 0;
    QL_TRY_E(echain_layout_job(fn, i, M, d, &u, &ppr));
    if ((d.group != 0) != w4) return efail(fn, QLIN_ERR_INVALID, "mixed weight formats", i);
    d.unit0 = (int)units;
    d.cnt0 = (int)cnts;
    d.part = parts;
    d.level = 0;
    d.emit = (i == 0) ? 1 : 0;
    units += u;
    if (d.xch) {
      cnts += d.ntiles;
      parts += ppr * M;
    }
    a.jobs[i] = d;
  }
  if (units > 0x7FFFFFFFLL) return set_error(QLIN_ERR_UNSUPPORTED, "echain_call: grid too large");
  bool poll = false;
  if (parts > 0) {
    int resident = 0;
    QL_TRY_E(ecall_resident(w4, &resident));
    const char* ep = getenv("QLIN_ECALL_POLL");
    poll = !(ep && strcmp(ep, "0") == 0) && ws && units <= resident && (size_t)parts * 4 <= poll_bytes &&
           wsb >= counter_bytes + poll_bytes;
  }
  if (cnts > 0 || parts > 0) {
    if (poll) {
      a.cnt = (unsigned*)ws;
      a.part = (float*)((char*)ws + counter_bytes);
    } else {
      if (!ws || (size_t)cnts * 4 > counter_bytes || wsb < counter_bytes + poll_bytes + (size_t)parts * 4) {
        char msg[200];
        snprintf(msg, sizeof(msg), "%s: the workspace cannot hold %lld split-K partial floats", fn, parts);
        return set_error(QLIN_ERR_WORKSPACE, msg);
      }
      a.cnt = (unsigned*)ws;
      a.part = (float*)((char*)ws + counter_bytes + poll_bytes);
      if (clear) {
        const hipError_t e = clear_counters(ws, cnts, stream);
        if (e != hipSuccess) return set_error(QLIN_ERR_HIP, "echain_call: counter clear failed");
      }
    }
  }
  a.njobs = njobs;
  a.M = M;
  a.nunits = (int)units;
  if (w4) {
    if (poll) hipLaunchKernelGGL((ecall_kernel<true, true>), dim3((unsigned)units), dim3(ET), 0, stream, a);
    else hipLaunchKernelGGL((ecall_kernel<true, false>), dim3((unsigned)units), dim3(ET), 0, stream, a);
  } else {
    if (poll) hipLaunchKernelGGL((ecall_kernel<false, true>), dim3((unsigned)units), dim3(ET), 0, stream, a);
    else hipLaunchKernelGGL((ecall_kernel<false, false>), dim3((unsigned)units), dim3(ET), 0, stream, a);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char msg[200];
    snprintf(msg, sizeof(msg), "%s: HIP error %d (%s)", fn, (int)e, hipGetErrorString(e));
    return set_error(QLIN_ERR_HIP, msg);
  }
  return QLIN_OK;
}

bool echain_covers(const SkArgs& a, int wk, int M) {
  if (M < 1 || M > EMAXM || a.K % 64 != 0) return false;
  if (wk == WK_W4 && a.group % 64 != 0) return false;
  if (a.pro.kind == PRO_NONE && (!ealigned(a.x, 16) || !ealigned(a.xs, 4))) return false;
  for (int s = 0; s < a.nseg; ++s)
    if (a.seg[s].n % 16 != 0) return false;
  return true;
}

// An engine-signature call (SkArgs as abi.hip builds it) as echain jobs: one per
// proj3 column segment, one for gemm or gate/up.
int echain_engine_call(const char* fn, const SkArgs& a, int wk, int epi, int M, void* ws, size_t ws_bytes,
                       size_t counter_bytes, size_t poll_bytes, hipStream_t stream, bool clear) {
  EJob base;
  memset(&base, 0, sizeof(base));
  base.aq = (const int8_t*)a.x;
  base.as = a.xs;
  base.pro = a.pro;
  base.K = a.K;
  base.group = wk == WK_W4 ? a.group : 0;
  base.sdt = a.sdt;
  base.odt = a.odt;
  EJob jobs[3];
  int nj = 0;
  if (epi == EPI_STORE) {
    for (int s = 0; s < a.nseg; ++s) {
      EJob d = base;
      d.w[0] = a.seg[s].w;
      d.s[0] = a.seg[s].s;
      d.z[0] = a.seg[s].z;
      d.N = a.seg[s].n;
      d.out = (uint16_t*)a.out + a.seg[s].col0;
      d.ldo = a.ldo;
      d.res = a.res ? (const uint16_t*)a.res + a.seg[s].col0 : nullptr;
      d.ldr = a.ldr;
      d.epi = EE_STORE;
      d.nsets = 1;
      jobs[nj++] = d;
    }
  } else {
    EJob d = base;
    for (int s = 0; s < 2; ++s) {
      d.w[s] = a.seg[s].w;
      d.s[s] = a.seg[s].s;
      d.z[s] = a.seg[s].z;
    }
    d.N = a.seg[0].n;
    d.nsets = 2;
    d.epi = epi == EPI_GATEUP ? EE_GATEUP : EE_GATEUP_Q;
    d.out = a.out;
    d.ldo = a.ldo;
    d.oq = a.oq;
    d.os = a.os;
    jobs[nj++] = d;
  }
  return echain_call(fn, jobs, nj, M, ws, ws_bytes, counter_bytes, poll_bytes, stream, clear);
}

// ------------------------------------------------------------------ chain plans

namespace {

struct ELayout {
  long long jobs_off, unit_off, need_off, cnt_off, flag_off, part_off, bytes;
  int nunits, nlevels, ncnt, w4;
};

long long ealign256(long long v) { return (v + 255) / 256 * 256; }

EJob job_from(const qlin_echain_job& q) {
  EJob d;
  memset(&d, 0, sizeof(d));
  d.aq = q.a_q;
  d.as = q.a_s;
  d.w[0] = (const uint8_t*)q.w;
  d.s[0] = q.scale;
  d.z[0] = q.zero;
  d.w[1] = (const uint8_t*)q.w2;
  d.s[1] = q.scale2;
  d.z[1] = q.zero2;
  d.out = q.out;
  d.ldo = q.ldo;
  d.res = q.residual;
  d.ldr = q.residual ? q.ldr : 0;
  d.oq = q.out_q;
  d.os = q.out_s;
  d.K = q.K;
  d.N = q.N;
  d.group = q.group;
  d.sdt = q.scale_dtype;
  d.odt = QLIN_BF16;
  d.level = q.level;
  d.emit = 1;
  switch (q.kind) {
    case QLIN_EJ_GEMM: d.epi = EE_STORE, d.nsets = 1; break;
    case QLIN_EJ_GATE_UP: d.epi = EE_GATEUP, d.nsets = 2; break;
    case QLIN_EJ_GATE_UP_QUANT: d.epi = EE_GATEUP_Q, d.nsets = 2; break;
    default: d.epi = -1, d.nsets = 0; break;
  }
  return d;
}

int elayout(const char* fn, const qlin_echain_job* jobs, int njobs, int M, ELayout* L, std::vector<EJob>* out,
            std::vector<int>* unit_job, std::vector<unsigned>* need) {
  if (!jobs || njobs <= 0) return set_error(QLIN_ERR_INVALID, "qlin_echain: no jobs");
  if (M < 1 || M > EMAXM) return set_error(QLIN_ERR_UNSUPPORTED, "qlin_echain: M must be 1-8");
  const bool w4 = jobs[0].group != 0;
  int prev = 0;
  long long units = 0, ncnt = 0, parts = 0;
  for (int i = 0; i < njobs; ++i) {
    const qlin_echain_job& q = jobs[i];
    if (q.kind != QLIN_EJ_GEMM && q.kind != QLIN_EJ_GATE_UP && q.kind != QLIN_EJ_GATE_UP_QUANT)
      return efail(fn, QLIN_ERR_INVALID, "unknown job kind", i);
    if (q.level < prev || q.level > prev + 1 || (i == 0 && q.level != 0))
      return efail(fn, QLIN_ERR_INVALID, "levels start at 0 and rise by at most 1 along the list", i);
    if ((q.group != 0) != w4) return efail(fn, QLIN_ERR_UNSUPPORTED, "a chain holds W8 jobs or W4 jobs, not both", i);
    EJob d = job_from(q);
    if (q.pro.kind != 0) {
      ProArgs& p = d.pro;
      p.kind = q.pro.kind;
      p.x = q.pro.x;
      p.ldx = q.pro.ldx;
      p.xdt = q.pro.x_dtype;
      p.g = q.pro.g;
      p.ldg = q.pro.ldg;
      p.w = q.pro.w;
      p.wdt = q.pro.w_dtype;
      p.hd = q.pro.hd;
      p.one_plus = q.pro.one_plus;
      p.eps = q.pro.eps;
      p.q = q.pro.q;
      p.s = q.pro.s;
      QL_TRY_E(check_producer(fn, p, M, d.K));
      if (!p.q && (q.a_q || q.a_s)) return efail(fn, QLIN_ERR_INVALID, "a producer job takes no a_q / a_s", i);
    }
    long long u = 0, ppr = 0;
    QL_TRY_E(echain_layout_job(fn, i, M, d, &u, &ppr));
    d.unit0 = (int)units;
    d.cnt0 = (int)ncnt;
    d.part = parts;
    if (out) {
      out->push_back(d);
      for (long long t = 0; t < u; ++t) unit_job->push_back(i);
      if ((int)need->size() <= q.level) need->resize(q.level + 1, 0u);
      (*need)[q.level] += (unsigned)d.ntiles;
    }
    units += u;
    if (d.xch) {
      ncnt += d.ntiles;
      parts += ppr * M;
    }
    if (units > (1LL << 30)) return efail(fn, QLIN_ERR_UNSUPPORTED, "too many work units", i);
    prev = q.level;
  }
  L->nunits = (int)units;
  L->nlevels = prev + 1;
  L->ncnt = (int)(kLevel0 + 32LL * L->nlevels + ncnt);
  L->w4 = w4 ? 1 : 0;
  L->jobs_off = ealign256(sizeof(EHdr));
  L->unit_off = ealign256(L->jobs_off + (long long)njobs * sizeof(EJob));
  L->need_off = ealign256(L->unit_off + units * 4);
  L->cnt_off = ealign256(L->need_off + (long long)L->nlevels * 4);
  L->flag_off = ealign256(L->cnt_off + (long long)L->ncnt * 4);
  L->part_off = ealign256(L->flag_off + (long long)L->nlevels * 128);
  L->bytes = ealign256(L->part_off + parts * 4);
  return QLIN_OK;
}

}  // namespace
}  // namespace qlin

extern "C" size_t qlin_echain_bytes(const qlin_echain_job* jobs, int njobs, int M) {
  qlin::ELayout L;
  if (qlin::elayout("qlin_echain_bytes", jobs, njobs, M, &L, nullptr, nullptr, nullptr) != QLIN_OK) return 0;
  return (size_t)L.bytes;
}

extern "C" int qlin_echain_init(const qlin_echain_job* jobs, int njobs, int M, void* plan, size_t plan_bytes,
                                void* stream) {
  using namespace qlin;
  set_error(QLIN_OK, "");
  ELayout L;
  std::vector<EJob> d;
  std::vector<int> uj;
  std::vector<unsigned> need;
  const int rc = elayout("qlin_echain_init", jobs, njobs, M, &L, &d, &uj, &need);
  if (rc != QLIN_OK) return rc;
  if (!plan || plan_bytes < (size_t)L.bytes) return set_error(QLIN_ERR_WORKSPACE, "qlin_echain_init: plan buffer too small");
  if (!ealigned(plan, 16)) return set_error(QLIN_ERR_UNSUPPORTED, "qlin_echain_init: plan must be 16-byte aligned");
  need.resize(L.nlevels, 0u);
  // the image runs to the end of the plan: the partial-sum slots start empty (-0.0)
  std::vector<uint8_t> img((size_t)L.bytes, 0);
  const uint32_t mark = 0x80000000u;
  for (size_t o = (size_t)L.part_off; o + 4 <= img.size(); o += 4) memcpy(img.data() + o, &mark, 4);
  EHdr h;
  memset(&h, 0, sizeof(h));
  h.magic = kMagic;
  h.nunits = L.nunits;
  h.njobs = njobs;
  h.nlevels = L.nlevels;
  h.M = M;
  h.w4 = L.w4;
  h.jobs_off = L.jobs_off;
  h.unit_off = L.unit_off;
  h.need_off = L.need_off;
  h.cnt_off = L.cnt_off;
  h.flag_off = L.flag_off;
  h.part_off = L.part_off;
  h.bytes = L.bytes;
  memcpy(img.data(), &h, sizeof(h));
  memcpy(img.data() + L.jobs_off, d.data(), d.size() * sizeof(EJob));
  memcpy(img.data() + L.unit_off, uj.data(), uj.size() * sizeof(int));
  memcpy(img.data() + L.need_off, need.data(), need.size() * sizeof(unsigned));
  hipError_t e = hipMemcpyAsync(plan, img.data(), img.size(), hipMemcpyHostToDevice, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) {
    char msg[160];
    snprintf(msg, sizeof(msg), "qlin_echain_init: copy: HIP error %d (%s)", (int)e, hipGetErrorString(e));
    return set_error(QLIN_ERR_HIP, msg);
  }
  std::lock_guard<std::mutex> lk(g_emu);
  const EPlanInfo info{plan, L.w4, L.jobs_off, L.unit_off, L.need_off};
  for (auto& p : g_eplans)
    if (p.plan == plan) {
      p = info;
      return QLIN_OK;
    }
  g_eplans.push_back(info);
  return QLIN_OK;
}

extern "C" int qlin_echain_run(void* plan, void* stream) {
  using namespace qlin;
  set_error(QLIN_OK, "");
  if (!plan || !ealigned(plan, 16)) return set_error(QLIN_ERR_INVALID, "qlin_echain_run: null or misaligned plan");
  EPlanInfo pi{};
  bool found = false;
  {
    std::lock_guard<std::mutex> lk(g_emu);
    for (auto& p : g_eplans)
      if (p.plan == plan) pi = p, found = true;
  }
  if (!found) return set_error(QLIN_ERR_INVALID, "qlin_echain_run: plan not initialized by qlin_echain_init in this process");
  int grid = 0;
  const int rc = egrid(pi.w4 != 0, &grid);
  if (rc != QLIN_OK) return rc;
  uint8_t* const p = (uint8_t*)plan;
  const EJob* jobs = (const EJob*)(p + pi.jobs_off);
  const int* units = (const int*)(p + pi.unit_off);
  const unsigned* need = (const unsigned*)(p + pi.need_off);
  const hipStream_t st = (hipStream_t)stream;
  if (pi.w4) hipLaunchKernelGGL(echain_kernel<true>, dim3(grid), dim3(ET), 0, st, p, jobs, units, need);
  else hipLaunchKernelGGL(echain_kernel<false>, dim3(grid), dim3(ET), 0, st, p, jobs, units, need);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char msg[160];
    snprintf(msg, sizeof(msg), "qlin_echain_run: HIP error %d (%s)", (int)e, hipGetErrorString(e));
    return set_error(QLIN_ERR_HIP, msg);
  }
  return QLIN_OK;
}
