// Persistent multi-GEMV launch ("chain"): the decode-step linears of many layers in one
// kernel, gfx950.
//
// A chain is a list of A16 GEMV jobs (fp16 activations x[M][K], M <= 16; W8 int8 [K][N]
// with per-column scales, or W4 packed nibbles [K/2][N] with group-128 scales and
// optional zeros -- the engine layouts of weights.py:297-309) with dependency levels:
// the jobs of level L > 0 read their activations only after every job of level L-1
// has written its output.  One launch runs the whole list: the decode step of a model
// (per layer q/k/v, o, gate/up, down, then the vocabulary head) with no kernel
// boundary between GEMVs.  This is the reference's own stated next step for a decode
// that is dispatch-bound at one launch per linear (ENGINEERING.md:383-399).
//
//   * Work unit = (job, 128-column tile, K range of 4 waves x 128 rows): 64 KB of W8
//     weights, 32 KB of packed W4 (one group of 128 per wave).  Workgroups of 4 waves
//     take units from 8 queues (workgroup b from queue b % 8; queue q hands out units
//     q, q + 8, ... in order; the next index is fetched while the current unit runs),
//     so a unit only ever waits for units of lower levels, all taken before it: every
//     wait ends whether or not all workgroups are resident.  Within a level the units
//     go round robin over its jobs (every job's first unit, then every job's second).
//   * A unit's weight (and scale, zero) loads are in flight before it waits: above
//     level 0 it waits for the level below (one thread polls the level's done flag with
//     a bounded spin), then reads its activations with device-coherent loads (level 0:
//     issued with the weights).  The last ring cycle of a unit refills each slot with
//     the next unit's first step as soon as the slot's MFMAs are issued, so a wave's
//     loads stay in flight across the unit boundary.
//   * Each wave computes its 128-row K range for the tile's 128 columns on
//     v_mfma_f32_16x16x32_f16 with exactly converted weights (the skinny decode
//     kernel's operand construction: qlin_dev.h w8_pair_f16 / w4_pair_offset with the
//     per-group offset correction); the 4 waves are summed in LDS in wave order.
//   * A tile split over several units (K splits) exchanges fp32 partials through
//     device-coherent stores and an arrival counter; the last unit to arrive sums the
//     splits in split order (deterministic), applies the W8 column scale and the
//     residual (one fmaf), and stores the 16-bit output with device-coherent stores.
//     After those stores complete it counts the tile for its level, and the level's
//     last tile sets the level's flag.
//   * The K order of an output depends on (K, N) and on the size of the job's level
//     (levels with many units take longer units), never on M: rows of an M = 4 chain
//     equal an M = 1 chain of the same jobs bit for bit, but the same linear in a chain
//     of other levels (or another layer count) may differ in the last bits.
//   * The last workgroup to leave resets the queues, the exit and level counters and
//     the flags, so a plan can be launched again (and replayed in a HIP graph) without
//     clearing, and publishes the launch's error word (a dependency wait that gave up):
//     the header's `err` always describes the last finished launch.
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/qlin.h"
#include "qlin_dev.h"
#include "qlin_internal.h"

namespace qlin {
namespace {

constexpr int CW = 4;              // waves per workgroup = per work unit
constexpr int CT = 64 * CW;
constexpr int TNC = 128;           // columns per tile: 16 lanes x 8 columns
constexpr int TNP = TNC + 4;       // padded LDS row
constexpr int RING = 4;            // 32-wide K steps a wave has in flight (its register ring)
constexpr int KU = CW * RING * 32; // K rows of the shortest unit: 512 (W4: one group of 128 per wave)
constexpr int kSpinLimit = 1 << 22;        // polls of a dependency before giving up
constexpr int kWaitVm0 = 0x0F70;           // s_waitcnt vmcnt(0) (expcnt, lgkmcnt left at their maxima)
// Levels whose units at the shortest length outnumber the workgroups that fit the chip
// this many times over (kPlanSlots: 3 workgroups on each of 256 CUs) take longer units
// -- up to kMaxR shortest units or a tile's whole K -- streamed through the same
// register ring: fewer split-K exchanges, the same parallelism.
constexpr int kPlanSlots = 768;
constexpr int kLongFactor = 2;
// Longest unit: 4 x KU = 2048 K rows.  With a tile's whole K allowed (down's 6144 in
// units of 5120 and 1024, lin_out's 4096 in one) the flat decode sweep's units differ
// in length and the last round of workgroups ends unevenly; uniform 2048-row units
// are faster (W8 180-181 vs 182.3-182.6 us per launch, W4 107-112 vs 111-113 us,
// alternated three times).
constexpr int kMaxR = 4;
// A unit-table entry holds its job (low kJobBits bits) and its index within the job.
constexpr int kJobBits = 12;
constexpr int kMaxJobs = 1 << kJobBits;

// Device descriptor of one job.
struct alignas(16) ChainJob {
  const _Float16* x;
  long long ldx;
  const uint8_t* w;
  const void* s;
  const uint8_t* z;
  void* out;
  long long ldo;
  const void* res;
  long long ldr;
  long long part;   // first float of this job's partials within the partial region
  int K, N, wk, sdt, odt;
  int ntiles, splits, unit0, cnt0, level, index;
  int wsteps;       // 32-wide K steps per wave per unit (a multiple of RING)
  int pad_[3];
};

// Header at the start of a plan (device memory).
struct alignas(16) ChainHdr {
  int magic, nunits, njobs, nlevels;
  int M, err, ncnt, w4;
  long long jobs_off, unit_off, need_off, cnt_off, flag_off, part_off, bytes;
  int err_run;  // set by a wait that gives up during a launch; moved to `err` at its end
  int pad_[3];
};
constexpr int kMagic = 0x71636831;  // "qch1"

// Counters (uint32 indices from cnt_off).  Every counter that many workgroups update
// sits on a 128-byte line of its own: atomics on one address serialize (about 18 ns
// each, measured), so the hot ones are spread out.
//   [32 q]                              queue q (q < kQueues): units q, q + 8, q + 16, ...
//   [32 kQueues]                        workgroups that have left
//   [kLevel0 + 32 l]                    finished tiles of level l
//   [kLevel0 + 32 nlevels + 16 njobs + cnt0 + tile]
//                                       split-K arrivals of a tile (reset by its last unit)
// Level done flags follow in a region of their own, one per 128-byte line.
constexpr int kQueues = 8;
constexpr int kLevel0 = 32 * (kQueues + 1);

__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ u32x4 ld_x_coherent(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolSc1);
}

template <int COLS>
__device__ __forceinline__ void ld8(const uint8_t* p, uint32_t d[2]) {
  const u32x2 v = ld_global_nt<u32x2>(p);
  d[0] = v.x;
  d[1] = v.y;
}

// Registers a unit's weights (and W4 group scales, zeros) are loaded into: a ring of
// RING steps.
template <bool W4>
struct UnitRegs {
  static constexpr int STEPS = RING;
  static constexpr int NR = W4 ? 4 : 8;  // weight rows per lane per step
  uint32_t w[STEPS][NR][2];
  u32x4 sraw[2];  // W4: raw group scales of the lane's 8 columns
  uint32_t zr[2];  // W4: their zeros (read when the job has a zeros tensor)
};

// A unit's place: job descriptor (uniform), tile, K split.
struct UnitPos {
  ChainJob J;
  int tile, split;
};

__device__ __forceinline__ UnitPos decode_unit(const ChainJob* __restrict__ jobs, const int* __restrict__ unit_job,
                                               int u) {
  UnitPos p;
  const int e = (int)__builtin_amdgcn_readfirstlane((uint32_t)unit_job[u]);
  p.J = jobs[e & (kMaxJobs - 1)];
  const int local = e >> kJobBits;
  p.tile = local / p.J.splits;
  p.split = local - p.tile * p.J.splits;
  return p;
}

// The wave's first K row and 32-wide steps of a unit.
template <bool W4>
__device__ __forceinline__ void wave_range(const UnitPos& P, int* k0, int* nsteps) {
  const int kw = P.J.wsteps * 32;
  const int wave = threadIdx.x >> 6;
  *k0 = P.split * (CW * kw) + wave * kw;
  *nsteps = max(0, min(P.J.wsteps, (P.J.K - *k0) / 32));  // W4: 0 or 4 (K % 128 == 0)
}

// Issues the weight loads of step i of the wave's range into one ring slot.  Steps past
// the range (the last split of a K that is not a multiple of the unit) load the wave's
// last in-range step again, or step 0 of the matrix if it has none: every register is
// written, so none stays live from the previous unit.
template <bool W4>
__device__ __forceinline__ void load_w_step(const UnitPos& P, int k0, int nsteps, int i,
                                            uint32_t (&w)[UnitRegs<W4>::NR][2]) {
  constexpr int NR = UnitRegs<W4>::NR;
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int N = P.J.N;
  const int col = P.tile * TNC + j * 8;  // lane's first column; N % 16 == 0, so col < N => col + 8 <= N
  const int ccl = col < N ? col : 0;
  const int kb = nsteps > 0 ? k0 : 0;
  const int slast = nsteps > 0 ? nsteps - 1 : 0;
  const int sc = i < slast ? i : slast;
  const long long r0 = W4 ? (long long)((kb + 32 * sc) / 2 + 4 * g) : (long long)(kb + 32 * sc + 8 * g);
  const uint8_t* base = P.J.w + r0 * N + ccl;
#pragma unroll
  for (int r = 0; r < NR; ++r) ld8<8>(base + (long long)r * N, w[r]);
}

// Issues the W4 scale and zero loads of group `grp` of the wave's range (clamped to the
// matrix's last group).  Jobs without zeros read the scales' address instead, and the
// fold uses z = 8: no load is merged at a control-flow join.
__device__ __forceinline__ void load_group(const UnitPos& P, int k0, int grp, UnitRegs<true>& R) {
  const int lane = threadIdx.x & 63, j = lane & 15;
  const int K = P.J.K, N = P.J.N;
  const int col = P.tile * TNC + j * 8;
  const int ccl = col < N ? col : 0;
  const int gi = min(k0 / 128 + grp, K / 128 - 1);
  const long long idx = (long long)gi * N + ccl;
  const bool f32 = P.J.sdt == DT_F32;
  const uint8_t* sb = (const uint8_t*)P.J.s + idx * (f32 ? 4 : 2);
  R.sraw[0] = ld_global_nt<u32x4>(sb);
  R.sraw[1] = ld_global_nt<u32x4>(sb + (f32 ? 16 : 0));
  ld8<8>(P.J.z ? P.J.z + idx : sb, R.zr);
}

// Issues every load of a unit's first RING steps (weights, W4 scales and zeros; nothing
// waits for them here).
template <bool W4>
__device__ __forceinline__ void issue_loads(const UnitPos& P, UnitRegs<W4>& R) {
  constexpr int STEPS = UnitRegs<W4>::STEPS;
  const int lane = threadIdx.x & 63, j = lane & 15;
  const int K = P.J.K, N = P.J.N;
  int k0, nsteps;
  wave_range<W4>(P, &k0, &nsteps);
  const int col = P.tile * TNC + j * 8;
  const int ccl = col < N ? col : 0;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) load_w_step<W4>(P, k0, nsteps, s, R.w[s]);
  if constexpr (W4) load_group(P, k0, 0, R);
  (void)K;
  (void)ccl;
}

// Activations of step i of the wave's range, device-coherent (an earlier job may have
// written them).  Every step is loaded (no branch around the accumulators): a step past
// the wave's range, a row past M, or any step when `now` is false reads at an offset
// beyond the buffer's range, which returns zeros and moves no data.
__device__ __forceinline__ u32x4 load_x_step(const UnitPos& P, __amdgpu_buffer_rsrc_t xr, int M, bool now, int k0,
                                             int nsteps, int i) {
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const unsigned off = (unsigned)(((long long)j * P.J.ldx + k0 + 32 * i + 8 * g) * 2);
  return ld_x_coherent(xr, (now && i < nsteps && j < M) ? off : 0xFFFFFFF0u);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t x_rsrc(const UnitPos& P, int M) {
  return part_rsrc(P.J.x, (unsigned)(((long long)(M - 1) * P.J.ldx + P.J.K) * 2));
}

// The activations of a unit's first RING steps.
template <bool W4>
__device__ __forceinline__ void load_x(const UnitPos& P, int M, bool now, u32x4 xv[UnitRegs<W4>::STEPS]) {
  constexpr int STEPS = UnitRegs<W4>::STEPS;
  int k0, nsteps;
  wave_range<W4>(P, &k0, &nsteps);
  const __amdgpu_buffer_rsrc_t xr = x_rsrc(P, M);
#pragma unroll
  for (int s = 0; s < STEPS; ++s) xv[s] = load_x_step(P, xr, M, now, k0, nsteps, s);
}

// M <= 4: the activations of one ring cycle (RING steps, 128 K rows of rows 0-3)
// in one 64-lane load, lane 16 r + c holding row r, K rows k0 + 128 cyc + 8 c .. + 7 (two
// whole 128-byte lines per row), instead of RING loads with 4 M of 64 lanes active and
// half a line per row each.  Rows past M, steps past the wave's range and any step when
// `now` is false read zeros, as in load_x_step.
__device__ __forceinline__ u32x4 load_x_cycle(const UnitPos& P, __amdgpu_buffer_rsrc_t xr, int M, bool now, int k0,
                                              int nsteps, int cyc) {
  const int lane = threadIdx.x & 63, r = lane >> 4, c = lane & 15;
  const int step = RING * cyc + (c >> 2);
  const unsigned off = (unsigned)(((long long)r * P.J.ldx + k0 + 128 * cyc + 8 * c) * 2);
  return ld_x_coherent(xr, (now && step < nsteps && r < M) ? off : 0xFFFFFFF0u);
}

// The first ring cycle's activations of a unit (one load per lane).
__device__ __forceinline__ u32x4 load_x_first_cycle(const UnitPos& P, int M, bool now) {
  int k0, nsteps;
  wave_range<false>(P, &k0, &nsteps);
  return load_x_cycle(P, x_rsrc(P, M), M, now, k0, nsteps, 0);
}

// Step s's MFMA operand from a cycle's activations: lane (j, g) takes row j, K rows
// 32 s + 8 g .. + 7, which lane 16 j + 4 s + g holds.  Rows 4-15 take a copy of row j & 3
// (no select: it would put each permute under a branch); MFMA rows are independent and
// the workgroup sum reads rows below M only.
__device__ __forceinline__ u32x4 x_of_step(const u32x4 xc, int s) {
  const int lane = threadIdx.x & 63, j = lane & 15, g = lane >> 4;
  const int src = ((j & 3) * 16 + 4 * s + g) * 4;
  u32x4 v;
  v.x = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)xc.x);
  v.y = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)xc.y);
  v.z = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)xc.z);
  v.w = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)xc.w);
  return v;
}

// Keeps a ring slot's refill where the source puts it: right after the slot's MFMAs,
// activations first.  Left to itself the scheduler sinks every refill of a ring cycle
// below the cycle's last MFMA, and the first step of the next cycle then waits for all
// of them (the counter is in order), so a wave had no loads in flight while it
// computed.
__device__ __forceinline__ void refill_fence() { __builtin_amdgcn_sched_barrier(0); }

// One 32-wide W8 step: 8 MFMAs of the lane's 8 columns against the step's activations.
__device__ __forceinline__ void w8_step(const uint32_t (&w)[8][2], u32x4 x, f32x4 (&acc)[8]) {
  const f16x8 av = bitcast<f16x8>(x);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int q = t >> 2, b = t & 3;
    u32x4 bw;
    bw.x = w8_pair_f16(w[0][q], w[1][q], b);
    bw.y = w8_pair_f16(w[2][q], w[3][q], b);
    bw.z = w8_pair_f16(w[4][q], w[5][q], b);
    bw.w = w8_pair_f16(w[6][q], w[7][q], b);
    acc[t] = mfma_f16(av, bitcast<f16x8>(bw), acc[t]);
  }
}

// Level L's tile count reaches need[L] (the level's tiles) -> its done flag (one per
// 128-byte line from flag_off) is set by the unit whose tile completed it.
__device__ __forceinline__ unsigned* level_flag(uint8_t* plan, const ChainHdr& H, int l) {
  return (unsigned*)(plan + H.flag_off) + 32 * l;
}

// The read-only parts of the plan (job descriptors, unit table, level sizes) come as
// separate restrict-qualified arguments so that the compiler reads them with scalar
// loads: the descriptors' pointers then stay in scalar registers.
template <bool W4, bool XC>
__global__ __launch_bounds__(CT) __attribute__((amdgpu_waves_per_eu(3))) void chain_kernel(uint8_t* plan, const ChainJob* __restrict__ jobs,
                                                   const int* __restrict__ unit_job,
                                                   const unsigned* __restrict__ need) {
  constexpr int STEPS = UnitRegs<W4>::STEPS;
  const ChainHdr H = *(const ChainHdr*)plan;
  unsigned* const cnt = (unsigned*)(plan + H.cnt_off);
  __shared__ __attribute__((aligned(16))) float red[CW * 16 * TNP];
  __shared__ int s_unit, s_flag;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int j = lane & 15, g = lane >> 4;
  const int M = H.M;
  const int R4 = ((M + 3) >> 2) * 4;
  const int nch = M * (TNC / 4);  // 4-column chunks of a tile's real rows
  const long long MT = (long long)M * TNC;

  // Workgroup b takes units from queue q = b % 8 (unit q + 8 i for the i-th take):
  // every queue hands its units out in increasing order, so a unit only waits for units
  // taken before it (in its own queue or in another, whose workgroups run).
  const int q = (int)(blockIdx.x % kQueues);
  unsigned* const queue = cnt + 32 * q;
  if (tid == 0)
    s_unit = (int)__hip_atomic_fetch_add(queue, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * kQueues + q;
  __syncthreads();
  int u = s_unit;
  UnitRegs<W4> R;
  UnitPos P;
  u32x4 xv[STEPS];
  u32x4 xc = u32x4{0u, 0u, 0u, 0u};  // XC: the current ring cycle's activations
  // a level-0 unit's activations go out with its weights; a later level's after its wait
  if (u < H.nunits) {
    P = decode_unit(jobs, unit_job, u);
    issue_loads<W4>(P, R);
    if constexpr (XC) xc = load_x_first_cycle(P, M, P.J.level == 0);
    else load_x<W4>(P, M, P.J.level == 0, xv);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // see the reload of a dependent unit's activations
  }
  while (u < H.nunits) {
    // the next unit's index, fetched now and read after this unit's partial stores
    int nxt = 0;
    if (tid == 0) nxt = (int)__hip_atomic_fetch_add(queue, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * kQueues + q;
    const ChainJob& J = P.J;
    const int N = J.N, S = J.splits, tile = P.tile, split = P.split;
    int k0, nsteps;
    wave_range<W4>(P, &k0, &nsteps);

    // ---------------- dependency: level L waits for every tile of level L-1 ----------------
    if (J.level > 0) {
      if (tid == 0) {
        const unsigned* f = level_flag(plan, H, J.level - 1);
        int spins = 0, nap = 1;
        while (ld_agent(f) == 0u) {
          if (++spins > kSpinLimit) {
            __hip_atomic_store((int*)(plan + offsetof(ChainHdr, err_run)), 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
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

    // ---------------- activations of a dependent unit, read after its wait ----------------
    // The wait makes this path enter the ring cycles with nothing in flight.  Otherwise
    // these activations, loaded after the whole ring of weights, would make the wait
    // insertion assume that order at the top of every ring cycle (where it merges with
    // the cycles' own in-order refills, activations first) and drain the ring there.
    if (J.level > 0) {
      if constexpr (XC) xc = load_x_first_cycle(P, M, true);
      else load_x<W4>(P, M, true, xv);
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
    }

    // The next unit is made known before this unit's last ring cycle (its index was
    // fetched at this unit's start, so that atomic's latency is hidden), and the last
    // cycle refills each ring slot with the next unit's step as soon as the slot's
    // MFMAs are issued: the wave's loads stay in flight across the unit boundary,
    // under this unit's fold, sum, exchange and epilogue.  Past the last unit the
    // loads need no branch either: they all read the first rows of tile 0 of this
    // unit's job, a few KB that every workgroup shares in L2 (re-reading this unit's
    // own first steps instead, long evicted, cost 10 % more HBM reads).
    int un = 0, k0n = 0, nstepsn = 0;
    bool xn_now = false;
    UnitPos Pn;
    auto publish_next = [&]() {
      if (tid == 0) s_unit = nxt;
      __syncthreads();
      un = (int)__builtin_amdgcn_readfirstlane((uint32_t)s_unit);
      const bool more = un < H.nunits;  // uniform
      Pn = decode_unit(jobs, unit_job, more ? un : u);
      if (!more) Pn.tile = 0, Pn.split = 0;
      xn_now = more && Pn.J.level == 0;
      wave_range<W4>(Pn, &k0n, &nstepsn);
      if (!more) k0n = 0, nstepsn = 0;
    };

    // ---------------- MFMA ----------------
    f32x4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (XC && !W4) {
      // as below, with each cycle's activations in one register per lane: the cycle's
      // step operands are permuted out of it at the cycle's start, and the next cycle's
      // load goes out with the refill of the first slot
      const int ncyc = J.wsteps / RING;
      const __amdgpu_buffer_rsrc_t xr = x_rsrc(P, M);
      for (int cyc = 0; cyc + 1 < ncyc; ++cyc) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) xv[s] = x_of_step(xc, s);
        static_for<0, RING>([&](auto sc) {
          constexpr int s = decltype(sc)::value;
          w8_step(R.w[s], xv[s], acc);
          refill_fence();
          if constexpr (s == 0) xc = load_x_cycle(P, xr, M, true, k0, nsteps, cyc + 1);
          load_w_step<false>(P, k0, nsteps, RING * (cyc + 1) + s, R.w[s]);
          refill_fence();
        });
      }
      publish_next();
      const __amdgpu_buffer_rsrc_t xrn = x_rsrc(Pn, M);
#pragma unroll
      for (int s = 0; s < STEPS; ++s) xv[s] = x_of_step(xc, s);
      static_for<0, RING>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        w8_step(R.w[s], xv[s], acc);
        refill_fence();
        if constexpr (s == 0) xc = load_x_cycle(Pn, xrn, M, xn_now, k0n, nstepsn, 0);
        load_w_step<false>(Pn, k0n, nstepsn, s, R.w[s]);
        refill_fence();
      });
    } else if constexpr (!W4) {
      // the wave's steps through the RING-deep register ring: each step's slot is
      // refilled with the step RING ahead as soon as its MFMAs are issued; the last
      // RING steps issue no loads
      const int ncyc = J.wsteps / RING;
      const __amdgpu_buffer_rsrc_t xr = x_rsrc(P, M);
      for (int cyc = 0; cyc + 1 < ncyc; ++cyc) {
        static_for<0, RING>([&](auto sc) {
          constexpr int s = decltype(sc)::value;
          w8_step(R.w[s], xv[s], acc);
          const int nx = RING * (cyc + 1) + s;
          refill_fence();
          xv[s] = load_x_step(P, xr, M, true, k0, nsteps, nx);
          load_w_step<false>(P, k0, nsteps, nx, R.w[s]);
          refill_fence();
        });
      }
      publish_next();
      const __amdgpu_buffer_rsrc_t xrn = x_rsrc(Pn, M);
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        w8_step(R.w[s], xv[s], acc);
        refill_fence();
        xv[s] = load_x_step(Pn, xrn, M, xn_now, k0n, nstepsn, s);
        load_w_step<false>(Pn, k0n, nstepsn, s, R.w[s]);
        refill_fence();
      }
    } else {
      // (1024 + lo, 64 + hi) operands.  One ring cycle of RING steps is one group of
      // 128; at its end the group folds scale * (acc - (c1 + z c2)) into the wave's LDS
      // slot (tot = fma(scale, d, tot), the first group a plain product), which the
      // workgroup sum below reads, and the next group's scales are loaded.
      const f16x8 boff = f16x8{(_Float16)1024.0f, (_Float16)64.0f, (_Float16)1024.0f, (_Float16)64.0f,
                               (_Float16)1024.0f, (_Float16)64.0f, (_Float16)1024.0f, (_Float16)64.0f};
      const f16x8 bone = f16x8{(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f,
                               (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};
      const int ncyc = J.wsteps / RING;
      const bool hz = J.z != nullptr;
      const __amdgpu_buffer_rsrc_t xr = x_rsrc(P, M);
      __amdgpu_buffer_rsrc_t xrn = xr;
      float* const slot = red + wave * 16 * TNP;
      // wl: 1 = refill with this unit's next steps, 2 = with the next unit's first steps
      auto cycle = [&](int cyc, auto wl) {
        constexpr int LOADS = decltype(wl)::value;
        f32x4 c1 = f32x4{0.f, 0.f, 0.f, 0.f}, c2 = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (XC) {
#pragma unroll
          for (int s = 0; s < STEPS; ++s) xv[s] = x_of_step(xc, s);
        }
        static_for<0, RING>([&](auto scc) {
          constexpr int st = decltype(scc)::value;
          const f16x8 av = bitcast<f16x8>(xv[st]);
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int qq = t >> 2, b = t & 3;
            u32x4 bw;
            bw.x = w4_pair_offset(R.w[st][0][qq], b);
            bw.y = w4_pair_offset(R.w[st][1][qq], b);
            bw.z = w4_pair_offset(R.w[st][2][qq], b);
            bw.w = w4_pair_offset(R.w[st][3][qq], b);
            acc[t] = mfma_f16(av, bitcast<f16x8>(bw), acc[t]);
          }
          c1 = mfma_f16(av, boff, c1);
          c2 = mfma_f16(av, bone, c2);
          refill_fence();
          if constexpr (LOADS == 1) {
            const int nx = RING * (cyc + 1) + st;
            if constexpr (!XC) xv[st] = load_x_step(P, xr, M, true, k0, nsteps, nx);
            else if constexpr (st == 0) xc = load_x_cycle(P, xr, M, true, k0, nsteps, cyc + 1);
            load_w_step<true>(P, k0, nsteps, nx, R.w[st]);
          } else {
            if constexpr (!XC) xv[st] = load_x_step(Pn, xrn, M, xn_now, k0n, nstepsn, st);
            else if constexpr (st == 0) xc = load_x_cycle(Pn, xrn, M, xn_now, k0n, nstepsn, 0);
            load_w_step<true>(Pn, k0n, nstepsn, st, R.w[st]);
          }
          refill_fence();
        });
        float sc[8];
        cvt_scale4(R.sraw[0], J.sdt, sc);
        if (J.sdt == DT_F32) {
          cvt_scale4(R.sraw[1], J.sdt, sc + 4);
        } else {
          const u32x4 hi = u32x4{R.sraw[0].z, R.sraw[0].w, 0u, 0u};
          cvt_scale4(hi, J.sdt, sc + 4);
        }
        if constexpr (XC) {
          // One-load cycles put activation row j & 3 in MFMA row j, so every lane group
          // holds rows 0-3 (copies, bit for bit): lane group g folds row g, all rows in
          // one pass, with the same operations as the per-row fold below.
          if (g < M) {
            auto pick = [&](const f32x4& v) { return g == 0 ? v[0] : g == 1 ? v[1] : g == 2 ? v[2] : v[3]; };
            const float c1g = pick(c1), c2g = pick(c2);
            f32x4* const row = (f32x4*)(slot + g * TNP + j * 8);
            f32x4 o[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
            if (cyc > 0) o[0] = row[0], o[1] = row[1];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const float zt = hz ? (float)((R.zr[t >> 2] >> (8 * (t & 3))) & 0xFFu) : 8.0f;
              const float d = pick(acc[t]) - fmaf(zt, c2g, c1g);
              o[t >> 2][t & 3] = fmaf(sc[t], d, o[t >> 2][t & 3]);
            }
            row[0] = o[0];
            row[1] = o[1];
          }
        } else if (4 * g < R4) {
          float zf[8];
#pragma unroll
          for (int t = 0; t < 8; ++t) zf[t] = hz ? (float)((R.zr[t >> 2] >> (8 * (t & 3))) & 0xFFu) : 8.0f;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            // only the rows below M: the sum never reads the others (most of the fold's
            // instructions at M = 1)
            if (4 * g + r < M) {
              f32x4* const row = (f32x4*)(slot + (4 * g + r) * TNP + j * 8);
              f32x4 o[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
              if (cyc > 0) o[0] = row[0], o[1] = row[1];
              // the first group: fma with a zero addend, the product rounded once
#pragma unroll
              for (int t = 0; t < 8; ++t) {
                const float d = acc[t][r] - fmaf(zf[t], c2[r], c1[r]);
                o[t >> 2][t & 3] = fmaf(sc[t], d, o[t >> 2][t & 3]);
              }
              row[0] = o[0];
              row[1] = o[1];
            }
          }
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        if constexpr (LOADS == 1) load_group(P, k0, cyc + 1, R);
        else load_group(Pn, k0n, 0, R);
      };
      for (int cyc = 0; cyc + 1 < ncyc; ++cyc) cycle(cyc, std::integral_constant<int, 1>{});
      publish_next();
      xrn = x_rsrc(Pn, M);
      cycle(ncyc - 1, std::integral_constant<int, 2>{});
    }

    // ---------------- workgroup sum over the 4 waves (wave order) ----------------
    // (W4 waves have folded their groups into their slots already)
    if (!W4 && 4 * g < R4) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * 16 + 4 * g + r) * TNP + j * 8 + t] = acc[t][r];
    }
    __syncthreads();
    float* const part = (float*)(plan + H.part_off) + J.part;
    const __amdgpu_buffer_rsrc_t pr = part_rsrc(part, (unsigned)((long long)J.ntiles * S * MT * 4));
    f32x4 v[2];  // chunks tid and tid + 256 (M <= 16: at most 512 chunks)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + CT * i;
      v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (c < nch) {
        const int row = c >> 5, cc = (c & 31) * 4;
        f32x4 sum = *(const f32x4*)&red[row * TNP + cc];
#pragma unroll
        for (int wv = 1; wv < CW; ++wv) sum = sum + *(const f32x4*)&red[(wv * 16 + row) * TNP + cc];
        v[i] = sum;
      }
    }
    if (S > 1) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = tid + CT * i;
        if (c < nch) st_coherent(v[i], pr, (unsigned)((((long long)tile * S + split) * MT + c * 4) * 4));
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0);  // every partial store of this thread has completed
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    __syncthreads();  // (split-K: every partial store of the workgroup has completed)

    // ---------------- split-K: the last unit of a tile to arrive sums the splits in order ----------------
    bool finish = true;
    if (S > 1) {
      if (tid == 0) {
        unsigned* cp = cnt + kLevel0 + 32 * H.nlevels + 16 * H.njobs + J.cnt0 + tile;
        const unsigned prev = __hip_atomic_fetch_add(cp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = prev == (unsigned)(S - 1);
        if (last) __hip_atomic_store(cp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_flag = last;
      }
      __syncthreads();
      finish = s_flag != 0;  // uniform
      if (finish) {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int c = tid + CT * i;
          if (c < nch) {
            const unsigned off = (unsigned)(((long long)tile * S * MT + c * 4) * 4);
            f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
            for (int p0 = 0; p0 < S; p0 += 8) {
              f32x4 pp[8];
#pragma unroll
              for (int q = 0; q < 8; ++q) pp[q] = ld_coherent(pr, off + (unsigned)(min(p0 + q, S - 1) * MT * 4));
#pragma unroll
              for (int q = 0; q < 8; ++q)
                if (p0 + q < S) sum = (p0 + q == 0) ? pp[q] : sum + pp[q];
            }
            v[i] = sum;
          }
        }
      }
    }

    // ---------------- epilogue: column scale (W8), residual, 16-bit store, level count ----------------
    if (finish) {
      const __amdgpu_buffer_rsrc_t orr = part_rsrc(J.out, (unsigned)(((long long)(M - 1) * J.ldo + N) * 2));
      const __amdgpu_buffer_rsrc_t rr =
          part_rsrc(J.res ? J.res : J.out, (unsigned)(((long long)(M - 1) * (J.res ? J.ldr : J.ldo) + N) * 2));
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = tid + CT * i;
        if (c < nch) {
          const int row = c >> 5, gc = tile * TNC + (c & 31) * 4;
          if (gc < N) {
            float cs[4] = {1.f, 1.f, 1.f, 1.f};
            if constexpr (!W4) cvt_scale4(ld_scale4_raw(J.s, J.sdt, gc), J.sdt, cs);
            float y[4];
            if (J.res) {
              const u32x2 rv = bitcast<u32x2>(
                  __builtin_amdgcn_raw_buffer_load_b64(rr, (unsigned)(((long long)row * J.ldr + gc) * 2), 0, kCpolSc1));
              const uint32_t rw[2] = {rv.x, rv.y};
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const uint16_t h = (uint16_t)(rw[e >> 1] >> (16 * (e & 1)));
                y[e] = fmaf(v[i][e], cs[e], J.odt == DT_BF16 ? bf16_to_f32(h) : (float)bitcast<_Float16>(h));
              }
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e) y[e] = v[i][e] * cs[e];
            }
            u32x2 o;
            o.x = (uint32_t)to_out16(y[0], J.odt) | ((uint32_t)to_out16(y[1], J.odt) << 16);
            o.y = (uint32_t)to_out16(y[2], J.odt) | ((uint32_t)to_out16(y[3], J.odt) << 16);
            __builtin_amdgcn_raw_buffer_store_b64(o, orr, (unsigned)(((long long)row * J.ldo + gc) * 2), 0, kCpolSc1);
          }
        }
      }
      // The tile counts for its level; the level's last tile sets the level's flag (one
      // atomic on the critical path between levels).  The last level has no reader of its
      // flag (the kernel's end publishes its outputs), so its tiles skip the count and the
      // wait for their stores, which on this hardware also waits for the next unit's
      // ring loads issued before them.
      if (J.level + 1 < H.nlevels) {  // uniform
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);  // the tile's output has reached the coherence point
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        if (tid == 0) {
          const unsigned pl =
              __hip_atomic_fetch_add(cnt + kLevel0 + 32 * J.level, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (pl + 1 == need[J.level])
            __hip_atomic_store(level_flag(plan, H, J.level), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    __syncthreads();  // every thread is done with red, s_unit and s_flag of this unit
    P = Pn;
    u = un;
  }
  // the last workgroup to leave resets the queue, exit and level counters and flags
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(cnt + 32 * kQueues, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == gridDim.x - 1) {
      for (int l = 0; l < H.nlevels; ++l) {
        __hip_atomic_store(cnt + kLevel0 + 32 * l, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(level_flag(plan, H, l), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      for (int qq = 0; qq < kQueues; ++qq) __hip_atomic_store(cnt + 32 * qq, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(cnt + 32 * kQueues, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int* const er = (int*)(plan + offsetof(ChainHdr, err_run));
      const int e = __hip_atomic_load(er, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store((int*)(plan + offsetof(ChainHdr, err)), e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(er, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ------------------------------------------------------------------ host side

struct Layout {
  long long jobs_off, unit_off, need_off, cnt_off, flag_off, part_off, bytes;
  int nunits, nlevels, ncnt, w4;
  long long part_floats;
};

long long align256(long long v) { return (v + 255) / 256 * 256; }

int fail_chain(int code, const char* fmt, int i, int a = 0, int b = 0) {
  char msg[256];
  snprintf(msg, sizeof(msg), fmt, i, a, b);
  return set_error(code, msg);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Validates the jobs and computes the plan layout (and, if `jobs_out`, the descriptors).
//
// Unit length: each wave of a unit folds RING steps of 32 K rows (the shortest unit, KU
// = 512 rows per unit) or, for levels with many units, a multiple of that streamed
// through the ring: r = (the level's shortest units) / (kLongFactor * kPlanSlots), at
// most kMaxR (2048 rows) and a tile's whole K.  Within a level, jobs are laid out longest unit first, so the
// queues hand out the long units early and the short ones fill the end.
int layout_chain(const qlin_chain_job* jobs, int njobs, int M, Layout* L, std::vector<ChainJob>* jobs_out,
                 std::vector<int>* unit_job, std::vector<unsigned>* need) {
  if (!jobs || njobs <= 0) return set_error(QLIN_ERR_INVALID, "qlin_chain: no jobs");
  if (njobs > kMaxJobs) return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: %d jobs (at most %d)", njobs, kMaxJobs);
  if (M < 1 || M > 16) return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: M=%d (1-16 rows)", M);
  int prev_level = 0;
  const bool w4_chain = jobs[0].group != 0;
  std::vector<long long> level_units;  // units per level at the shortest unit length
  for (int i = 0; i < njobs; ++i) {
    const qlin_chain_job& q = jobs[i];
    const bool w4 = q.group != 0;
    if (q.K <= 0 || q.N <= 0) return fail_chain(QLIN_ERR_INVALID, "qlin_chain: job %d: bad sizes K=%d N=%d", i, q.K, q.N);
    if (w4 && q.group != 128)
      return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d: W4 group %d (group 128 only)", i, q.group);
    if (q.K % (w4 ? 128 : 32) != 0)
      return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d: K=%d not a multiple of %d", i, q.K, w4 ? 128 : 32);
    if (q.N % 16 != 0) return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d: N=%d not a multiple of 16", i, q.N);
    if (!q.x || !q.w || !q.scale || !q.out) return fail_chain(QLIN_ERR_INVALID, "qlin_chain: job %d: null pointer", i);
    if (!aligned16(q.x) || !aligned16(q.w) || !aligned16(q.scale) || (q.zero && !aligned16(q.zero)) ||
        !aligned16(q.out) || (q.residual && !aligned16(q.residual)))
      return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d: pointers must be 16-byte aligned", i);
    if (q.ldx < q.K || q.ldx % 8 != 0 || q.ldo < q.N || q.ldo % 4 != 0 ||
        (q.residual && (q.ldr < q.N || q.ldr % 4 != 0)))
      return fail_chain(QLIN_ERR_INVALID, "qlin_chain: job %d: row strides (ldx >= K, multiple of 8; ldo/ldr >= N, multiple of 4)", i);
    if (q.scale_dtype != QLIN_F16 && q.scale_dtype != QLIN_BF16 && q.scale_dtype != QLIN_F32)
      return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d: scale dtype %d", i, q.scale_dtype);
    if (q.out_dtype != QLIN_F16 && q.out_dtype != QLIN_BF16)
      return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d: output dtype %d", i, q.out_dtype);
    if (!w4 && q.zero) return fail_chain(QLIN_ERR_INVALID, "qlin_chain: job %d: zeros given for a W8 job", i);
    if (w4 != w4_chain)
      return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d: a chain holds W8 jobs or W4 jobs, not both", i);
    if (q.level < 0 || q.level < prev_level || q.level > prev_level + 1 || (i == 0 && q.level != 0))
      return fail_chain(QLIN_ERR_INVALID, "qlin_chain: job %d: level %d (levels start at 0 and rise by at most 1)", i,
                        q.level);
    // byte offsets within 32-bit buffer ranges
    if (((long long)(M - 1) * q.ldx + q.K) * 2 >= (1LL << 31) || ((long long)(M - 1) * q.ldo + q.N) * 2 >= (1LL << 31))
      return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d: activation or output too large", i);
    const int ntiles = (q.N + TNC - 1) / TNC;
    if ((long long)ntiles * ((q.K + KU - 1) / KU) * M * TNC * 4 >= (1LL << 31))
      return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d: partials too large", i);
    prev_level = q.level;
    if ((int)level_units.size() <= q.level) level_units.resize(q.level + 1, 0);
    level_units[q.level] += (long long)ntiles * ((q.K + KU - 1) / KU);
  }
  const int nlevels = prev_level + 1;
  // per job: steps per wave, and the layout order (level, then longest unit first)
  std::vector<int> wsteps(njobs), order(njobs);
  for (int i = 0; i < njobs; ++i) {
    const qlin_chain_job& q = jobs[i];
    const long long lr = level_units[q.level] / ((long long)kLongFactor * kPlanSlots);
    const int r = (int)std::max<long long>(1, std::min<long long>(std::min<long long>(lr, kMaxR), (q.K + KU - 1) / KU));
    wsteps[i] = RING * r;
    order[i] = i;
  }
  auto unit_rows = [&](int i) { return std::min(jobs[i].K, CW * wsteps[i] * 32); };
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
    if (jobs[a].level != jobs[b].level) return jobs[a].level < jobs[b].level;
    return unit_rows(a) > unit_rows(b);
  });
  long long units = 0, ncnt = 0, parts = 0;
  std::vector<int> job_units;
  for (int oi = 0; oi < njobs; ++oi) {
    const int i = order[oi];
    const qlin_chain_job& q = jobs[i];
    const bool w4 = q.group != 0;
    const int ku = CW * wsteps[i] * 32;
    const int splits = (q.K + ku - 1) / ku;
    const int ntiles = (q.N + TNC - 1) / TNC;
    if (jobs_out) {
      ChainJob d;
      memset(&d, 0, sizeof(d));
      d.x = (const _Float16*)q.x;
      d.ldx = q.ldx;
      d.w = (const uint8_t*)q.w;
      d.s = q.scale;
      d.z = q.zero;
      d.out = q.out;
      d.ldo = q.ldo;
      d.res = q.residual;
      d.ldr = q.residual ? q.ldr : 0;
      d.part = parts;
      d.K = q.K;
      d.N = q.N;
      d.wk = w4 ? WK_W4 : WK_W8;
      d.sdt = q.scale_dtype;
      d.odt = q.out_dtype;
      d.ntiles = ntiles;
      d.splits = splits;
      d.unit0 = (int)units;
      d.cnt0 = (int)ncnt;
      d.level = q.level;
      d.index = i;
      d.wsteps = wsteps[i];
      jobs_out->push_back(d);
      job_units.push_back((int)((long long)ntiles * splits));
      if ((long long)ntiles * splits >= (1LL << (31 - kJobBits)))
        return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: job %d has too many work units", i);
      if ((int)need->size() <= q.level) need->resize(q.level + 1, 0u);
      (*need)[q.level] += (unsigned)ntiles;  // tiles of the level
    }
    units += (long long)ntiles * splits;
    if (splits > 1) {
      ncnt += ntiles;
      parts += (long long)ntiles * splits * M * TNC;
    }
    if (units > (1LL << 30)) return fail_chain(QLIN_ERR_UNSUPPORTED, "qlin_chain: too many work units (job %d)", i);
  }
  if (jobs_out) {
    // The unit order within a level: round robin over its jobs by unit index (the
    // first unit of every job, then the second, ...), so the units in flight at any
    // time read the same tiles of many matrices rather than neighbouring tiles of one
    // (QLIN_CHAIN_ORDER=0: each job's units together).
    const char* eo = getenv("QLIN_CHAIN_ORDER");
    const bool rr = !(eo && strcmp(eo, "0") == 0);
    int first = 0;
    while (first < njobs) {
      int last = first;
      while (last < njobs && jobs[order[last]].level == jobs[order[first]].level) ++last;
      if (rr) {
        int most = 0;
        for (int oi = first; oi < last; ++oi) most = std::max(most, job_units[oi]);
        for (int r = 0; r < most; ++r)
          for (int oi = first; oi < last; ++oi)
            if (r < job_units[oi]) unit_job->push_back(oi | (r << kJobBits));
      } else {
        for (int oi = first; oi < last; ++oi)
          for (int r = 0; r < job_units[oi]; ++r) unit_job->push_back(oi | (r << kJobBits));
      }
      first = last;
    }
  }
  L->nunits = (int)units;
  L->nlevels = nlevels;
  L->ncnt = (int)(kLevel0 + 32LL * L->nlevels + 16LL * njobs + ncnt);
  L->part_floats = parts;
  L->jobs_off = align256(sizeof(ChainHdr));
  L->unit_off = align256(L->jobs_off + (long long)njobs * sizeof(ChainJob));
  L->need_off = align256(L->unit_off + units * 4);
  L->w4 = w4_chain ? 1 : 0;
  L->cnt_off = align256(L->need_off + (long long)L->nlevels * 4);
  L->flag_off = align256(L->cnt_off + (long long)L->ncnt * 4);
  L->part_off = align256(L->flag_off + (long long)L->nlevels * 128);
  L->bytes = align256(L->part_off + parts * 4);
  return QLIN_OK;
}

std::mutex g_mu;
int g_grid[64][4][2];                    // per device, kernel variant and grid form (below): workgroups
struct PlanInfo {
  const void* plan;
  int w4, M, nlevels;
  long long jobs_off, unit_off, need_off;
};

// Kernel variant of a plan: 0 W8, 1 W4, 2 W8 and 3 W4 with one activation load per ring
// cycle (M = 2-4; QLIN_CHAIN_XC=0 turns it off).  Every variant gives the same bits.  At
// M = 1 the per-step loads have only 4 lanes active anyway, and the permutes' latency
// at each cycle's start made the one-load form 1 % slower there (measured).
int chain_variant(const PlanInfo& pi) {
  const char* e = getenv("QLIN_CHAIN_XC");
  const bool xc = pi.M >= 2 && pi.M <= 4 && !(e && strcmp(e, "0") == 0);
  if (pi.w4) return xc ? 3 : 1;
  return xc ? 2 : 0;
}
std::vector<PlanInfo> g_plans;  // plans initialized in this process

// Workgroups of a launch: every workgroup that fits (3 per CU), except for W8 chains of
// one level (the decode sweep), which take 2 per CU.  A launch's third workgroup per
// CU starts its first unit 15-40 us late (the CU issues the older waves' loads first),
// and a launch of one level ends when its slowest workgroup finishes its last unit:
// with 2 per CU each workgroup streams faster and the last units end sooner (W8 sweep
// 178.1-178.2 vs 180.4-182.0 us per launch).  W4 units carry half the bytes and run
// best with 3 per CU (106-108 vs 113-115 us), as do W8 chains with dependency levels
// (2168 vs 2088 GB/s) and W4 ones (a 9B-class 32-layer chain 1553 vs 1909 us per launch;
// the 2B-class W4 step with layer levels 338-340 vs 366-367 us).
int chain_grid(int variant, bool two_per_cu, int* grid) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) return set_error(QLIN_ERR_HIP, "qlin_chain_run: hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_grid[dev][variant][two_per_cu] == 0) {
    int cus = 0, per = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) {
      if (variant == 1) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, chain_kernel<true, false>, CT, 0);
      else if (variant == 2) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, chain_kernel<false, true>, CT, 0);
      else if (variant == 3) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, chain_kernel<true, true>, CT, 0);
      else e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, chain_kernel<false, false>, CT, 0);
    }
    if (e != hipSuccess || cus <= 0 || per <= 0) return set_error(QLIN_ERR_HIP, "qlin_chain_run: occupancy query failed");
    g_grid[dev][variant][two_per_cu] = cus * (two_per_cu ? std::min(per, 2) : per);
  }
  *grid = g_grid[dev][variant][two_per_cu];
  return QLIN_OK;
}

void remember_plan(const PlanInfo& info) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& p : g_plans)
    if (p.plan == info.plan) {
      p = info;
      return;
    }
  g_plans.push_back(info);
}

bool find_plan(const void* plan, PlanInfo* out) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& p : g_plans)
    if (p.plan == plan) {
      *out = p;
      return true;
    }
  return false;
}

}  // namespace
}  // namespace qlin

extern "C" size_t qlin_chain_bytes(const qlin_chain_job* jobs, int njobs, int M) {
  qlin::Layout L;
  if (qlin::layout_chain(jobs, njobs, M, &L, nullptr, nullptr, nullptr) != QLIN_OK) return 0;
  return (size_t)L.bytes;
}

extern "C" int qlin_chain_init(const qlin_chain_job* jobs, int njobs, int M, void* plan, size_t plan_bytes,
                               void* stream) {
  using namespace qlin;
  set_error(QLIN_OK, "");
  Layout L;
  std::vector<ChainJob> d;
  std::vector<int> uj;
  std::vector<unsigned> need;
  const int rc = layout_chain(jobs, njobs, M, &L, &d, &uj, &need);
  if (rc != QLIN_OK) return rc;
  if (!plan || plan_bytes < (size_t)L.bytes) return set_error(QLIN_ERR_WORKSPACE, "qlin_chain_init: plan buffer too small");
  if (!aligned16(plan)) return set_error(QLIN_ERR_UNSUPPORTED, "qlin_chain_init: plan must be 16-byte aligned");
  need.resize(L.nlevels, 0u);
  // header, descriptors, unit table, level sizes and zeroed counters, in one copy
  std::vector<uint8_t> img((size_t)L.part_off, 0);
  ChainHdr h;
  memset(&h, 0, sizeof(h));
  h.magic = kMagic;
  h.nunits = L.nunits;
  h.njobs = njobs;
  h.nlevels = L.nlevels;
  h.M = M;
  h.ncnt = L.ncnt;
  h.jobs_off = L.jobs_off;
  h.unit_off = L.unit_off;
  h.need_off = L.need_off;
  h.cnt_off = L.cnt_off;
  h.flag_off = L.flag_off;
  h.part_off = L.part_off;
  h.w4 = L.w4;
  h.bytes = L.bytes;
  memcpy(img.data(), &h, sizeof(h));
  memcpy(img.data() + L.jobs_off, d.data(), d.size() * sizeof(ChainJob));
  memcpy(img.data() + L.unit_off, uj.data(), uj.size() * sizeof(int));
  memcpy(img.data() + L.need_off, need.data(), need.size() * sizeof(unsigned));
  hipError_t e = hipMemcpyAsync(plan, img.data(), img.size(), hipMemcpyHostToDevice, (hipStream_t)stream);
  if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);  // img is freed on return
  if (e != hipSuccess) {
    char msg[160];
    snprintf(msg, sizeof(msg), "qlin_chain_init: copy: HIP error %d (%s)", (int)e, hipGetErrorString(e));
    return set_error(QLIN_ERR_HIP, msg);
  }
  remember_plan(PlanInfo{plan, L.w4, M, L.nlevels, L.jobs_off, L.unit_off, L.need_off});
  return QLIN_OK;
}

extern "C" int qlin_chain_run(void* plan, void* stream) {
  using namespace qlin;
  set_error(QLIN_OK, "");
  if (!plan || !aligned16(plan)) return set_error(QLIN_ERR_INVALID, "qlin_chain_run: null or misaligned plan");
  PlanInfo pi;
  if (!find_plan(plan, &pi))
    return set_error(QLIN_ERR_INVALID, "qlin_chain_run: plan not initialized by qlin_chain_init in this process");
  int grid = 0;
  const int variant = chain_variant(pi);
  const int rc = chain_grid(variant, !pi.w4 && pi.nlevels == 1, &grid);
  if (rc != QLIN_OK) return rc;
  uint8_t* const p = (uint8_t*)plan;
  const ChainJob* jobs = (const ChainJob*)(p + pi.jobs_off);
  const int* units = (const int*)(p + pi.unit_off);
  const unsigned* need = (const unsigned*)(p + pi.need_off);
  const hipStream_t st = (hipStream_t)stream;
  if (variant == 1) hipLaunchKernelGGL((chain_kernel<true, false>), dim3(grid), dim3(CT), 0, st, p, jobs, units, need);
  else if (variant == 2) hipLaunchKernelGGL((chain_kernel<false, true>), dim3(grid), dim3(CT), 0, st, p, jobs, units, need);
  else if (variant == 3) hipLaunchKernelGGL((chain_kernel<true, true>), dim3(grid), dim3(CT), 0, st, p, jobs, units, need);
  else hipLaunchKernelGGL((chain_kernel<false, false>), dim3(grid), dim3(CT), 0, st, p, jobs, units, need);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char msg[160];
    snprintf(msg, sizeof(msg), "qlin_chain_run: HIP error %d (%s)", (int)e, hipGetErrorString(e));
    return set_error(QLIN_ERR_HIP, msg);
  }
  return QLIN_OK;
}
