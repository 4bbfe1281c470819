// extern "C" entry points of libqlin.so (declared in include/qlin.h).
//
// Every entry point validates its arguments (shape, group, dtype, alignment) and
// returns a status before anything is launched; the launch plan (column tile width,
// waves per workgroup, split-K) is chosen here from K and N.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "../../include/qlin.h"
#include "qlin_dev.h"
#include "qlin_internal.h"

using namespace qlin;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(const char* fn, hipError_t e) {
  if (e == hipSuccess) return QLIN_OK;
  return fail(QLIN_ERR_HIP, "%s: HIP error %d (%s)", fn, (int)e, hipGetErrorString(e));
}

// Fill kernel behind clear_counters (a kernel node, not a memset, so a call that clears
// its counters can be captured in a graph).
__global__ void zero_u32(unsigned* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

#define QL_TRY(expr)              \
  do {                            \
    const int rc_ = (expr);       \
    if (rc_ != QLIN_OK) return rc_; \
  } while (0)


// Workspace: [counters | polling-exchange slots | partial sums].  Counters and slots
// must be zero between calls (every kernel leaves them so; the slots are used only by
// the engine decode units' polling exchange).
constexpr size_t kWorkspaceBytes = size_t(256) << 20;
constexpr size_t kCounterBytes = size_t(1) << 20;
constexpr size_t kPollBytes = size_t(4) << 20;
constexpr size_t kPartBase = kCounterBytes + kPollBytes;
constexpr int kWideTiles = 512;          // 256-column tiles at which no K split is needed
// narrow launches: most waves to spread K over, and least K per wave (measured with
// 8-wave workgroups: many short waves keep the most weight bytes in flight)
constexpr long long kTargetWavesW8 = 2048;
constexpr long long kTargetWavesW4 = 1024;
constexpr int kMinWaveKW8 = 64;
// fp16-activation W8 launches of at most this many (column tile x 32-row) units run
// one 32-row step per wave (measured: 2048x2048 and 2048x512 gain 0.4-0.9 us per
// launch; larger launches lose with that many workgroups)
constexpr long long kOneStepUnits = 1024;
constexpr int kMinWaveKW4 = 128;
// largest one-pass tile (weight bytes per set; measured with the weights streaming
// from HBM: 64 KB tiles win, 128 KB tiles lose to split-K)
constexpr long long kOnePassTileBytes = 64 * 1024;

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
bool dtype_scale_ok(int dt) { return dt == QLIN_F16 || dt == QLIN_BF16 || dt == QLIN_F32; }
bool dtype_out_ok(int dt) { return dt == QLIN_F16 || dt == QLIN_BF16; }
bool group_ok(int g) { return g == 32 || (g > 0 && g % 64 == 0); }


struct Problem {
  int act, wk, epi;
  bool hz;
  int M, K, group;
  int nsets;  // weight sets per output tile (1, or 2 for gate/up)
  int ncols;  // total output columns
};

// Fills L (kernel variant, grid, LDS) and a.kchunk / a.splits / a.ntiles / seg tiles.
// Launch-plan override for tuning sweeps: QLIN_SKINNY_PLAN="cols,waves,units" (0 keeps
// the default for that field; units = K granules of one wave).  Unset in normal use.
void plan_override(const Problem& P, int& cols, int& waves, int& upw) {
  const char* e = getenv("QLIN_SKINNY_PLAN");
  if (!e || !*e) return;
  int c = 0, w = 0, u = 0;
  if (sscanf(e, "%d,%d,%d", &c, &w, &u) != 3) return;
  if (c == 4 || c == 8 || c == 16) cols = c;
  if (P.epi != EPI_STORE && cols == 16) cols = 8;  // gate/up kernels: 4- and 8-column tiles
  if (w >= 1 && w <= 16) waves = w;  // clamped to the variant's maximum by the caller
  if (u >= 1) upw = u;
}

// ---------------------------------------------------------------------------
// Engine-signature calls with at least kRowsM rows (prefill chunks, chunk remainders)
//
// One K order for every M: the result of a row depends on (K, N) and the call kind,
// never on M, on the chunking of a prompt or on which kernel family runs, so a
// chunked prefill equals an unchunked one bit for bit.  The order is the tiled int8
// kernel's: K/64 blocks in S contiguous splits; within a split, lane 0 folds the
// blocks at even offsets and lane 1 those at odd offsets (acc = fma(float(dot),
// scale, acc) from zero, in increasing K); split value = lane 0 + lane 1; total =
// ((v0 + v1) + v2) + ...; then the W8 column scale (and residual, one rounding).
// The 16-row skinny tiles reproduce it with two waves per split (lanes == 2).
// S is chosen for the engine's 512-row chunk and then held for every M.
// Calls with fewer rows (decode: one sequence, or up to eight best-of candidates,
// engine.py:392) run the engine decode work units (echain.hip), whose results depend
// on (K, N) and the call kind only, so batch rows equal single rows; a chunk remainder
// of 1-8 rows therefore agrees with the unchunked prefill to the tolerance, not bit
// for bit.
constexpr int kRowsM = kDecodeRowsMax + 1;
constexpr int kRefChunkM = 512;

// Column tiles of 128 over the call's column ranges.
long long tiles128(const Problem& P, const SkArgs& a) {
  long long t = 0;
  for (int s = 0; s < (P.epi == EPI_STORE ? a.nseg : 1); ++s) t += (a.seg[s].n + 127) / 128;
  return t;
}

// Time models of the two kernel families for an engine call of M rows split S ways,
// fitted to MI355X measurements (both families forced, M = 17-512, W8 and W4-g128, the
// layer shapes 2048x2048, 6144x2048, 2048x8192 and gate/up 2048x6144, weights rotated
// over 600 MB so they stream from HBM):
//   tiled: 7 us + rounds of 256 workgroups x 128-wide K stages x weight sets x t_stage,
//          t_stage = 1.05 us + 2.5 ns per workgroup in the round (W4: 1.8 us + 1.6 ns),
//          + the split-K exchange (1.45 us per split, 12 ns per workgroup, 0.1 us per MB
//          of partial tiles)
//   rows:  5 us + 0.125 us (W4 0.17) per 16-row tile per million weight elements,
//          + 1.45 us per split
// t_tiled is negative where the tiled kernel does not cover the call.
void engine_times(const Problem& P, const SkArgs& a, int M, int S, double* t_tiled, double* t_rows) {
  const int nb = P.K / 64;
  *t_tiled = -1.0;
  SkArgs probe = a;
  probe.M = M;
  if (prefill_i8_ok(probe, P.wk, P.epi)) {
    const long long tiles = (long long)((M + 127) / 128) * tiles128(P, a);
    const long long wgs = tiles * S;
    const double occ = (double)std::min<long long>(wgs, 256);
    const double t_stage = (P.wk == WK_W4 ? 1.8e-6 + 1.6e-9 * occ : 1.05e-6 + 2.5e-9 * occ) * P.nsets;
    double t = 7e-6 + (double)((wgs + 255) / 256) * ((nb / S + 1) / 2) * t_stage;
    if (S > 1) t += 1.45e-6 * S + 12e-9 * wgs + 0.1e-12 * (double)wgs * P.nsets * 128 * 128 * sizeof(float);
    *t_tiled = t;
  }
  const double elems = (double)P.K * P.ncols * P.nsets / 1e6;
  *t_rows = 5e-6 + (P.wk == WK_W4 ? 0.17e-6 : 0.125e-6) * ((M + 15) / 16) * elems + (S > 1 ? 1.45e-6 * S : 0.0);
}

// Split count of the K order: the S (1, 2, 4 or 8, dividing K into ranges of at least
// two 64-wide blocks) whose faster family is fastest at the engine's 512-row chunk.
// QLIN_ENGINE_SPLITS overrides it (tuning; it changes the K order).
int engine_splits(const Problem& P, const SkArgs& a) {
  const int nb = P.K / 64;
  const char* es = getenv("QLIN_ENGINE_SPLITS");
  if (es && *es) return atoi(es);
  double best = 0.0;
  int S = 1;
  SkArgs b = a;
  b.x = nullptr;  // the choice must not depend on where the activations sit
  for (int s = 1; s <= 8; s *= 2) {
    if (nb % s != 0 || (s > 1 && nb / s < 2)) break;
    double tt, tr;
    engine_times(P, b, kRefChunkM, s, &tt, &tr);
    const double t = (tt >= 0.0 && tt < tr) ? tt : tr;
    if (s == 1 || t < best) best = t, S = s;
  }
  return S;
}

// The rows [m0, m0 + rows) of a call as a call of its own (rows are independent).
SkArgs row_block(const SkArgs& a, int m0, int rows) {
  SkArgs b = a;
  b.M = rows;
  b.x = (const int8_t*)a.x + (long long)m0 * a.K;
  b.xs = a.xs + (long long)m0 * (a.K / 64);
  if (a.out) b.out = (uint16_t*)a.out + (long long)m0 * a.ldo;
  if (a.res) b.res = (const uint16_t*)a.res + (long long)m0 * a.ldr;
  if (a.oq) b.oq = a.oq + (long long)m0 * a.ncols;
  if (a.os) b.os = a.os + (long long)m0 * (a.ncols / 64);
  if (a.pro.kind != PRO_NONE) {
    ProArgs& p = b.pro;
    p.x = (const uint16_t*)a.pro.x + (long long)m0 * a.pro.ldx;
    if (a.pro.g) p.g = (const uint16_t*)a.pro.g + (long long)m0 * a.pro.ldg;
    if (a.pro.q) p.q = a.pro.q + (long long)m0 * a.K, p.s = a.pro.s + (long long)m0 * (a.K / 64);
    p.tq = a.pro.tq + (long long)m0 * a.K;
    p.ts = a.pro.ts + (long long)m0 * (a.K / 64);
  }
  return b;
}

// Activation producer of a call (a.pro): run it as a launch of its own, writing the
// codes and scales to a.pro.tq / a.pro.ts, which the call then reads as its
// activations.
int pro_materialize(const char* fn, SkArgs& a, hipStream_t stream) {
  ProArgs p = a.pro;
  p.q = p.tq;
  p.s = p.ts;
  QL_TRY(hip_status(fn, launch_producer(p, a.M, a.K, stream)));
  a.x = p.tq;
  a.xs = p.ts;
  a.pro.kind = PRO_NONE;
  return QLIN_OK;
}

// Fused prologue for a skinny launch plan: places the code block of the workgroup's
// rows and K range after the finish layout in dynamic LDS.  False when the plan has
// no fused instantiation, the block does not fit, or the prologue would hold each
// thread for more than kProItems values (every column tile of a row tile makes the
// same codes: cheap for decode's short K ranges, slower than one producer launch for
// 16-row tiles over long ones); the caller then makes the codes with their own launch.
constexpr long long kProItems = 32;
bool pro_plan(SkLaunch& L, SkArgs& a, int K, int rows) {
  L.pro = 1;
  if (!skinny_pro_ok(L, a.group)) {
    L.pro = 0;
    return false;
  }
  const int kr = (a.lanes == 2) ? a.kchunk : std::min(K, L.waves * a.kchunk);
  const int mt = std::min(16, rows);
  const long long work = (long long)mt * kr + (a.pro.kind == PRO_RMSNORM ? (long long)mt * K : 0);
  if (work > kProItems * 64 * L.waves) {
    L.pro = 0;
    return false;
  }
  const size_t off = (L.lds + 15) & ~(size_t)15;
  const int ldq = kr + 16;  // 16 bytes of padding staggers the rows over the LDS banks
  const size_t bytes = (size_t)mt * ldq + (size_t)mt * (kr / 64) * sizeof(float) + (size_t)mt * sizeof(float);
  if (bytes > kProLdsBytes) {
    L.pro = 0;
    return false;
  }
  a.pro.lds_off = (int)off;
  a.pro.ldq = ldq;
  L.lds = off + bytes;
  return true;
}

int engine_rows(const char* fn, const Problem& P, SkArgs& a, void* workspace, size_t ws_bytes,
                hipStream_t stream, bool clear) {
  const int S = engine_splits(P, a);
  const int nb = P.K / 64;
  if (S < 1 || S > 64 || nb % S != 0 || (S > 1 && nb / S < 2))
    return fail(QLIN_ERR_UNSUPPORTED, "%s: %d K splits do not divide K=%d into ranges of at least 128", fn, S, P.K);
  // family: the tiled int8 kernel where it applies and a time model prefers it to the
  // 16-row tiles; both give the same bits.  QLIN_ENGINE_PREFILL=tiled|skinny forces one.
  const char* e = getenv("QLIN_ENGINE_PREFILL");
  const bool force_rows = e && strcmp(e, "skinny") == 0;
  const bool force_tiled = e && strcmp(e, "tiled") == 0;
  // time models of the two families (engine_times) at this M
  bool tiled = false;
  if (!force_rows) {
    double t_tiled, t_rows;
    engine_times(P, a, P.M, S, &t_tiled, &t_rows);
    tiled = t_tiled >= 0.0 && (force_tiled || t_tiled < t_rows);
  }
  // the tiled kernel has no producer prologue: make the activations first
  if (tiled && a.pro.kind != PRO_NONE) QL_TRY(pro_materialize(fn, a, stream));
  const int TN = tiled ? 128 : (S == 1 ? 64 : 128);
  long long ntiles = 0;
  for (int s = 0; s < (P.epi == EPI_STORE ? a.nseg : 1); ++s) ntiles += (a.seg[s].n + TN - 1) / TN;
  // rows per launch: the split-K partials and arrival counters of a launch must fit
  // the workspace (rows are independent, so blocks of rows give the same bits)
  const size_t part_cap = (workspace && ws_bytes > kPartBase) ? ws_bytes - kPartBase : 0;
  const int rstep = tiled ? 128 : 16;
  long long mb_rows = P.M;
  if (S > 1) {
    const double row_bytes = (double)S * P.nsets * ntiles * TN * sizeof(float);  // per row of partials
    const long long cap_rows = (long long)((double)part_cap / row_bytes) / rstep * rstep;
    const long long cnt_rows = (long long)(kCounterBytes / sizeof(unsigned)) / ntiles * rstep;
    mb_rows = std::min<long long>(P.M, std::min(cap_rows, cnt_rows));
    if (mb_rows < std::min(P.M, rstep))
      return fail(QLIN_ERR_WORKSPACE, "%s: the workspace (%zu bytes) cannot hold %d K splits of %lld columns", fn,
                  ws_bytes, S, (long long)ntiles * TN);
  }
  if (clear && S > 1) {
    // one counter per (16-row tile, column tile) at most, for the rows of one launch
    const long long n = ((mb_rows + 15) / 16) * ntiles;
    QL_TRY(hip_status(fn, clear_counters(workspace, std::min<long long>(n, kCounterBytes / sizeof(unsigned)), stream)));
  }
  for (long long m0 = 0; m0 < P.M; m0 += mb_rows) {
    const int rows = (int)std::min<long long>(mb_rows, P.M - m0);
    SkArgs b = row_block(a, (int)m0, rows);
    b.splits = S;
    b.cnt = S > 1 ? (unsigned*)workspace : nullptr;
    b.part = S > 1 ? (float*)((char*)workspace + kPartBase) : nullptr;
    hipError_t err;
    if (tiled) {
      if (!b.x || !b.xs) return fail(QLIN_ERR_INVALID, "%s: internal error: no activations for the tiled kernel", fn);
      err = launch_prefill_i8(b, P.wk, P.hz, P.epi, stream);
    } else {
      SkLaunch L;
      L.act = P.act;
      L.wk = P.wk;
      L.hz = P.hz ? 1 : 0;
      L.epi = P.epi;
      L.cols = TN / 16;
      L.waves = 2;
      L.pro = 0;
      int acc = 0;
      for (int s = 0; s < b.nseg; ++s) {
        b.seg[s].tile0 = (P.epi == EPI_STORE) ? acc : 0;
        if (P.epi == EPI_STORE) acc += (b.seg[s].n + TN - 1) / TN;
      }
      b.ntiles = (int)ntiles;
      b.kchunk = P.K / S;
      b.lanes = 2;
      const int rtiles = (rows + 15) / 16;
      if (ntiles * S > 0x7FFFFFFFLL || rtiles > 65535)
        return fail(QLIN_ERR_UNSUPPORTED, "%s: grid too large (M=%d, N=%d)", fn, P.M, P.ncols);
      L.grid = dim3((unsigned)(ntiles * S), (unsigned)rtiles, 1);
      const int rg0 = ((rows < 16 ? rows : 16) + 3) / 4;
      L.lds = ((size_t)L.waves * P.nsets * rg0 * 4 * (TN + 4) + (size_t)P.nsets * TN) * sizeof(float);
      if (b.pro.kind != PRO_NONE && !pro_plan(L, b, P.K, rows)) QL_TRY(pro_materialize(fn, b, stream));
      if (!L.pro && (!b.x || !b.xs)) return fail(QLIN_ERR_INVALID, "%s: internal error: no activations", fn);
      err = launch_skinny(L, b, stream);
    }
    if (err != hipSuccess) return hip_status(fn, err);
  }
  return QLIN_OK;
}

// Chooses the kernel variant, column tile, waves per workgroup and split-K, then launches.
// Every choice depends on K, N (and whether M > 16), never on M itself, so an output row
// is computed the same way for every M <= 16.  Engine-signature calls with kRowsM rows
// or more take engine_rows (one K order for every M).
// clear: zero the arrival counters the launch can use first (a scratch whose counters
// are not known to be zero).
int plan_and_launch(const char* fn, const Problem& P, SkArgs& a, void* workspace, size_t ws_bytes,
                    hipStream_t stream, bool clear = false) {
  // decode rows (one sequence or up to eight best-of rows) run on the engine decode
  // work units, the units an engine chain runs: a call equals its chain job bit for bit
  // (QLIN_ENGINE_DECODE=skinny keeps such calls on the skinny decode plans below, for
  // comparisons; it changes the K order)
  if (P.act == ACT_I8 && P.M <= kDecodeRowsMax && echain_covers(a, P.wk, P.M)) {
    const char* ed = getenv("QLIN_ENGINE_DECODE");
    if (!(ed && strcmp(ed, "skinny") == 0))
      return echain_engine_call(fn, a, P.wk, P.epi, P.M, workspace, ws_bytes, kCounterBytes, kPollBytes, stream,
                                clear);
  }
  if (P.act == ACT_I8 && P.M >= kRowsM) return engine_rows(fn, P, a, workspace, ws_bytes, stream, clear);
  SkLaunch L;
  L.act = P.act;
  L.wk = P.wk;
  L.hz = P.hz ? 1 : 0;
  L.epi = P.epi;
  L.pro = 0;

  auto count_tiles = [&](int tn) {
    int nt = 0;
    if (P.epi == EPI_STORE) {
      for (int s = 0; s < a.nseg; ++s) nt += (a.seg[s].n + tn - 1) / tn;
    } else {
      nt = (a.seg[0].n + tn - 1) / tn;
    }
    return nt;
  };
  // K granule of one wave's range: the MFMA step, the activation group (int8) and
  // whole W4 weight groups
  int kalign = (P.act == ACT_I8) ? 64 : 32;
  if (P.wk == WK_W4 && P.group > kalign) kalign = P.group;
  const int nunits = P.K / kalign;
  const int rtiles = (P.M + 15) / 16;
  const bool wide = P.M > 16 || count_tiles(256) >= kWideTiles;

  // Measured on MI355X: wide W8 launches stream best as single-wave workgroups over
  // 128-column tiles, wide W4 over 256-column tiles; narrow launches over 128-column
  // tiles with K spread first over the waves of one workgroup (up to 8, reduced in
  // LDS) and only then over workgroups.
  int cols = (wide && P.wk == WK_W4 && P.epi == EPI_STORE && P.M <= 16) ? 16 : 8;
  int waves = (wide && P.M <= 16) ? 1 : (wide ? 4 : (skinny_big(P.act, P.wk, P.epi, cols) ? 8 : 4)), upw = 0;
  // Narrow launches whose whole-K 64-column tile of one weight set is small read it in
  // one pass: 4-column lanes, K over the 8 waves of one workgroup, no split-K exchange
  // (partial store, arrival counter and final read are three memory round trips).
  // Larger tiles keep split-K: a CU moves only 16 bytes per cycle with 4-byte lanes.
  const long long tile_bytes = (long long)P.K * 64 / (P.wk == WK_W4 ? 2 : 1);
  if (!wide && tile_bytes <= kOnePassTileBytes) cols = 4, waves = 8;
  plan_override(P, cols, waves, upw);
  const bool one_pass = cols == 4;
  const int maxw = one_pass ? 8 : (skinny_big(P.act, P.wk, P.epi, cols) ? 8 : 4);
  if (waves > maxw) waves = maxw;
  const int TN = 16 * cols;
  const int ntiles = count_tiles(TN);
  int ntile_acc = 0;
  for (int s = 0; s < a.nseg; ++s) {
    a.seg[s].tile0 = (P.epi == EPI_STORE) ? ntile_acc : 0;
    if (P.epi == EPI_STORE) ntile_acc += (a.seg[s].n + TN - 1) / TN;
  }
  a.ntiles = ntiles;

  int splits;
  if (one_pass) {
    if (waves > nunits) waves = nunits;
    upw = (nunits + waves - 1) / waves;
    splits = 1;
  } else if (wide) {
    if (waves > nunits) waves = nunits;
    if (upw == 0) upw = (nunits + waves - 1) / waves;
    splits = (nunits + upw * waves - 1) / (upw * waves);
    if (P.M > 16) splits = 1, upw = (nunits + waves - 1) / waves;
  } else {
    // narrow N: spread K over up to kTargetWaves waves, each at least kMinWaveK deep
    const long long target = (P.wk == WK_W4) ? kTargetWavesW4 : kTargetWavesW8;
    int min_k = (P.wk == WK_W4) ? kMinWaveKW4 : kMinWaveKW8;
    if (P.act == ACT_F16 && P.wk == WK_W8 && (long long)ntiles * nunits <= kOneStepUnits) min_k = 32;
    const int min_upw = (min_k + kalign - 1) / kalign;
    if (upw == 0) {
      upw = (int)(((long long)ntiles * nunits + target - 1) / target);
      if (upw < min_upw) upw = min_upw;
    }
    if (upw > nunits) upw = nunits;
    const int chunks = (nunits + upw - 1) / upw;  // waves per tile
    if (waves > chunks) waves = chunks;
    splits = (chunks + waves - 1) / waves;
  }
  // partial sums must fit the workspace; without a workspace there is no cross-workgroup split
  const size_t part_cap = (workspace && ws_bytes > kPartBase) ? ws_bytes - kPartBase : 0;
  auto fits = [&](int s) {
    const size_t need = (size_t)s * P.nsets * (size_t)P.M * (size_t)P.ncols * sizeof(float);
    const size_t cnt_need = (size_t)rtiles * ntiles * sizeof(unsigned);
    return need <= part_cap && cnt_need <= kCounterBytes;
  };
  while (splits > 1 && !fits(splits)) {
    upw *= 2;
    splits = (nunits + upw * waves - 1) / (upw * waves);
  }
  if (splits <= 1) {
    splits = 1;
    upw = (nunits + waves - 1) / waves;
  }
  a.kchunk = upw * kalign;
  a.splits = splits;
  if (splits > 1) {
    a.cnt = (unsigned*)workspace;
    a.part = (float*)((char*)workspace + kPartBase);
  } else {
    a.cnt = nullptr;
    a.part = nullptr;
  }
  L.cols = cols;
  L.waves = waves;
  L.grid = dim3((unsigned)(ntiles * splits), (unsigned)rtiles, 1);
  // LDS: one finish-layout slot per wave ([set][row][column], rows of the first row
  // tile rounded up to 4, row stride TN + 4 floats), then the tile's column scales
  const int rg0 = (((P.M < 16) ? P.M : 16) + 3) / 4;
  L.lds = ((size_t)waves * P.nsets * rg0 * 4 * (TN + 4) + (size_t)P.nsets * TN) * sizeof(float);
  if ((long long)ntiles * splits > 0x7FFFFFFFLL || rtiles > 65535)
    return fail(QLIN_ERR_UNSUPPORTED, "%s: grid too large (M=%d, N=%d)", fn, P.M, P.ncols);
  // activation producer: fused into the prologue of narrow plans; wide plans (every
  // workgroup would redo the whole row) make the activations with a launch of their own
  if (a.pro.kind != PRO_NONE && (wide || !pro_plan(L, a, P.K, P.M))) QL_TRY(pro_materialize(fn, a, stream));
  // every launch reads its activations from memory unless its prologue makes them
  if (!L.pro && (!a.x || (P.act == ACT_I8 && !a.xs)))
    return fail(QLIN_ERR_INVALID, "%s: internal error: no activations", fn);
  if (clear && splits > 1) QL_TRY(hip_status(fn, clear_counters(workspace, (long long)rtiles * ntiles, stream)));
  return hip_status(fn, launch_skinny(L, a, stream));
}

int check_common(const char* fn, int M, int K, int N) {
  if (M < 0 || K <= 0 || N < 0) return fail(QLIN_ERR_INVALID, "%s: bad sizes M=%d K=%d N=%d", fn, M, K, N);
  return QLIN_OK;
}

int check_weight(const char* fn, const void* w, const void* s, const uint8_t* z, int n, int wk) {
  if (n == 0) return QLIN_OK;
  if (!w || !s) return fail(QLIN_ERR_INVALID, "%s: null weight or scale", fn);
  if (n % 16 != 0) return fail(QLIN_ERR_UNSUPPORTED, "%s: N=%d is not a multiple of 16", fn, n);
  if (!aligned(w, 16) || !aligned(s, 16) || (z && !aligned(z, 16)))
    return fail(QLIN_ERR_UNSUPPORTED, "%s: weight/scale/zero pointers must be 16-byte aligned", fn);
  (void)wk;
  return QLIN_OK;
}

int check_engine_act(const char* fn, const int8_t* a_q, const float* a_s, int M, int K) {
  if (M > 0 && (!a_q || !a_s)) return fail(QLIN_ERR_INVALID, "%s: null activations", fn);
  if (K % 64 != 0) return fail(QLIN_ERR_UNSUPPORTED, "%s: K=%d is not a multiple of 64", fn, K);
  if (!aligned(a_s, 4)) return fail(QLIN_ERR_UNSUPPORTED, "%s: a_s must be 4-byte aligned", fn);
  return QLIN_OK;
}

// Engine-signature calls take any N and pointers aligned to their element size only
// (the reference's kernels mask every edge, kernels/gemm.py:50-57).  The fast kernels
// need N % 16 == 0, 16-byte aligned weights, scales, zeros and 16-bit rows (row
// strides multiples of 8) and 8-byte aligned codes; a valid call outside those rules
// runs on the edge kernel (edge.hip).
int check_engine_weight(const char* fn, const void* w, const void* s, int n, int sdt) {
  if (n == 0) return QLIN_OK;
  if (!w || !s) return fail(QLIN_ERR_INVALID, "%s: null weight or scale", fn);
  if (!aligned(s, sdt == QLIN_F32 ? 4 : 2))
    return fail(QLIN_ERR_UNSUPPORTED, "%s: scales must be aligned to their element size", fn);
  return QLIN_OK;
}

bool engine_weight_fast(const void* w, const void* s, const uint8_t* z, int n) {
  return n == 0 || (n % 16 == 0 && aligned(w, 16) && aligned(s, 16) && (!z || aligned(z, 16)));
}

int check_engine_out(const char* fn, const void* p, int64_t ld, int N, const char* what) {
  if (!p) return fail(QLIN_ERR_INVALID, "%s: null %s", fn, what);
  if (ld < N) return fail(QLIN_ERR_INVALID, "%s: %s row stride %lld < N=%d", fn, what, (long long)ld, N);
  if (!aligned(p, 2)) return fail(QLIN_ERR_UNSUPPORTED, "%s: %s must be 2-byte aligned", fn, what);
  return QLIN_OK;
}

bool engine_out_fast(const void* p, int64_t ld) { return aligned(p, 16) && ld % 8 == 0; }

// A call on the edge kernel; a producer first runs as a launch of its own into the
// codes setup_pro chose.
int engine_edge(const char* fn, int wk, int epi, const int8_t* a_q, const float* a_s, int M, int K, const Seg* segs,
                int nseg, int ncols, int group, int sdt, void* out, int64_t ldo, const void* res, int64_t ldr,
                int8_t* oq, float* os, const ProArgs* pa, hipStream_t st) {
  if (pa && pa->kind != PRO_NONE) {
    ProArgs p = *pa;
    p.q = p.tq;
    p.s = p.ts;
    QL_TRY(hip_status(fn, launch_producer(p, M, K, st)));
    a_q = p.tq;
    a_s = p.ts;
  }
  EdgeArgs e;
  memset(&e, 0, sizeof(e));
  e.x = a_q;
  e.xs = a_s;
  e.M = M;
  e.K = K;
  for (int i = 0; i < nseg; ++i) e.seg[i] = segs[i];
  e.nseg = nseg;
  e.ncols = ncols;
  e.group = (wk == WK_W4) ? group : 64;
  e.sdt = sdt;
  e.epi = epi;
  e.odt = QLIN_BF16;
  e.out = out;
  e.ldo = ldo;
  e.res = res;
  e.ldr = ldr;
  e.oq = oq;
  e.os = os;
  return hip_status(fn, launch_edge(e, wk, st));
}

// Validates an activation producer (kernels/norm.py:28-57, 95-137, 168-188) for M rows
// of K columns and completes it: norm_gated reads v contiguous (row stride K), and the
// codes go to q / s or, without them, to the end of the workspace, which is taken off
// *wsb so no split-K partial reaches it.
int setup_pro(const char* fn, ProArgs& p, int M, int K, void* ws, size_t* wsb) {
  QL_TRY(check_producer(fn, p, M, K));
  if (p.q) {
    p.tq = p.q;
    p.ts = p.s;
  } else {
    const size_t qb = ((size_t)M * K + 255) & ~(size_t)255;
    const size_t sb = ((size_t)M * (K / 64) * sizeof(float) + 255) & ~(size_t)255;
    if (!ws || *wsb < kPartBase + qb + sb)
      return fail(QLIN_ERR_WORKSPACE, "%s: no room in the workspace for the activation codes", fn);
    *wsb -= qb + sb;
    p.tq = (int8_t*)ws + *wsb;
    p.ts = (float*)((char*)ws + *wsb + qb);
  }
  p.lds_off = 0;
  p.ldq = 0;
  return QLIN_OK;
}

}  // namespace

int qlin::check_producer(const char* fn, ProArgs& p, int M, int K) {
  (void)M;
  if (p.kind != PRO_RMSNORM && p.kind != PRO_GATE_MUL && p.kind != PRO_NORM_GATED)
    return fail(QLIN_ERR_INVALID, "%s: unknown producer kind %d", fn, p.kind);
  if (K % 64 != 0) return fail(QLIN_ERR_UNSUPPORTED, "%s: K=%d is not a multiple of 64", fn, K);
  if (p.xdt != QLIN_BF16 && p.xdt != QLIN_F16)
    return fail(QLIN_ERR_UNSUPPORTED, "%s: activation dtype %d (need bf16 or fp16)", fn, p.xdt);
  if (!p.x) return fail(QLIN_ERR_INVALID, "%s: null producer input", fn);
  if (p.kind == PRO_NORM_GATED) p.ldx = K;
  if (p.ldx < K || p.ldx % 8 != 0 || !aligned(p.x, 16))
    return fail(QLIN_ERR_UNSUPPORTED, "%s: producer input must be 16-byte aligned with a row stride >= K and a "
                "multiple of 8", fn);
  if (p.kind != PRO_GATE_MUL) {
    if (!p.w) return fail(QLIN_ERR_INVALID, "%s: null norm weight", fn);
    if (!dtype_scale_ok(p.wdt)) return fail(QLIN_ERR_UNSUPPORTED, "%s: norm weight dtype %d", fn, p.wdt);
    if (!aligned(p.w, 16)) return fail(QLIN_ERR_UNSUPPORTED, "%s: norm weight must be 16-byte aligned", fn);
  }
  if (p.kind != PRO_RMSNORM) {
    if (!p.g) return fail(QLIN_ERR_INVALID, "%s: null gate input", fn);
    if (p.ldg % 8 != 0 || !aligned(p.g, 16))
      return fail(QLIN_ERR_UNSUPPORTED, "%s: gate input must be 16-byte aligned with a row stride multiple of 8", fn);
  }
  if (p.kind == PRO_GATE_MUL) {
    if (p.hd <= 0 || p.hd % 8 != 0 || K % p.hd != 0)
      return fail(QLIN_ERR_UNSUPPORTED, "%s: head size %d must be a multiple of 8 dividing K=%d", fn, p.hd, K);
    if (p.ldg < 2LL * K) return fail(QLIN_ERR_INVALID, "%s: gate row stride %lld < 2 K", fn, (long long)p.ldg);
  }
  if (p.kind == PRO_NORM_GATED) {
    if ((p.hd != 128 && p.hd != 256 && p.hd != 512) || K % p.hd != 0)
      return fail(QLIN_ERR_UNSUPPORTED, "%s: head size %d (need 128, 256 or 512, dividing K=%d)", fn, p.hd, K);
    if (p.ldg < K) return fail(QLIN_ERR_INVALID, "%s: z row stride %lld < K", fn, (long long)p.ldg);
  }
  if ((p.q == nullptr) != (p.s == nullptr)) return fail(QLIN_ERR_INVALID, "%s: give both q and s, or neither", fn);
  if (p.q && (!aligned(p.q, 8) || !aligned(p.s, 4)))
    return fail(QLIN_ERR_UNSUPPORTED, "%s: q must be 8-byte aligned", fn);
  return QLIN_OK;
}

hipError_t qlin::clear_counters(void* ws, long long n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_u32, dim3((unsigned)std::min<long long>(256, (n + 255) / 256)), dim3(256), 0, stream,
                     (unsigned*)ws, (int)n);
  return hipGetLastError();
}

namespace {

int check_out16(const char* fn, const void* p, int64_t ld, int N, const char* what) {
  if (!p) return fail(QLIN_ERR_INVALID, "%s: null %s", fn, what);
  if (ld < N) return fail(QLIN_ERR_INVALID, "%s: %s row stride %lld < N=%d", fn, what, (long long)ld, N);
  if (!aligned(p, 16) || ld % 8 != 0)
    return fail(QLIN_ERR_UNSUPPORTED, "%s: %s must be 16-byte aligned with a row stride multiple of 8", fn,
                what);
  return QLIN_OK;
}

int check_group(const char* fn, int group, int K) {
  if (!group_ok(group)) return fail(QLIN_ERR_UNSUPPORTED, "%s: weight group %d (need 32 or a multiple of 64)", fn, group);
  if (K % group != 0) return fail(QLIN_ERR_INVALID, "%s: K=%d not a multiple of the group %d", fn, K, group);
  return QLIN_OK;
}


Seg make_seg(const void* w, const void* s, const uint8_t* z, int n, int col0) {
  Seg g;
  g.w = (const uint8_t*)w;
  g.s = s;
  g.z = z;
  g.n = n;
  g.col0 = col0;
  g.tile0 = 0;
  return g;
}

SkArgs base_args() {
  SkArgs a;
  memset(&a, 0, sizeof(a));
  return a;
}

// Common body of gemm_i8 / gemm_w4.
int engine_gemm(const char* fn, int wk, const int8_t* a_q, const float* a_s, int M, int K, const void* b,
                const void* b_s, int bs_dtype, const uint8_t* b_z, int group, int N, void* out, int64_t ldo,
                const void* residual, int64_t ldr, void* ws, size_t wsb, void* stream, bool clear = false,
                const ProArgs* pro = nullptr) {
  QL_TRY(check_common(fn, M, K, N));
  if (M == 0 || N == 0) return QLIN_OK;
  ProArgs pa{};
  if (pro) {
    pa = *pro;
    QL_TRY(setup_pro(fn, pa, M, K, ws, &wsb));
  } else {
    QL_TRY(check_engine_act(fn, a_q, a_s, M, K));
  }
  if (!dtype_scale_ok(bs_dtype)) return fail(QLIN_ERR_UNSUPPORTED, "%s: scale dtype %d", fn, bs_dtype);
  if (wk == WK_W4) QL_TRY(check_group(fn, group, K));
  QL_TRY(check_engine_weight(fn, b, b_s, N, bs_dtype));
  QL_TRY(check_engine_out(fn, out, ldo, N, "out"));
  if (residual) QL_TRY(check_engine_out(fn, residual, ldr, N, "residual"));
  if (!engine_weight_fast(b, b_s, b_z, N) || !engine_out_fast(out, ldo) ||
      (residual && !engine_out_fast(residual, ldr)) || (!pro && !aligned(a_q, 8))) {
    const Seg s0 = make_seg(b, b_s, b_z, N, 0);
    return engine_edge(fn, wk, EPI_STORE, a_q, a_s, M, K, &s0, 1, N, group, bs_dtype, out, ldo, residual, ldr,
                       nullptr, nullptr, pro ? &pa : nullptr, (hipStream_t)stream);
  }
  SkArgs a = base_args();
  a.x = a_q;
  a.xs = a_s;
  a.M = M;
  a.K = K;
  a.seg[0] = make_seg(b, b_s, b_z, N, 0);
  a.nseg = 1;
  a.ncols = N;
  a.group = (wk == WK_W4) ? group : 64;
  a.sdt = bs_dtype;
  a.out = out;
  a.ldo = ldo;
  a.odt = QLIN_BF16;
  a.res = residual;
  a.ldr = ldr;
  a.pro = pa;
  Problem P{ACT_I8, wk, EPI_STORE, b_z != nullptr, M, K, a.group, 1, N};
  if (clear && (!ws || wsb <= kPartBase)) return fail(QLIN_ERR_WORKSPACE, "%s: no scratch", fn);
  return plan_and_launch(fn, P, a, ws, wsb, (hipStream_t)stream, clear);
}

int engine_proj3(const char* fn, int wk, const int8_t* a_q, const float* a_s, int M, int K, const void* w1,
                 const void* s1, const uint8_t* z1, int n1, const void* w2, const void* s2, const uint8_t* z2,
                 int n2, const void* w3, const void* s3, const uint8_t* z3, int n3, int bs_dtype, int group,
                 void* out, int64_t ldo, void* ws, size_t wsb, void* stream, const ProArgs* pro = nullptr) {
  const int NT = n1 + n2 + n3;
  QL_TRY(check_common(fn, M, K, NT));
  if (n1 < 0 || n2 < 0 || n3 < 0) return fail(QLIN_ERR_INVALID, "%s: negative N", fn);
  if (M == 0 || NT == 0) return QLIN_OK;
  ProArgs pa{};
  if (pro) {
    pa = *pro;
    QL_TRY(setup_pro(fn, pa, M, K, ws, &wsb));
  } else {
    QL_TRY(check_engine_act(fn, a_q, a_s, M, K));
  }
  if (!dtype_scale_ok(bs_dtype)) return fail(QLIN_ERR_UNSUPPORTED, "%s: scale dtype %d", fn, bs_dtype);
  if (wk == WK_W4) QL_TRY(check_group(fn, group, K));
  QL_TRY(check_engine_weight(fn, w1, s1, n1, bs_dtype));
  QL_TRY(check_engine_weight(fn, w2, s2, n2, bs_dtype));
  QL_TRY(check_engine_weight(fn, w3, s3, n3, bs_dtype));
  QL_TRY(check_engine_out(fn, out, ldo, NT, "out"));
  const bool hz = (z1 || z2 || z3);
  if (hz && ((n1 && !z1) || (n2 && !z2) || (n3 && !z3)))
    return fail(QLIN_ERR_INVALID, "%s: zeros must be given for every projection or for none", fn);
  if (!engine_weight_fast(w1, s1, z1, n1) || !engine_weight_fast(w2, s2, z2, n2) ||
      !engine_weight_fast(w3, s3, z3, n3) || !engine_out_fast(out, ldo) || (!pro && !aligned(a_q, 8))) {
    Seg sg[3];
    int ns = 0, col = 0;
    const void* wv[3] = {w1, w2, w3};
    const void* sv[3] = {s1, s2, s3};
    const uint8_t* zv[3] = {z1, z2, z3};
    const int nv[3] = {n1, n2, n3};
    for (int i = 0; i < 3; ++i) {
      if (nv[i] == 0) continue;
      sg[ns++] = make_seg(wv[i], sv[i], zv[i], nv[i], col);
      col += nv[i];
    }
    return engine_edge(fn, wk, EPI_STORE, a_q, a_s, M, K, sg, ns, NT, group, bs_dtype, out, ldo, nullptr, 0,
                       nullptr, nullptr, pro ? &pa : nullptr, (hipStream_t)stream);
  }
  SkArgs a = base_args();
  a.x = a_q;
  a.xs = a_s;
  a.M = M;
  a.K = K;
  int ns = 0, col = 0;
  const void* ws_[3] = {w1, w2, w3};
  const void* ss_[3] = {s1, s2, s3};
  const uint8_t* zs_[3] = {z1, z2, z3};
  const int ns_[3] = {n1, n2, n3};
  for (int i = 0; i < 3; ++i) {
    if (ns_[i] == 0) continue;
    a.seg[ns++] = make_seg(ws_[i], ss_[i], zs_[i], ns_[i], col);
    col += ns_[i];
  }
  a.nseg = ns;
  a.ncols = NT;
  a.group = (wk == WK_W4) ? group : 64;
  a.sdt = bs_dtype;
  a.out = out;
  a.ldo = ldo;
  a.odt = QLIN_BF16;
  a.pro = pa;
  Problem P{ACT_I8, wk, EPI_STORE, hz, M, K, a.group, 1, NT};
  return plan_and_launch(fn, P, a, ws, wsb, (hipStream_t)stream);
}

int engine_gate_up(const char* fn, int wk, int epi, const int8_t* a_q, const float* a_s, int M, int K,
                   const void* wg, const void* sg, const uint8_t* zg, const void* wu, const void* su,
                   const uint8_t* zu, int bs_dtype, int group, int N, void* out, int8_t* out_q, float* out_s,
                   void* ws, size_t wsb, void* stream, const ProArgs* pro = nullptr) {
  QL_TRY(check_common(fn, M, K, N));
  if (M == 0 || N == 0) return QLIN_OK;
  ProArgs pa{};
  if (pro) {
    pa = *pro;
    QL_TRY(setup_pro(fn, pa, M, K, ws, &wsb));
  } else {
    QL_TRY(check_engine_act(fn, a_q, a_s, M, K));
  }
  if (!dtype_scale_ok(bs_dtype)) return fail(QLIN_ERR_UNSUPPORTED, "%s: scale dtype %d", fn, bs_dtype);
  if (wk == WK_W4) QL_TRY(check_group(fn, group, K));
  QL_TRY(check_engine_weight(fn, wg, sg, N, bs_dtype));
  QL_TRY(check_engine_weight(fn, wu, su, N, bs_dtype));
  if ((zg == nullptr) != (zu == nullptr))
    return fail(QLIN_ERR_INVALID, "%s: zeros must be given for both gate and up or for neither", fn);
  bool fast = engine_weight_fast(wg, sg, zg, N) && engine_weight_fast(wu, su, zu, N) && (pro || aligned(a_q, 8));
  if (epi == EPI_GATEUP) {
    QL_TRY(check_engine_out(fn, out, N, N, "out"));
    fast = fast && engine_out_fast(out, N);
  } else {
    if (N % 64 != 0) return fail(QLIN_ERR_UNSUPPORTED, "%s: N=%d is not a multiple of 64", fn, N);
    if (!out_q || !out_s) return fail(QLIN_ERR_INVALID, "%s: null out_q/out_s", fn);
    if (!aligned(out_s, 4)) return fail(QLIN_ERR_UNSUPPORTED, "%s: out_s must be 4-byte aligned", fn);
    fast = fast && aligned(out_q, 16);
  }
  if (!fast) {
    const Seg sgs[2] = {make_seg(wg, sg, zg, N, 0), make_seg(wu, su, zu, N, 0)};
    return engine_edge(fn, wk, epi, a_q, a_s, M, K, sgs, 2, N, group, bs_dtype, out, N, nullptr, 0, out_q, out_s,
                       pro ? &pa : nullptr, (hipStream_t)stream);
  }
  SkArgs a = base_args();
  a.x = a_q;
  a.xs = a_s;
  a.M = M;
  a.K = K;
  a.seg[0] = make_seg(wg, sg, zg, N, 0);
  a.seg[1] = make_seg(wu, su, zu, N, 0);
  a.nseg = 2;
  a.ncols = N;
  a.group = (wk == WK_W4) ? group : 64;
  a.sdt = bs_dtype;
  a.out = out;
  a.ldo = N;
  a.odt = QLIN_BF16;
  a.oq = out_q;
  a.os = out_s;
  a.pro = pa;
  Problem P{ACT_I8, wk, epi, zg != nullptr, M, K, a.group, 2, N};
  return plan_and_launch(fn, P, a, ws, wsb, (hipStream_t)stream);
}

// Prefill plan: the LDS-tiled kernel with a tile shape and a split-K factor, or the
// skinny kernel over row tiles, whichever a time model fitted to MI355X
// measurements (fp16 x int8, W4 about 1.3x slower per tile) prefers:
//   tiled:  fixed + rounds x (K tiles per workgroup) x t_tile(workgroups per CU)
//           + split-K: about 3 us of arrival round trips plus 0.5 us per MB of
//             partials written and read back
//   skinny: fixed + cost per (row x MB of int8-sized weights): its 16-row tiles
//           re-read the weights from L2
struct PfPlan {
  bool tiled;
  int shape;
  int splits;
  int sk;  // balanced schedule: K tiles per workgroup (0 = off)
};

PfPlan plan_prefill(int wk, int M, int K, int N, size_t part_cap) {
  // Time model fitted to MI355X measurements with the weights streaming from HBM
  // (M = 128 / 512 / 2048 on the 2048x6144, 6144x2048 and 2048x2048 shapes):
  //   tiled:  5 us + rounds x (K tiles per split) x t_tile  (x 1.3 for W4)
  //           + split-K exchange: 1.45 us per split (the last workgroup reads the
  //             splits one round trip each) + 12 ns per workgroup + 0.1 us per MB of
  //             partial tiles; a split level is tried only while the level below it
  //             leaves CUs idle (split-K exists to fill the chip)
  //   balanced: 5 us + (K tiles per workgroup) x t_tile + the exchange of the
  //             tiles shared by two workgroups (below)
  //   rows:   16-row tiles, 4 waves over the whole K per 128 columns:
  //           7.1 us (W4 5.8) + max(1, workgroups / 256) x 3.4 ns (W4 2.7) per K row
  struct Cand {
    int shape;
    int per_cu;        // workgroups one CU can hold
    double t_tile[2];  // seconds per 64-wide K tile of a workgroup, 1 or 2 per CU
  };
  const bool w4 = wk == WK_W4;
  const double w4f = w4 ? 1.3 : 1.0;
  const Cand cands[2] = {{PF_128x128_K2, 2, {0.48e-6, 1.35e-6}}, {PF_256x256, 1, {1.96e-6, 1.96e-6}}};
  const int nk = K / 64;
  PfPlan best{false, PF_128x128_K2, 1, 0};
  const double row_wgs = (double)((M + 15) / 16) * ((N + 127) / 128);
  double best_t = (w4 ? 5.8e-6 : 7.1e-6) + (row_wgs > 256 ? row_wgs / 256 : 1.0) * (w4 ? 2.7e-9 : 3.4e-9) * K;
  for (const Cand& c : cands) {
    int bm, bn, waves;
    prefill_geometry(c.shape, &bm, &bn, &waves);
    const long long tiles = (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    for (int S = 1; S <= 16; S *= 2) {
      if (nk % S != 0 || nk / S < 2) break;
      const double part_bytes = (double)tiles * S * waves * 128 * 64 * sizeof(float);
      if (S > 1 && (part_bytes > (double)part_cap || tiles > (long long)(kCounterBytes / sizeof(unsigned)))) break;
      const long long wgs = tiles * S;
      if (S > 1 && tiles * (S / 2) >= 256LL * c.per_cu) break;
      const int occ = (wgs > 256 && c.per_cu > 1) ? 2 : 1;
      const double rounds = (double)((wgs + 256LL * occ - 1) / (256LL * occ));
      const double tile_bytes = (double)wgs * bm * bn * sizeof(float);  // one partial tile per workgroup
      const double t = 5e-6 + rounds * (nk / S) * c.t_tile[occ - 1] * w4f +
                       (S > 1 ? 1.45e-6 * S + 12e-9 * wgs + 0.1e-12 * tile_bytes : 0.0);
      if (t < best_t) {
        best_t = t;
        best = PfPlan{true, c.shape, S, 0};
      }
    }
    // Balanced schedule: every CU slot gets the same run of (tile, K tile) units,
    // crossing tile boundaries.  A tile split over two workgroups moves about 1.8
    // fp32 partial tiles (one store, two when both pieces end together, and one
    // load), at about 0.22 us per MB, plus about 2 us for the second piece's
    // pipeline start (measured, W8 and W4, M = 2048: 2048x6144 in 192 tiles, where
    // this loses to one tile per workgroup, and 4096x12288 in 384 tiles, where it
    // wins by 9 %).
    const long long slots = 256LL * c.per_cu;
    const long long units = tiles * nk;
    if (tiles % slots != 0 && tiles > slots / 2 &&
        tiles <= (long long)(kCounterBytes / sizeof(unsigned)) &&
        (double)tiles * 2 * waves * 128 * 64 * sizeof(float) <= (double)part_cap) {
      const int sk = (int)((units + slots - 1) / slots);
      if (prefill_balanced_ok(tiles, nk, sk)) {
        const int occ = c.per_cu > 1 ? 2 : 1;
        const double xbytes = 1.8 * (double)tiles * bm * bn * sizeof(float);
        const double t = 5e-6 + sk * c.t_tile[occ - 1] * w4f + 2e-6 + 0.22e-12 * xbytes;
        if (t < best_t) {
          best_t = t;
          best = PfPlan{true, c.shape, 1, sk};
        }
      }
    }
  }
  return best;
}

// Tile order of a plan with one tile per workgroup (or its K splits): each XCD runs one
// contiguous eighth of the order, and the order goes down gm row tiles before the next
// column tile, so an XCD's run covers about gm row tiles x (run / gm) column tiles.
// gm minimises what one run reads into its XCD's L2: rows x (BM x K fp16 activations)
// + columns x (the weights of BN columns).  QLIN_PREFILL_GM overrides it (0: the order
// in groups of 8 row tiles with workgroups in launch order).
int prefill_tile_group(int wk, int M, int K, int N, int shape) {
  const char* e = getenv("QLIN_PREFILL_GM");
  if (e && *e) return std::max(0, atoi(e));
  int bm, bn, waves;
  prefill_geometry(shape, &bm, &bn, &waves);
  const long long tm = (M + bm - 1) / bm, tn = (N + bn - 1) / bn;
  const long long run = std::max<long long>(1, (tm * tn + 7) / 8);
  const double arow = (double)bm * K * 2.0, wcol = (double)K * bn * (wk == WK_W4 ? 0.5 : 1.0);
  int best = 1;
  double best_c = 0.0;
  for (int gm = 1; gm <= 64; gm *= 2) {
    const long long h = std::min<long long>(gm, tm);
    const long long rows = std::min(h, run), cols = (run + h - 1) / h;
    const double c = (double)rows * arow + (double)cols * wcol;
    if (gm == 1 || c < best_c) best_c = c, best = gm;
    if (gm >= tm) break;
  }
  return best;
}

int a16_linear(const char* fn, int wk, const void* x, int x_dtype, int M, int K, int64_t ldx, const void* w,
               const void* scale, int s_dtype, const uint8_t* zero, int group, int N, void* out, int out_dtype,
               int64_t ldo, const void* residual, int64_t ldr, void* ws, size_t wsb, void* stream) {
  QL_TRY(check_common(fn, M, K, N));
  if (M == 0 || N == 0) return QLIN_OK;
  if (!x) return fail(QLIN_ERR_INVALID, "%s: null x", fn);
  if (x_dtype != QLIN_F16) return fail(QLIN_ERR_UNSUPPORTED, "%s: activation dtype %d (fp16 only)", fn, x_dtype);
  if (!dtype_scale_ok(s_dtype)) return fail(QLIN_ERR_UNSUPPORTED, "%s: scale dtype %d", fn, s_dtype);
  if (!dtype_out_ok(out_dtype)) return fail(QLIN_ERR_UNSUPPORTED, "%s: output dtype %d", fn, out_dtype);
  if (K % 32 != 0) return fail(QLIN_ERR_UNSUPPORTED, "%s: K=%d is not a multiple of 32", fn, K);
  if (ldx < K) return fail(QLIN_ERR_INVALID, "%s: x row stride %lld < K", fn, (long long)ldx);
  if (!aligned(x, 16) || ldx % 8 != 0)
    return fail(QLIN_ERR_UNSUPPORTED, "%s: x must be 16-byte aligned with a row stride multiple of 8", fn);
  if (wk == WK_W4) QL_TRY(check_group(fn, group, K));
  QL_TRY(check_weight(fn, w, scale, zero, N, wk));
  QL_TRY(check_out16(fn, out, ldo, N, "out"));
  if (residual) QL_TRY(check_out16(fn, residual, ldr, N, "residual"));
  // More than 16 rows: the LDS-tiled MFMA kernel (tile shape and split-K from a time
  // model) or row tiles of 16 through the skinny kernel, whichever the model prefers.
  // QLIN_PREFILL ("skinny" or "tiled"), QLIN_PREFILL_SHAPE and QLIN_PREFILL_SPLITS
  // override the choice for tuning.
  const char* pimpl = getenv("QLIN_PREFILL");
  const bool force_skinny = pimpl && strcmp(pimpl, "skinny") == 0;
  const bool force_tiled = pimpl && strcmp(pimpl, "tiled") == 0;
  // the DMA kernel addresses activations with 32-bit byte offsets
  const bool fits32 = ((long long)(M - 1) * ldx + K) * 2 < (1LL << 31);
  const size_t part_cap = (ws && wsb > kPartBase) ? wsb - kPartBase : 0;
  if (M > 16 && K % 64 == 0 && !force_skinny) {
    TlArgs t;
    t.x = (const _Float16*)x;
    t.ldx = ldx;
    t.w = (const uint8_t*)w;
    t.s = scale;
    t.z = zero;
    t.M = M;
    t.N = N;
    t.K = K;
    t.group = (wk == WK_W4) ? group : 32;
    t.sdt = s_dtype;
    t.out = out;
    t.ldo = ldo;
    t.odt = out_dtype;
    t.res = residual;
    t.ldr = ldr;
    t.splits = 1;
    t.part = nullptr;
    t.cnt = nullptr;
    t.sk = 0;
    t.gm = 0;
    if (fits32) {
      PfPlan p = plan_prefill(wk, M, K, N, part_cap);
      if (getenv("QLIN_PREFILL_VERBOSE"))
        fprintf(stderr, "qlin prefill plan M=%d K=%d N=%d: %s shape=%d splits=%d sk=%d\n", M, K, N,
                p.tiled ? "tiled" : "skinny", p.shape, p.splits, p.sk);
      const char* e = getenv("QLIN_PREFILL_SHAPE");
      const char* e2 = getenv("QLIN_PREFILL_SPLITS");
      const char* e3 = getenv("QLIN_PREFILL_SK");
      if ((e && *e) || (e2 && *e2) || (e3 && *e3)) {
        p.tiled = true;
        if (e && *e) p.shape = atoi(e);
        p.splits = (e2 && *e2) ? atoi(e2) : 1;
        p.sk = (e3 && *e3) ? atoi(e3) : 0;
        int bm, bn, waves;
        prefill_geometry(p.shape, &bm, &bn, &waves);
        const size_t tiles = (size_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        if (!prefill_shape_ok(p.shape))
          return fail(QLIN_ERR_UNSUPPORTED, "%s: QLIN_PREFILL_SHAPE=%d unknown", fn, p.shape);
        if (p.splits < 1 || (K / 64) % p.splits != 0 ||
            (p.splits > 1 && (tiles * p.splits * waves * 128 * 64 * sizeof(float) > part_cap ||
                              tiles > kCounterBytes / sizeof(unsigned))))
          return fail(QLIN_ERR_UNSUPPORTED, "%s: QLIN_PREFILL_SPLITS=%d unusable here", fn, p.splits);
        if (p.sk != 0 && (p.sk < 0 || p.splits != 1 || !prefill_balanced_ok((long long)tiles, K / 64, p.sk) ||
                          tiles * 2 * waves * 128 * 64 * sizeof(float) > part_cap ||
                          tiles > kCounterBytes / sizeof(unsigned)))
          return fail(QLIN_ERR_UNSUPPORTED, "%s: QLIN_PREFILL_SK=%d unusable here", fn, p.sk);
      }
      if (p.tiled || force_tiled) {
        t.splits = p.splits;
        t.sk = p.sk;
        if (p.sk == 0) t.gm = prefill_tile_group(wk, M, K, N, p.shape);
        if (p.splits > 1 || p.sk > 0) {
          t.cnt = (unsigned*)ws;
          t.part = (float*)((char*)ws + kPartBase);
        }
        return hip_status(fn, launch_prefill(t, wk, zero != nullptr, p.shape, (hipStream_t)stream));
      }
    }
  }
  SkArgs a = base_args();
  a.x = x;
  a.ldx = ldx;
  a.M = M;
  a.K = K;
  a.seg[0] = make_seg(w, scale, zero, N, 0);
  a.nseg = 1;
  a.ncols = N;
  a.group = (wk == WK_W4) ? group : 32;
  a.sdt = s_dtype;
  a.out = out;
  a.ldo = ldo;
  a.odt = out_dtype;
  a.res = residual;
  a.ldr = ldr;
  Problem P{ACT_F16, wk, EPI_STORE, zero != nullptr, M, K, a.group, 1, N};
  return plan_and_launch(fn, P, a, ws, wsb, (hipStream_t)stream);
}

}  // namespace

namespace qlin {

int set_error(int code, const char* msg) { return fail(code, "%s", msg); }

int gemm_i8_scratch(const char* fn, const int8_t* a_q, const float* a_s, int M, int K, const int8_t* b,
                    const void* b_s, int bs_dtype, int N, void* out, int64_t ldo, const void* residual,
                    int64_t ldr, void* scratch, size_t scratch_bytes, void* stream) {
  g_err[0] = 0;
  return engine_gemm(fn, WK_W8, a_q, a_s, M, K, b, b_s, bs_dtype, nullptr, 64, N, out, ldo, residual, ldr,
                     scratch, scratch_bytes, stream, true);
}

size_t counter_bytes() { return kCounterBytes; }
size_t poll_bytes() { return kPollBytes; }

}  // namespace qlin

extern "C" {

int qlin_version(void) { return QLIN_ABI_VERSION; }

const char* qlin_last_error(void) { return g_err; }

size_t qlin_workspace_bytes(void) { return kWorkspaceBytes; }

int qlin_gemm_i8(const int8_t* a_q, const float* a_s, int M, int K, const int8_t* b, const void* b_s, int bs_dtype,
                 int N, void* out, int64_t ldo, const void* residual, int64_t ldr, void* workspace,
                 size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return engine_gemm("qlin_gemm_i8", WK_W8, a_q, a_s, M, K, b, b_s, bs_dtype, nullptr, 64, N, out, ldo, residual,
                     ldr, workspace, workspace_bytes, stream);
}

int qlin_gemm_w4(const int8_t* a_q, const float* a_s, int M, int K, const uint8_t* b, const void* b_s,
                 int bs_dtype, const uint8_t* b_z, int group, int N, void* out, int64_t ldo, const void* residual,
                 int64_t ldr, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return engine_gemm("qlin_gemm_w4", WK_W4, a_q, a_s, M, K, b, b_s, bs_dtype, b_z, group, N, out, ldo, residual,
                     ldr, workspace, workspace_bytes, stream);
}

int qlin_proj3_i8(const int8_t* a_q, const float* a_s, int M, int K, const int8_t* w1, const void* s1, int n1,
                  const int8_t* w2, const void* s2, int n2, const int8_t* w3, const void* s3, int n3, int bs_dtype,
                  void* out, int64_t ldo, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return engine_proj3("qlin_proj3_i8", WK_W8, a_q, a_s, M, K, w1, s1, nullptr, n1, w2, s2, nullptr, n2, w3, s3,
                      nullptr, n3, bs_dtype, 64, out, ldo, workspace, workspace_bytes, stream);
}

int qlin_proj3_w4(const int8_t* a_q, const float* a_s, int M, int K, const uint8_t* w1, const void* s1,
                  const uint8_t* z1, int n1, const uint8_t* w2, const void* s2, const uint8_t* z2, int n2,
                  const uint8_t* w3, const void* s3, const uint8_t* z3, int n3, int bs_dtype, int group, void* out,
                  int64_t ldo, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return engine_proj3("qlin_proj3_w4", WK_W4, a_q, a_s, M, K, w1, s1, z1, n1, w2, s2, z2, n2, w3, s3, z3, n3,
                      bs_dtype, group, out, ldo, workspace, workspace_bytes, stream);
}

int qlin_mlp_gate_up_i8(const int8_t* a_q, const float* a_s, int M, int K, const int8_t* wg, const void* sg,
                        const int8_t* wu, const void* su, int bs_dtype, int N, void* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return engine_gate_up("qlin_mlp_gate_up_i8", WK_W8, EPI_GATEUP, a_q, a_s, M, K, wg, sg, nullptr, wu, su, nullptr,
                        bs_dtype, 64, N, out, nullptr, nullptr, workspace, workspace_bytes, stream);
}

int qlin_mlp_gate_up_w4(const int8_t* a_q, const float* a_s, int M, int K, const uint8_t* wg, const void* sg,
                        const uint8_t* zg, const uint8_t* wu, const void* su, const uint8_t* zu, int bs_dtype,
                        int group, int N, void* out, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return engine_gate_up("qlin_mlp_gate_up_w4", WK_W4, EPI_GATEUP, a_q, a_s, M, K, wg, sg, zg, wu, su, zu, bs_dtype,
                        group, N, out, nullptr, nullptr, workspace, workspace_bytes, stream);
}

int qlin_mlp_gate_up_quant_i8(const int8_t* a_q, const float* a_s, int M, int K, const int8_t* wg, const void* sg,
                              const int8_t* wu, const void* su, int bs_dtype, int N, int8_t* out_q, float* out_s,
                              void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return engine_gate_up("qlin_mlp_gate_up_quant_i8", WK_W8, EPI_GATEUP_Q, a_q, a_s, M, K, wg, sg, nullptr, wu, su,
                        nullptr, bs_dtype, 64, N, nullptr, out_q, out_s, workspace, workspace_bytes, stream);
}

int qlin_mlp_gate_up_quant_w4(const int8_t* a_q, const float* a_s, int M, int K, const uint8_t* wg, const void* sg,
                              const uint8_t* zg, const uint8_t* wu, const void* su, const uint8_t* zu,
                              int bs_dtype, int group, int N, int8_t* out_q, float* out_s, void* workspace,
                              size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return engine_gate_up("qlin_mlp_gate_up_quant_w4", WK_W4, EPI_GATEUP_Q, a_q, a_s, M, K, wg, sg, zg, wu, su, zu,
                        bs_dtype, group, N, nullptr, out_q, out_s, workspace, workspace_bytes, stream);
}

int qlin_linear_w8(const void* x, int x_dtype, int M, int K, int64_t ldx, const int8_t* w, const void* scale,
                   int s_dtype, int N, void* out, int out_dtype, int64_t ldo, const void* residual, int64_t ldr,
                   void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return a16_linear("qlin_linear_w8", WK_W8, x, x_dtype, M, K, ldx, w, scale, s_dtype, nullptr, 32, N, out,
                    out_dtype, ldo, residual, ldr, workspace, workspace_bytes, stream);
}

int qlin_linear_w4(const void* x, int x_dtype, int M, int K, int64_t ldx, const uint8_t* w, const void* scale,
                   int s_dtype, const uint8_t* zero, int group, int N, void* out, int out_dtype, int64_t ldo,
                   const void* residual, int64_t ldr, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  return a16_linear("qlin_linear_w4", WK_W4, x, x_dtype, M, K, ldx, w, scale, s_dtype, zero, group, N, out,
                    out_dtype, ldo, residual, ldr, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Activation producers (kernels/norm.py) and the linears that make their own
// activations from them
// ---------------------------------------------------------------------------

static ProArgs pro_from(const qlin_producer* p) {
  ProArgs a{};
  a.kind = p->kind;
  a.x = p->x;
  a.ldx = p->ldx;
  a.xdt = p->x_dtype;
  a.g = p->g;
  a.ldg = p->ldg;
  a.w = p->w;
  a.wdt = p->w_dtype;
  a.hd = p->hd;
  a.one_plus = p->one_plus;
  a.eps = p->eps;
  a.q = p->q;
  a.s = p->s;
  return a;
}

static int produce(const char* fn, ProArgs p, int M, int K, void* stream) {
  if (M < 0 || K < 0) return fail(QLIN_ERR_INVALID, "%s: bad sizes M=%d K=%d", fn, M, K);
  if (M == 0 || K == 0) return QLIN_OK;
  if (!p.q || !p.s) return fail(QLIN_ERR_INVALID, "%s: null q or s", fn);
  size_t none = 0;
  QL_TRY(setup_pro(fn, p, M, K, nullptr, &none));
  return hip_status(fn, launch_producer(p, M, K, (hipStream_t)stream));
}

int qlin_rmsnorm_quant(const void* x, int64_t ldx, int x_dtype, const void* w, int w_dtype, int M, int K, float eps,
                       int one_plus, int8_t* q, float* s, void* stream) {
  g_err[0] = 0;
  ProArgs p{};
  p.kind = PRO_RMSNORM;
  p.x = x;
  p.ldx = ldx;
  p.xdt = x_dtype;
  p.w = w;
  p.wdt = w_dtype;
  p.one_plus = one_plus ? 1 : 0;
  p.eps = eps;
  p.q = q;
  p.s = s;
  return produce("qlin_rmsnorm_quant", p, M, K, stream);
}

int qlin_gate_mul_quant(const void* a, int64_t lda, const void* g, int64_t ldg, int dtype, int M, int N, int hd,
                        int8_t* q, float* s, void* stream) {
  g_err[0] = 0;
  ProArgs p{};
  p.kind = PRO_GATE_MUL;
  p.x = a;
  p.ldx = lda;
  p.xdt = dtype;
  p.g = g;
  p.ldg = ldg;
  p.hd = hd;
  p.q = q;
  p.s = s;
  return produce("qlin_gate_mul_quant", p, M, N, stream);
}

int qlin_norm_gated_quant(const void* v, const void* z, int64_t ldz, int dtype, const void* w, int w_dtype, int T,
                          int N, int hd, float eps, int8_t* q, float* s, void* stream) {
  g_err[0] = 0;
  ProArgs p{};
  p.kind = PRO_NORM_GATED;
  p.x = v;
  p.ldx = N;
  p.xdt = dtype;
  p.g = z;
  p.ldg = ldz;
  p.w = w;
  p.wdt = w_dtype;
  p.hd = hd;
  p.eps = eps;
  p.q = q;
  p.s = s;
  return produce("qlin_norm_gated_quant", p, T, N, stream);
}

int qlin_pro_exp_f32(const float* x, float* y, int n, void* stream) {
  g_err[0] = 0;
  if (n < 0) return fail(QLIN_ERR_INVALID, "qlin_pro_exp_f32: n=%d", n);
  if (n > 0 && (!x || !y)) return fail(QLIN_ERR_INVALID, "qlin_pro_exp_f32: null pointer");
  return hip_status("qlin_pro_exp_f32", launch_pro_exp(x, y, n, (hipStream_t)stream));
}

#define QL_PRO_ARG(fn)                                                      \
  if (!pro) return fail(QLIN_ERR_INVALID, "%s: null producer", fn);        \
  const ProArgs pa = pro_from(pro);

int qlin_pro_gemm_i8(const qlin_producer* pro, int M, int K, const int8_t* b, const void* b_s, int bs_dtype, int N,
                     void* out, int64_t ldo, const void* residual, int64_t ldr, void* workspace,
                     size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  QL_PRO_ARG("qlin_pro_gemm_i8")
  return engine_gemm("qlin_pro_gemm_i8", WK_W8, nullptr, nullptr, M, K, b, b_s, bs_dtype, nullptr, 64, N, out, ldo,
                     residual, ldr, workspace, workspace_bytes, stream, false, &pa);
}

int qlin_pro_gemm_w4(const qlin_producer* pro, int M, int K, const uint8_t* b, const void* b_s, int bs_dtype,
                     const uint8_t* b_z, int group, int N, void* out, int64_t ldo, const void* residual, int64_t ldr,
                     void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  QL_PRO_ARG("qlin_pro_gemm_w4")
  return engine_gemm("qlin_pro_gemm_w4", WK_W4, nullptr, nullptr, M, K, b, b_s, bs_dtype, b_z, group, N, out, ldo,
                     residual, ldr, workspace, workspace_bytes, stream, false, &pa);
}

int qlin_pro_proj3_i8(const qlin_producer* pro, int M, int K, const int8_t* w1, const void* s1, int n1,
                      const int8_t* w2, const void* s2, int n2, const int8_t* w3, const void* s3, int n3, int bs_dtype,
                      void* out, int64_t ldo, void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  QL_PRO_ARG("qlin_pro_proj3_i8")
  return engine_proj3("qlin_pro_proj3_i8", WK_W8, nullptr, nullptr, M, K, w1, s1, nullptr, n1, w2, s2, nullptr, n2,
                      w3, s3, nullptr, n3, bs_dtype, 64, out, ldo, workspace, workspace_bytes, stream, &pa);
}

int qlin_pro_proj3_w4(const qlin_producer* pro, int M, int K, const uint8_t* w1, const void* s1, const uint8_t* z1,
                      int n1, const uint8_t* w2, const void* s2, const uint8_t* z2, int n2, const uint8_t* w3,
                      const void* s3, const uint8_t* z3, int n3, int bs_dtype, int group, void* out, int64_t ldo,
                      void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  QL_PRO_ARG("qlin_pro_proj3_w4")
  return engine_proj3("qlin_pro_proj3_w4", WK_W4, nullptr, nullptr, M, K, w1, s1, z1, n1, w2, s2, z2, n2, w3, s3, z3,
                      n3, bs_dtype, group, out, ldo, workspace, workspace_bytes, stream, &pa);
}

int qlin_pro_mlp_gate_up_quant_i8(const qlin_producer* pro, int M, int K, const int8_t* wg, const void* sg,
                                  const int8_t* wu, const void* su, int bs_dtype, int N, int8_t* out_q, float* out_s,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  QL_PRO_ARG("qlin_pro_mlp_gate_up_quant_i8")
  return engine_gate_up("qlin_pro_mlp_gate_up_quant_i8", WK_W8, EPI_GATEUP_Q, nullptr, nullptr, M, K, wg, sg, nullptr,
                        wu, su, nullptr, bs_dtype, 64, N, nullptr, out_q, out_s, workspace, workspace_bytes, stream,
                        &pa);
}

int qlin_pro_mlp_gate_up_quant_w4(const qlin_producer* pro, int M, int K, const uint8_t* wg, const void* sg,
                                  const uint8_t* zg, const uint8_t* wu, const void* su, const uint8_t* zu,
                                  int bs_dtype, int group, int N, int8_t* out_q, float* out_s, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  QL_PRO_ARG("qlin_pro_mlp_gate_up_quant_w4")
  return engine_gate_up("qlin_pro_mlp_gate_up_quant_w4", WK_W4, EPI_GATEUP_Q, nullptr, nullptr, M, K, wg, sg, zg, wu,
                        su, zu, bs_dtype, group, N, nullptr, out_q, out_s, workspace, workspace_bytes, stream, &pa);
}

int qlin_w4_unpack(const uint8_t* packed, int K, int N, uint8_t* nib, void* stream) {
  g_err[0] = 0;
  if (K < 0 || N < 0 || K % 2) return fail(QLIN_ERR_INVALID, "qlin_w4_unpack: bad sizes K=%d N=%d", K, N);
  if ((long long)K * N == 0) return QLIN_OK;
  if (!packed || !nib) return fail(QLIN_ERR_INVALID, "qlin_w4_unpack: null pointer");
  return hip_status("qlin_w4_unpack", launch_w4_unpack(packed, K, N, nib, (hipStream_t)stream));
}

int qlin_w4_dequant_f32(const uint8_t* packed, const void* scale, int s_dtype, const uint8_t* zero, int group, int K,
                        int N, float* out, void* stream) {
  g_err[0] = 0;
  if (K < 0 || N < 0 || K % 2) return fail(QLIN_ERR_INVALID, "qlin_w4_dequant_f32: bad sizes K=%d N=%d", K, N);
  if (group <= 0 || K % group) return fail(QLIN_ERR_INVALID, "qlin_w4_dequant_f32: bad group %d", group);
  if (!dtype_scale_ok(s_dtype)) return fail(QLIN_ERR_UNSUPPORTED, "qlin_w4_dequant_f32: scale dtype %d", s_dtype);
  if ((long long)K * N == 0) return QLIN_OK;
  if (!packed || !scale || !out) return fail(QLIN_ERR_INVALID, "qlin_w4_dequant_f32: null pointer");
  return hip_status("qlin_w4_dequant_f32",
                    launch_w4_dequant(packed, scale, s_dtype, zero, group, K, N, out, (hipStream_t)stream));
}

int qlin_w8_dequant_f32(const int8_t* w, const void* scale, int s_dtype, int K, int N, float* out, void* stream) {
  g_err[0] = 0;
  if (K < 0 || N < 0) return fail(QLIN_ERR_INVALID, "qlin_w8_dequant_f32: bad sizes K=%d N=%d", K, N);
  if (!dtype_scale_ok(s_dtype)) return fail(QLIN_ERR_UNSUPPORTED, "qlin_w8_dequant_f32: scale dtype %d", s_dtype);
  if ((long long)K * N == 0) return QLIN_OK;
  if (!w || !scale || !out) return fail(QLIN_ERR_INVALID, "qlin_w8_dequant_f32: null pointer");
  return hip_status("qlin_w8_dequant_f32", launch_w8_dequant(w, scale, s_dtype, K, N, out, (hipStream_t)stream));
}

int qlin_requant_w4_sym(const float* w, int K, int N, int group, uint8_t* packed, uint16_t* scale_bf16,
                        void* stream) {
  g_err[0] = 0;
  if (K < 0 || N < 0) return fail(QLIN_ERR_INVALID, "qlin_requant_w4_sym: bad sizes K=%d N=%d", K, N);
  if ((group != 32 && group != 64) || K % group != 0)
    return fail(QLIN_ERR_INVALID, "qlin_requant_w4_sym: group %d must be 32 or 64 and divide K=%d", group, K);
  if (K / group > 65535) return fail(QLIN_ERR_UNSUPPORTED, "qlin_requant_w4_sym: K=%d too large", K);
  if ((long long)K * N == 0) return QLIN_OK;
  if (!w || !packed || !scale_bf16) return fail(QLIN_ERR_INVALID, "qlin_requant_w4_sym: null pointer");
  return hip_status("qlin_requant_w4_sym",
                    launch_requant_w4(w, K, N, group, packed, scale_bf16, (hipStream_t)stream));
}

int qlin_requant_w8_row(const float* w, int K, int N, int8_t* q, float* scale, void* stream) {
  g_err[0] = 0;
  if (K < 0 || N < 0) return fail(QLIN_ERR_INVALID, "qlin_requant_w8_row: bad sizes K=%d N=%d", K, N);
  if ((K + 63) / 64 > 65535) return fail(QLIN_ERR_UNSUPPORTED, "qlin_requant_w8_row: K=%d too large", K);
  if ((long long)K * N == 0) return QLIN_OK;
  if (!w || !q || !scale) return fail(QLIN_ERR_INVALID, "qlin_requant_w8_row: null pointer");
  return hip_status("qlin_requant_w8_row", launch_requant_w8(w, K, N, q, scale, (hipStream_t)stream));
}

int qlin_w4_repack_gptq(const int32_t* qweight, int K, int N, uint8_t* packed, void* stream) {
  g_err[0] = 0;
  if (K < 0 || N < 0 || K % 8 != 0)
    return fail(QLIN_ERR_INVALID, "qlin_w4_repack_gptq: K=%d must be a multiple of 8, N=%d", K, N);
  if ((long long)K * N == 0) return QLIN_OK;
  if (!qweight || !packed) return fail(QLIN_ERR_INVALID, "qlin_w4_repack_gptq: null pointer");
  return hip_status("qlin_w4_repack_gptq", launch_repack_gptq(qweight, K, N, packed, (hipStream_t)stream));
}

int qlin_w4_repack_awq(const int32_t* qweight, int K, int N, uint8_t* packed, void* stream) {
  g_err[0] = 0;
  if (K < 0 || N < 0 || K % 2 != 0 || N % 8 != 0)
    return fail(QLIN_ERR_INVALID, "qlin_w4_repack_awq: K=%d must be even and N=%d a multiple of 8", K, N);
  if ((long long)K * N == 0) return QLIN_OK;
  if (!qweight || !packed) return fail(QLIN_ERR_INVALID, "qlin_w4_repack_awq: null pointer");
  if (!aligned(packed, 8)) return fail(QLIN_ERR_UNSUPPORTED, "qlin_w4_repack_awq: packed must be 8-byte aligned");
  return hip_status("qlin_w4_repack_awq", launch_repack_awq(qweight, K, N, packed, (hipStream_t)stream));
}

int qlin_w4_repack_ct(const int32_t* weight_packed, int N, int W, int K, uint8_t* packed, void* stream) {
  g_err[0] = 0;
  if (N < 0 || W < 0 || K < 0 || K % 2 != 0 || (long long)K > 8LL * W)
    return fail(QLIN_ERR_INVALID, "qlin_w4_repack_ct: need even K <= 8 W (N=%d W=%d K=%d)", N, W, K);
  if (N % 16 != 0) return fail(QLIN_ERR_UNSUPPORTED, "qlin_w4_repack_ct: N=%d is not a multiple of 16", N);
  if ((long long)N * K == 0) return QLIN_OK;
  if (!weight_packed || !packed) return fail(QLIN_ERR_INVALID, "qlin_w4_repack_ct: null pointer");
  if (!aligned(weight_packed, 4) || !aligned(packed, 16))
    return fail(QLIN_ERR_UNSUPPORTED, "qlin_w4_repack_ct: weight_packed 4-byte and packed 16-byte aligned");
  if ((K / 2 + 63) / 64 > 65535) return fail(QLIN_ERR_UNSUPPORTED, "qlin_w4_repack_ct: K=%d too large", K);
  return hip_status("qlin_w4_repack_ct", launch_repack_ct(weight_packed, N, W, K, packed, (hipStream_t)stream));
}

int qlin_w4_zeros_unpack(const int32_t* qzeros, int G, int N, int awq_order, int add, uint8_t* zeros,
                         void* stream) {
  g_err[0] = 0;
  if (G < 0 || N < 0 || N % 8 != 0)
    return fail(QLIN_ERR_INVALID, "qlin_w4_zeros_unpack: N=%d must be a multiple of 8 (G=%d)", N, G);
  if (add < 0 || add > 240) return fail(QLIN_ERR_INVALID, "qlin_w4_zeros_unpack: add=%d out of range", add);
  if ((long long)G * N == 0) return QLIN_OK;
  if (!qzeros || !zeros) return fail(QLIN_ERR_INVALID, "qlin_w4_zeros_unpack: null pointer");
  return hip_status("qlin_w4_zeros_unpack",
                    launch_zeros_unpack(qzeros, G, N, awq_order ? 1 : 0, add, zeros, (hipStream_t)stream));
}

}  // extern "C"
