// Host/device shared definitions of libqlin (not part of the public ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qlin {

// One weight matrix covering a contiguous range of output columns.
struct Seg {
  const uint8_t* w;  // int8 [K][n] or packed uint8 [K/2][n]
  const void* s;     // W8: scale[n]; W4: scale[K/group][n]
  const uint8_t* z;  // W4 zeros [K/group][n] or nullptr
  int n;             // columns of this matrix
  int col0;          // first output column it writes
  int tile0;         // first column tile that belongs to it
};

// Activation producer (kernels/norm.py) of an engine-signature call: the int8 codes
// and per-64 scales are made from 16-bit activations, by a launch of their own or in
// the prologue of the linear's launch (producers.h).
enum ProKind { PRO_NONE = 0, PRO_RMSNORM = 1, PRO_GATE_MUL = 2, PRO_NORM_GATED = 3 };

struct ProArgs {
  int kind;            // ProKind
  const void* x;       // rmsnorm: rows [M][ldx]; gate_mul: a [M][ldx]; norm_gated: v [M][K]
  long long ldx;
  int xdt;             // DT_BF16 or DT_F16 (x and g)
  const void* g;       // gate_mul: gate rows [M][ldg] (head h: 2 hd values, gates in the
                       // second half); norm_gated: z [M][ldg]
  long long ldg;
  const void* w;       // norm weight: rmsnorm [K], norm_gated [hd]
  int wdt;             // DT_BF16, DT_F16 or DT_F32
  int hd;              // head size (gate_mul, norm_gated)
  int one_plus;        // rmsnorm: scale by w + 1
  float eps;
  int8_t* q;           // codes [M][K] (written by the standalone producer; optional copy
  float* s;            // in a fused launch) and scales [M][K/64]
  int8_t* tq;          // where a call that cannot fuse the producer puts the codes and
  float* ts;           // scales first: q / s, or the end of the workspace
  int lds_off;         // fused launch: byte offset of the code block in dynamic LDS
  int ldq;             // fused launch: row stride of the LDS code block (bytes)
};

// Dynamic LDS a fused-prologue launch may add for its code block (plans that need
// more make their activations with a launch of their own).
constexpr size_t kProLdsBytes = 64 * 1024;

// Arguments of the skinny (row-tile of <= 16 rows) MFMA kernel.
struct SkArgs {
  const void* x;       // ACT_F16: fp16 [M][ldx]; ACT_I8: int8 [M][K]
  const float* xs;     // ACT_I8: fp32 [M][K/64]
  long long ldx;
  int M, K;
  Seg seg[3];          // EPI_STORE: up to 3 column segments; gate/up: seg[0]=gate, seg[1]=up
  int nseg;
  int ntiles;          // column tiles
  int ncols;           // total output columns
  int group;           // W4 weight group
  int sdt;             // scale element type (DT_*)
  void* out;           // EPI_STORE / EPI_GATEUP output (16-bit elements)
  long long ldo;
  int odt;             // output element type (DT_F16 / DT_BF16)
  const void* res;     // residual (odt) or nullptr
  long long ldr;
  int8_t* oq;          // EPI_GATEUP_Q int8 [M][ncols]
  float* os;           // EPI_GATEUP_Q fp32 [M][ncols/64]
  float* part;         // split-K partials [splits][nsets][M][ncols]
  unsigned* cnt;       // split-K arrival counters [row tiles][ntiles], zero between calls
  int kchunk;          // K range of one wave (lanes == 0) or of one split (lanes == 2)
  int splits;          // workgroups per column tile along K
  int lanes;           // int8 activations: 0 = wave w of split s folds the contiguous range
                       // [(s*waves + w)*kchunk, +kchunk); 2 = the two waves of split s fold
                       // the alternate 64-wide blocks of [s*kchunk, (s+1)*kchunk) (wave w:
                       // block offsets w, w+2, ...), the K order of the tiled int8 kernel
  ProArgs pro;         // fused prologue (launches with SkLaunch::pro set); x / xs unused
  int gm;              // tiled int8 kernel: row tiles per group of the tile order; > 0 also
                       // gives each XCD a contiguous run of the order (0: groups of 8,
                       // workgroups in order)
};

struct SkLaunch {
  int act, wk, hz, epi, cols;
  int ks;          // K-loop fold structure (KStruct in skinny_kernel.h), set by launch_skinny
  int waves;       // waves per workgroup
  int pro;         // 1: the launch makes its activations in a prologue (SkArgs::pro)
  dim3 grid;
  size_t lds;      // dynamic LDS bytes
};

hipError_t launch_skinny(const SkLaunch& L, const SkArgs& a, hipStream_t stream);
// the instantiations of each activation / weight family (skinny_f16.hip, skinny_i8w8.hip,
// skinny_i8w4.hip)
hipError_t launch_skinny_f16(const SkLaunch& L, const SkArgs& a, hipStream_t stream);
hipError_t launch_skinny_i8w8(const SkLaunch& L, const SkArgs& a, hipStream_t stream);
hipError_t launch_skinny_i8w4(const SkLaunch& L, const SkArgs& a, hipStream_t stream);
// Tiled int8-activation kernel for the engine-signature calls with more than 16 rows
// (prefill_i8.hip), store and gate/up epilogues: whether it covers the call (K % 64
// == 0, W4 groups of at least 64, every column range a multiple of 128), and its launch.
bool prefill_i8_ok(const SkArgs& a, int wk, int epi);
hipError_t launch_prefill_i8(SkArgs a, int wk, bool hz, int epi, hipStream_t stream);

// Engine-signature call outside the fast kernels' layout rules (edge.hip): any N,
// pointers aligned to their element size only.  Segments, epilogue and element types
// as SkArgs.
struct EdgeArgs {
  const int8_t* x;     // int8 codes [M][K]
  const float* xs;     // fp32 scales [M][K/64]
  int M, K;
  Seg seg[3];          // EPI_STORE: column segments; gate/up: seg[0] = gate, seg[1] = up
  int nseg;
  int ncols;
  int group;           // W4 weight group
  int sdt;             // weight-scale element type (DT_*)
  int epi;             // EpiKind
  int odt;             // 16-bit output (and residual) element type
  void* out;
  long long ldo;
  const void* res;
  long long ldr;
  int8_t* oq;          // EPI_GATEUP_Q codes [M][ncols]
  float* os;           // EPI_GATEUP_Q scales [M][ncols/64]
};
hipError_t launch_edge(const EdgeArgs& a, int wk, hipStream_t st);
// whether a skinny variant runs with up to 8 waves per workgroup (else 4)
bool skinny_big(int act, int wk, int epi, int cols);

// Arguments of the LDS-tiled (prefill) fp16-activation MFMA kernel.
struct TlArgs {
  const _Float16* x;  // fp16 [M][ldx]
  long long ldx;
  const uint8_t* w;   // int8 [K][N] or packed uint8 [K/2][N]
  const void* s;      // W8: scale[N]; W4: scale[K/group][N]
  const uint8_t* z;   // W4 zeros or nullptr
  int M, N, K;
  int group;
  int sdt;
  void* out;          // 16-bit [M][ldo]
  long long ldo;
  int odt;
  const void* res;    // 16-bit [M][ldr] or nullptr
  long long ldr;
  int splits;         // workgroups per output tile along K
  float* part;        // split-K partials [tiles][splits][waves][128 * 64], or nullptr
  unsigned* cnt;      // split-K arrival counters [tiles], zero between calls
  int sk;             // balanced schedule: K tiles per workgroup over all tiles (0 = off);
                      // partials [tiles][2][waves][128 * 64]
  int gm;             // one tile per workgroup: row tiles per group of the tile order; > 0
                      // also gives each XCD a contiguous run of the order (0: groups of 8,
                      // workgroups in order)
};

// LDS-DMA prefill kernel; `shape` picks the workgroup tile (rows x columns):
// PF_128x128 (2 waves), PF_256x256 (8 waves, two per SIMD) and PF_128x128_K2 (two
// wave groups split every K tile's substeps: 4 waves).
enum PrefillShape { PF_128x128 = 0, PF_256x256 = 1, PF_128x128_K2 = 2, PF_SHAPES = 3 };
hipError_t launch_prefill(const TlArgs& a, int wk, bool hz, int shape, hipStream_t stream);
// whether the balanced schedule with sk K tiles per workgroup gives every output tile
// at most two workgroups
bool prefill_balanced_ok(long long tiles, int nkt, int sk);
// rows, columns and waves of a prefill workgroup tile
void prefill_geometry(int shape, int* bm, int* bn, int* waves);
bool prefill_shape_ok(int shape);

// Sets the message qlin_last_error() returns on this thread; returns `code`.
int set_error(int code, const char* msg);
// qlin_gemm_i8 on a caller-owned scratch laid out like the workspace (counter_bytes()
// of arrival counters, poll_bytes() of polling-exchange slots that start zero, then
// partial sums): validates, clears the arrival counters the call can use with a fill
// kernel on `stream`, then plans and launches.
int gemm_i8_scratch(const char* fn, const int8_t* a_q, const float* a_s, int M, int K, const int8_t* b,
                    const void* b_s, int bs_dtype, int N, void* out, int64_t ldo, const void* residual,
                    int64_t ldr, void* scratch, size_t scratch_bytes, void* stream);
size_t counter_bytes();
size_t poll_bytes();

// Validates an activation producer for M rows of K columns (norm_gated's input row
// stride becomes K); returns a status with the message set.
int check_producer(const char* fn, ProArgs& p, int M, int K);
// Zeroes the first n arrival counters of a scratch with a fill kernel on `stream`.
hipError_t clear_counters(void* ws, long long n, hipStream_t stream);
// Engine decode work units (echain.hip): whether an engine-signature call of M rows
// runs on them (M <= 8, W8 or W4 groups that are multiples of 64, 16-byte aligned
// activations), and the call as a one-level launch of them.  The workspace holds
// `counter_bytes` of arrival counters, `poll_bytes` of polling-exchange slots (zero
// between calls), then split-K partials.
constexpr int kDecodeRowsMax = 8;
bool echain_covers(const SkArgs& a, int wk, int M);
int echain_engine_call(const char* fn, const SkArgs& a, int wk, int epi, int M, void* ws, size_t ws_bytes,
                       size_t counter_bytes, size_t poll_bytes, hipStream_t stream, bool clear);

// Standalone producer launch: codes and scales of all M rows into p.q / p.s.
hipError_t launch_producer(const ProArgs& p, int M, int K, hipStream_t st);
// Evaluates the producers' exp on n values (a test entry point).
hipError_t launch_pro_exp(const float* x, float* y, int n, hipStream_t st);
// whether a skinny launch plan (act, wk, hz, epi, cols, waves) has a fused-prologue
// instantiation (skinny_pro_w8.hip, skinny_pro_w4.hip) for weight group `group`
bool skinny_pro_ok(const SkLaunch& L, int group);

hipError_t launch_w4_unpack(const uint8_t* p, int K, int N, uint8_t* out, hipStream_t st);
hipError_t launch_w4_dequant(const uint8_t* p, const void* s, int sdt, const uint8_t* z,
                             int group, int K, int N, float* out, hipStream_t st);
hipError_t launch_w8_dequant(const int8_t* w, const void* s, int sdt, int K, int N, float* out,
                             hipStream_t st);
hipError_t launch_requant_w4(const float* w, int K, int N, int group, uint8_t* packed, uint16_t* sbf,
                             hipStream_t st);
hipError_t launch_requant_w8(const float* w, int K, int N, int8_t* q, float* scale, hipStream_t st);
hipError_t launch_repack_gptq(const int32_t* qw, int K, int N, uint8_t* packed, hipStream_t st);
hipError_t launch_repack_awq(const int32_t* qw, int K, int N, uint8_t* packed, hipStream_t st);
hipError_t launch_repack_ct(const int32_t* qw, int N, int W, int K, uint8_t* packed, hipStream_t st);
hipError_t launch_zeros_unpack(const int32_t* qz, int G, int N, int awq, int add, uint8_t* z, hipStream_t st);

}  // namespace qlin
