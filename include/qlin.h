/*
 * qlin.h -- C ABI of the MI355X (gfx950) quantized-linear library, libqlin.so.
 *
 * The library replaces the quantized GEMM/GEMV path of the Qwen3.5 prompt-enhancer
 * engine: the INT8 kernels of kernels/gemm.py and the W4 group-dequant kernels of
 * kernels/w4.py (reference paths).  Every entry point:
 *
 *   - takes plain device pointers, sizes and element strides (no framework types);
 *   - validates its arguments before launching anything and returns a status code
 *     (QLIN_OK == 0, negative on error; the message is in qlin_last_error());
 *   - launches asynchronously on `stream` (a hipStream_t, NULL = default stream),
 *     never synchronizes and never allocates memory;
 *   - writes only into caller-allocated outputs.  Split-K partial sums go through the
 *     caller-supplied `workspace` (at least qlin_workspace_bytes() bytes, zero-filled
 *     once before first use; the library leaves its counters and exchange slots at
 *     zero after every call).  Calls that share a workspace must not overlap in time.
 *
 * Layouts are the engine's (weights.py:297-309, quant_formats.py:6-9):
 *   W8  : int8  b[K][N] (N contiguous), scale[N]
 *   W4  : uint8 b[K/2][N]; byte (j, n) holds k = 2j in bits 0-3 and k = 2j+1 in
 *         bits 4-7; scale[K/G][N]; optional uint8 zero[K/G][N] (one real zero per
 *         group, not packed); the weight value is (nibble - z), z = 8 when absent.
 *   engine activations: int8 a_q[M][K] (row stride K) with fp32 a_s[M][K/64].
 * All matrices are row-major; `ld*` arguments are row strides in elements.
 *
 * Engine-signature entry points take any N and pointers aligned to their element
 * size only, as the reference's masked kernels do (kernels/gemm.py:50-57).  Their fast
 * kernels need N % 16 == 0 (per projection), 16-byte aligned weights, scales, zeros,
 * outputs and residuals, 16-bit row strides that are multiples of 8, and 8-byte
 * aligned a_q; a call outside those rules runs on a generic kernel (same arithmetic
 * per block, one K split; correct, not fast).  The A16 entry points (qlin_linear_*)
 * and the chains keep the fast rules and refuse other layouts.
 */
#ifndef QLIN_H
#define QLIN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QLIN_ABI_VERSION 1

/* status codes */
#define QLIN_OK 0
#define QLIN_ERR_INVALID (-1)     /* null pointer, negative or inconsistent size   */
#define QLIN_ERR_UNSUPPORTED (-2) /* valid, but shape/group/alignment/dtype unsupported */
#define QLIN_ERR_HIP (-3)         /* HIP runtime error while launching              */
#define QLIN_ERR_WORKSPACE (-4)   /* workspace missing or too small                 */

/* element type codes (scales, activations, outputs) */
#define QLIN_F16 1
#define QLIN_BF16 2
#define QLIN_F32 3

/* ABI version (QLIN_ABI_VERSION). */
int qlin_version(void);

/* Message describing the last error returned on the calling thread ("" if none). */
const char* qlin_last_error(void);

/* Workspace size (bytes) every entry point below accepts. */
size_t qlin_workspace_bytes(void);

/* ---------------------------------------------------------------------------
 * Engine-signature entry points (int8 activations + per-64 fp32 scales, bf16 out)
 * ------------------------------------------------------------------------- */

/* out[M,N] = bf16( sum_kb a_s[m,kb] * (a_q . b)[m,n,kb] * b_s[n] (+ residual) ).
 * Replaces gemm_i8 (kernels/gemm.py:60-92, kernel gemm.py:20-57).
 * b int8 [K,N]; b_s [N] of type bs_dtype; out/residual bf16 with row strides
 * ldo/ldr; residual may alias out (each element is read once before it is
 * written); residual NULL = none. */
int qlin_gemm_i8(const int8_t* a_q, const float* a_s, int M, int K,
                 const int8_t* b, const void* b_s, int bs_dtype, int N,
                 void* out, int64_t ldo, const void* residual, int64_t ldr,
                 void* workspace, size_t workspace_bytes, void* stream);

/* qlin_gemm_i8 without a workspace argument: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  Split-K partials and arrival
 * counters go to a static device array of 13 MiB per GPU (1 MiB of counters, 4 MiB of
 * slots that decode calls' split tiles exchange through and leave zero, 8 MiB of
 * partials), held until the process ends; nothing is allocated or freed per call.
 * Each call first zeroes the arrival counters it can use with a fill kernel on
 * `stream`.  Results equal qlin_gemm_i8's bit for bit: decode plans fit the scratch,
 * and a prefill call whose partials exceed it runs in blocks of rows (rows are
 * independent).  A call that cannot fit even one block of rows fails with
 * QLIN_ERR_WORKSPACE before launching anything.  Calls that overlap in time on one
 * GPU share the array and race: serialize them (one stream, or the engine's lock).
 * The replay of a HIP graph that holds a call is a call: it must not overlap another
 * call or replay on the same GPU either (streams do not separate them). */
int qlin_gemm_i8_noalloc(const int8_t* a_q, const float* a_s, int M, int K,
                         const int8_t* b, const void* b_s, int bs_dtype, int N,
                         void* out, int64_t ldo, const void* residual, int64_t ldr,
                         void* stream);

/* W4 twin of qlin_gemm_i8: replaces gemm_w4 (kernels/w4.py:139-166, kernel
 * w4.py:107-136).  b uint8 [K/2,N]; b_s [K/group, N]; b_z uint8 [K/group, N] or NULL
 * (z = 8).  group: 32, 64 or a multiple of 64 (quant_formats.py:42-49). */
int qlin_gemm_w4(const int8_t* a_q, const float* a_s, int M, int K,
                 const uint8_t* b, const void* b_s, int bs_dtype, const uint8_t* b_z,
                 int group, int N,
                 void* out, int64_t ldo, const void* residual, int64_t ldr,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Three W8 projections sharing (a_q, a_s); out[:, 0:n1], [n1:n1+n2], [n1+n2:n1+n2+n3]
 * with row stride ldo (bf16).  A NULL weight must come with n == 0.
 * Replaces proj3 (kernels/gemm.py:290-312, kernel gemm.py:234-287). */
int qlin_proj3_i8(const int8_t* a_q, const float* a_s, int M, int K,
                  const int8_t* w1, const void* s1, int n1,
                  const int8_t* w2, const void* s2, int n2,
                  const int8_t* w3, const void* s3, int n3, int bs_dtype,
                  void* out, int64_t ldo,
                  void* workspace, size_t workspace_bytes, void* stream);

/* W4 twin of qlin_proj3_i8 with per-projection zeros (NULL = 8).
 * Replaces proj3_w4 (kernels/w4.py:220-251, kernel w4.py:169-217). */
int qlin_proj3_w4(const int8_t* a_q, const float* a_s, int M, int K,
                  const uint8_t* w1, const void* s1, const uint8_t* z1, int n1,
                  const uint8_t* w2, const void* s2, const uint8_t* z2, int n2,
                  const uint8_t* w3, const void* s3, const uint8_t* z3, int n3,
                  int bs_dtype, int group,
                  void* out, int64_t ldo,
                  void* workspace, size_t workspace_bytes, void* stream);

/* out[M,N] (bf16, row stride N) = silu(gate) * up, gate/up W8.
 * Replaces mlp_gate_up (kernels/gemm.py:140-151, kernel gemm.py:95-137). */
int qlin_mlp_gate_up_i8(const int8_t* a_q, const float* a_s, int M, int K,
                        const int8_t* wg, const void* sg, const int8_t* wu, const void* su,
                        int bs_dtype, int N, void* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* W4 form of qlin_mlp_gate_up_i8.  No reference counterpart (the reference's
 * mlp_gate_up is W8 only); exported so the fused W4 quant epilogue can be checked
 * against the unfused composition, as .dev/test_fused.py does for W8. */
int qlin_mlp_gate_up_w4(const int8_t* a_q, const float* a_s, int M, int K,
                        const uint8_t* wg, const void* sg, const uint8_t* zg,
                        const uint8_t* wu, const void* su, const uint8_t* zu,
                        int bs_dtype, int group, int N, void* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* h = bf16(silu(gate) * up); per 64 columns sc = max(amax/127, 1e-8),
 * out_q = round_half_away(h / sc) clamped to +-127 (int8 [M,N], row stride N),
 * out_s = sc (fp32 [M, N/64]).  N % 64 == 0.
 * Replaces mlp_gate_up_quant (kernels/gemm.py:214-231, kernel gemm.py:154-211). */
int qlin_mlp_gate_up_quant_i8(const int8_t* a_q, const float* a_s, int M, int K,
                              const int8_t* wg, const void* sg,
                              const int8_t* wu, const void* su, int bs_dtype, int N,
                              int8_t* out_q, float* out_s,
                              void* workspace, size_t workspace_bytes, void* stream);

/* W4 twin.  Replaces mlp_gate_up_quant_w4 (kernels/w4.py:300-323, kernel
 * w4.py:254-297). */
int qlin_mlp_gate_up_quant_w4(const int8_t* a_q, const float* a_s, int M, int K,
                              const uint8_t* wg, const void* sg, const uint8_t* zg,
                              const uint8_t* wu, const void* su, const uint8_t* zu,
                              int bs_dtype, int group, int N,
                              int8_t* out_q, float* out_s,
                              void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Activation producers: the int8 codes + per-64 fp32 scales the engine-signature
 * entry points consume, made from 16-bit activations.  Per 64 columns
 * s = max(amax/127, 1e-8), q = round_half_away(y / s) clamped to +-127
 * (kernels/norm.py:15-25).  The arithmetic is fixed operation by operation (fp32,
 * no fused multiply-add; sums of squares in a fixed lane order; rsqrt as 1/sqrt;
 * exp by Cody-Waite reduction and a degree-7 Taylor polynomial), so the codes do
 * not depend on M or on which launch made them.
 * ------------------------------------------------------------------------- */

#define QLIN_PRO_RMSNORM 1
#define QLIN_PRO_GATE_MUL 2
#define QLIN_PRO_NORM_GATED 3

/* y = x * rsqrt(mean(x^2) + eps) * (w + 1 if one_plus else w), quantized.
 * x [M,K] bf16/fp16 (x_dtype), row stride ldx; w [K] (w_dtype bf16/fp16/fp32);
 * q int8 [M,K] (row stride K), s fp32 [M,K/64].  K % 64 == 0.
 * Replaces rmsnorm_quant (kernels/norm.py:48-57, kernel norm.py:28-41). */
int qlin_rmsnorm_quant(const void* x, int64_t ldx, int x_dtype, const void* w, int w_dtype,
                       int M, int K, float eps, int one_plus, int8_t* q, float* s, void* stream);

/* y = a * sigmoid(g[gate column]), quantized; a [M,N] (row stride lda), g [M,*] (row
 * stride ldg >= 2N) laid out as heads of 2*hd values with the gates in the second
 * half; both `dtype` (bf16/fp16).  hd % 8 == 0, N % hd == 0, N % 64 == 0.
 * Replaces gate_mul_quant (kernels/norm.py:182-188, kernel norm.py:168-179). */
int qlin_gate_mul_quant(const void* a, int64_t lda, const void* g, int64_t ldg, int dtype,
                        int M, int N, int hd, int8_t* q, float* s, void* stream);

/* Per (row, head of hd): y = bf16(v * rsqrt(mean_head(v^2) + eps) * w * silu(z)),
 * quantized.  v [T,N] contiguous, z [T,*] (row stride ldz), both `dtype`; w [hd]
 * (w_dtype).  hd in {128, 256, 512}.
 * Replaces norm_gated_quant (kernels/norm.py:127-137, kernel norm.py:95-124). */
int qlin_norm_gated_quant(const void* v, const void* z, int64_t ldz, int dtype,
                          const void* w, int w_dtype, int T, int N, int hd, float eps,
                          int8_t* q, float* s, void* stream);

/* The producers' exp on n fp32 values (test entry point: no reference counterpart;
 * the reference uses Triton's exp). */
int qlin_pro_exp_f32(const float* x, float* y, int n, void* stream);

/* One producer, as the qlin_pro_* linears below take it. */
typedef struct qlin_producer {
  int kind;         /* QLIN_PRO_RMSNORM, QLIN_PRO_GATE_MUL or QLIN_PRO_NORM_GATED */
  const void* x;    /* rmsnorm: x [M,K]; gate_mul: a [M,K]; norm_gated: v [M,K] contiguous */
  int64_t ldx;      /* row stride of x (ignored for norm_gated) */
  int x_dtype;      /* QLIN_BF16 or QLIN_F16, for x and g */
  const void* g;    /* gate_mul: gate rows; norm_gated: z; rmsnorm: NULL */
  int64_t ldg;
  const void* w;    /* norm weight (rmsnorm [K], norm_gated [hd]); gate_mul: NULL */
  int w_dtype;
  int hd;           /* head size (gate_mul, norm_gated) */
  int one_plus;     /* rmsnorm */
  float eps;
  int8_t* q;        /* optional: the codes [M,K] and scales [M,K/64] are written here */
  float* s;         /*   too (NULL: not kept; they then pass through the workspace) */
} qlin_producer;

/* The engine-signature linears with their activation producer in the same call: no
 * counterpart in the reference, whose engine launches the producer (kernels/norm.py)
 * and then the linear (kernels/gemm.py / w4.py) -- e.g. rmsnorm_quant + proj3 at
 * engine.py:220-226, gate_mul_quant + gemm_i8 at engine.py:265-268, norm_gated_quant +
 * gemm_i8 at engine.py:236-240, rmsnorm_quant + mlp_gate_up_quant at engine.py:272-276.
 * Results equal the two-call sequence bit for bit.  Decode-shaped launches make the
 * codes of their rows and K range in a prologue, with their first weight loads in
 * flight; wide launches (the vocab head) and prefill's tiled kernel run the producer
 * as a launch of its own first.  The producer's inputs must not overlap `out`.
 * Arguments after `K` are those of the entry point named in the suffix. */
int qlin_pro_gemm_i8(const qlin_producer* pro, int M, int K,
                     const int8_t* b, const void* b_s, int bs_dtype, int N,
                     void* out, int64_t ldo, const void* residual, int64_t ldr,
                     void* workspace, size_t workspace_bytes, void* stream);
int qlin_pro_gemm_w4(const qlin_producer* pro, int M, int K,
                     const uint8_t* b, const void* b_s, int bs_dtype, const uint8_t* b_z,
                     int group, int N,
                     void* out, int64_t ldo, const void* residual, int64_t ldr,
                     void* workspace, size_t workspace_bytes, void* stream);
int qlin_pro_proj3_i8(const qlin_producer* pro, int M, int K,
                      const int8_t* w1, const void* s1, int n1,
                      const int8_t* w2, const void* s2, int n2,
                      const int8_t* w3, const void* s3, int n3, int bs_dtype,
                      void* out, int64_t ldo,
                      void* workspace, size_t workspace_bytes, void* stream);
int qlin_pro_proj3_w4(const qlin_producer* pro, int M, int K,
                      const uint8_t* w1, const void* s1, const uint8_t* z1, int n1,
                      const uint8_t* w2, const void* s2, const uint8_t* z2, int n2,
                      const uint8_t* w3, const void* s3, const uint8_t* z3, int n3,
                      int bs_dtype, int group,
                      void* out, int64_t ldo,
                      void* workspace, size_t workspace_bytes, void* stream);
int qlin_pro_mlp_gate_up_quant_i8(const qlin_producer* pro, int M, int K,
                                  const int8_t* wg, const void* sg,
                                  const int8_t* wu, const void* su, int bs_dtype, int N,
                                  int8_t* out_q, float* out_s,
                                  void* workspace, size_t workspace_bytes, void* stream);
int qlin_pro_mlp_gate_up_quant_w4(const qlin_producer* pro, int M, int K,
                                  const uint8_t* wg, const void* sg, const uint8_t* zg,
                                  const uint8_t* wu, const void* su, const uint8_t* zu,
                                  int bs_dtype, int group, int N,
                                  int8_t* out_q, float* out_s,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * A16 weight-only core (fp16 activations; the form the engine's linears take when
 * activations stay in floating point).  The reference computes this on its CPU path
 * as "dequantize through quant_formats.py (quant_formats.py:6-9), then an fp32
 * matmul"; these entry points are its GPU counterpart.
 * ------------------------------------------------------------------------- */

/* out[M,N] = x[M,K] . (w[K,N] * scale[N]) (+ residual).
 * x: x_dtype (QLIN_F16), row stride ldx; out/residual: out_dtype (F16 or BF16). */
int qlin_linear_w8(const void* x, int x_dtype, int M, int K, int64_t ldx,
                   const int8_t* w, const void* scale, int s_dtype, int N,
                   void* out, int out_dtype, int64_t ldo,
                   const void* residual, int64_t ldr,
                   void* workspace, size_t workspace_bytes, void* stream);

/* out[M,N] = x . ((nibble - z) * scale[k/group, n]) (+ residual); zero NULL = 8. */
int qlin_linear_w4(const void* x, int x_dtype, int M, int K, int64_t ldx,
                   const uint8_t* w, const void* scale, int s_dtype,
                   const uint8_t* zero, int group, int N,
                   void* out, int out_dtype, int64_t ldo,
                   const void* residual, int64_t ldr,
                   void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Decode chains: many A16 GEMVs in one persistent launch
 *
 * A chain is a list of jobs, each an A16 linear as qlin_linear_w8 / qlin_linear_w4
 * computes it, for the same M (1-16 rows).  Jobs carry a dependency level: levels
 * start at 0 and rise by at most 1 along the list, and the jobs of level L > 0 read
 * their activations only after every job of level L-1 has written its output (so a
 * job may read another's output, or add to a residual another job wrote).  One
 * qlin_chain_run launch computes every job: the linears of a whole decode step with
 * no kernel boundary between them.  No reference counterpart as a function: the
 * reference launches one kernel per linear and names whole-step decode capture as its
 * next step (ENGINEERING.md:383-399); each job replaces one such launch.
 * ------------------------------------------------------------------------- */
typedef struct qlin_chain_job {
  const void* x;          /* fp16 activations [M][ldx] */
  int64_t ldx;
  const void* w;          /* W8: int8 [K][N]; W4: packed uint8 [K/2][N] */
  const void* scale;      /* W8: [N]; W4: [K/group][N] */
  int scale_dtype;        /* QLIN_F16, QLIN_BF16 or QLIN_F32 */
  const uint8_t* zero;    /* W4 zeros [K/group][N] or NULL (z = 8); NULL for W8 */
  int K, N;               /* W8: K % 32 == 0; W4: K % 128 == 0; N % 16 == 0 */
  int group;              /* 0 = W8; 128 = W4 group 128 (the only W4 group chains take) */
  void* out;              /* 16-bit [M][ldo] */
  int out_dtype;          /* QLIN_F16 or QLIN_BF16 */
  int64_t ldo;
  const void* residual;   /* out_dtype [M][ldr] or NULL; may alias out */
  int64_t ldr;
  int level;              /* dependency level */
} qlin_chain_job;

/* Bytes of device memory a chain plan needs (0 if the jobs are invalid; the reason
 * is in qlin_last_error()). */
size_t qlin_chain_bytes(const qlin_chain_job* jobs, int njobs, int M);

/* Validates the jobs and writes the plan (descriptors, work-unit table, zeroed
 * counters; room for split-K partials) into `plan`, caller-owned device memory of
 * at least qlin_chain_bytes() bytes, 16-byte aligned, kept for as long as the chain
 * is run.  Synchronizes `stream` once (the host image is copied).  The pointers of
 * the jobs are fixed in the plan: run it again after writing new inputs in place. */
int qlin_chain_init(const qlin_chain_job* jobs, int njobs, int M, void* plan, size_t plan_bytes,
                    void* stream);

/* Runs every job of the plan in one launch on `stream`, asynchronously; capturable
 * in a HIP graph.  The plan's counters return to zero when the launch ends.  Launches
 * of one plan must not overlap in time.  The int at byte offset 20 of the plan is 1
 * after a launch in which a dependency wait gave up (it polls about 4 M times), 0
 * otherwise; it describes the last finished launch. */
int qlin_chain_run(void* plan, void* stream);

/* ---------------------------------------------------------------------------
 * Engine decode chains: the engine-signature linears and their activation producers
 * between two mixer kernels, in one persistent launch
 *
 * The engine's decode step calls, between the attention / delta-rule kernels of two
 * layers (engine.py:236-279, 265-268, 272-279, 218-226):
 *   norm_gated_quant | gate_mul_quant -> gemm_i8 (o-projection, += hidden)
 *   -> rmsnorm_quant -> mlp_gate_up_quant -> gemm_i8 (down, += hidden)
 *   -> rmsnorm_quant -> proj3
 * A chain job is one of those linears -- what qlin_gemm_i8 / qlin_gemm_w4,
 * qlin_mlp_gate_up(_quant)_i8/_w4 or one column range of qlin_proj3_i8/_w4 computes --
 * with its activations either read from memory (a_q, a_s) or made by its producer
 * (`pro`, as the qlin_pro_* calls make them; the producer's input may be written by
 * an earlier level of the same chain).  Levels start at 0 and rise by at most 1 along
 * the list; level L > 0 starts only after every job of level L - 1 has written its
 * outputs.  Every job gives the same bits as the corresponding single call with 1-8
 * rows (those run the same work units as a one-job launch), and row m of an M-row
 * chain equals an M = 1 chain.  No reference counterpart as a function: the reference
 * launches a producer and a linear per projection and names whole-step capture as its
 * next step (ENGINEERING.md:383-399); each job replaces one such pair of launches.
 * ------------------------------------------------------------------------- */
#define QLIN_EJ_GEMM 1           /* out = a . W (+ residual), bf16 */
#define QLIN_EJ_GATE_UP 2        /* out = bf16(silu(a . Wg) * (a . Wu)) */
#define QLIN_EJ_GATE_UP_QUANT 3  /* out_q / out_s = per-64 int8 codes of that */

typedef struct qlin_echain_job {
  int kind;               /* QLIN_EJ_* */
  const int8_t* a_q;      /* int8 [M][K] (row stride K), or NULL with a producer */
  const float* a_s;       /* fp32 [M][K/64] */
  qlin_producer pro;      /* pro.kind 0: none; else as for the qlin_pro_* calls (pro.q /
                             pro.s, if given, receive the codes too) */
  int K, N;               /* K % 64 == 0, N % 16 == 0 (gate/up + quant: N % 64 == 0) */
  int group;              /* 0 = W8 (int8 [K][N], scale [N]); else the W4 group (a
                             multiple of 64 dividing K; packed [K/2][N], scale [K/G][N]) */
  const void* w;          /* the weight (gate for gate/up) */
  const void* scale;
  const uint8_t* zero;    /* W4 zeros [K/G][N] or NULL (z = 8) */
  const void* w2;         /* gate/up: the up weight, scale and zeros */
  const void* scale2;
  const uint8_t* zero2;
  int scale_dtype;        /* QLIN_F16, QLIN_BF16 or QLIN_F32 */
  void* out;              /* bf16 [M][ldo] (QLIN_EJ_GEMM, QLIN_EJ_GATE_UP) */
  int64_t ldo;
  const void* residual;   /* bf16 [M][ldr] or NULL; may alias out (QLIN_EJ_GEMM) */
  int64_t ldr;
  int8_t* out_q;          /* QLIN_EJ_GATE_UP_QUANT: codes [M][N], scales [M][N/64] */
  float* out_s;
  int level;              /* dependency level */
} qlin_echain_job;

/* Bytes of device memory an engine chain plan needs (0 if the jobs are invalid). */
size_t qlin_echain_bytes(const qlin_echain_job* jobs, int njobs, int M);

/* Validates the jobs (M = 1-8 rows; W8 jobs or W4 jobs, not both) and writes the plan
 * into `plan` (caller-owned device memory, qlin_echain_bytes() bytes, 16-byte
 * aligned), as qlin_chain_init does. */
int qlin_echain_init(const qlin_echain_job* jobs, int njobs, int M, void* plan, size_t plan_bytes,
                     void* stream);

/* Runs every job of the plan in one launch on `stream`, asynchronously; capturable in
 * a HIP graph.  Launches of one plan must not overlap in time.  The int at byte offset
 * 20 of the plan is 1 after a launch in which a wait gave up (a dependency or a split
 * tile's partial sums; each polls about 4 M times), 0 otherwise; it describes the last
 * finished launch.  The plan holds the split-K partial sums between the units of a
 * launch (its slots are left empty at the launch's end); after a launch that reported
 * 1, initialize the plan again (qlin_echain_init) before the next launch. */
int qlin_echain_run(void* plan, void* stream);

/* ---------------------------------------------------------------------------
 * Layout entry points (bit-exactness checks of the unpack / dequant)
 * ------------------------------------------------------------------------- */

/* nib[K,N] = nibble of packed[K/2,N] in natural K order (kernels/w4.py:51-61). */
int qlin_w4_unpack(const uint8_t* packed, int K, int N, uint8_t* nib, void* stream);

/* out[K,N] fp32 = (nibble - z) * scale[k/group, n] (quant_formats.py:6-8,
 * kernels/w4.py:103-104). */
int qlin_w4_dequant_f32(const uint8_t* packed, const void* scale, int s_dtype,
                        const uint8_t* zero, int group, int K, int N, float* out,
                        void* stream);

/* out[K,N] fp32 = w[k,n] * scale[n] (quant_formats.py:9). */
int qlin_w8_dequant_f32(const int8_t* w, const void* scale, int s_dtype, int K, int N,
                        float* out, void* stream);

/* ---------------------------------------------------------------------------
 * Load-time producers of the packed layouts (GPU requantization of fp32 weights)
 * ------------------------------------------------------------------------- */

/* Symmetric W4 per (group, column), replacing requant_w4_sym
 * (quant_formats.py:253-267): sc = max(amax over the group's K rows, 1e-8) / 7 in
 * fp32, code = clamp(round_half_even(w / sc), -8, 7) + 8, packed[K/2,N] with even K
 * in the low nibble (quant_formats.py:246-250), scale_bf16[K/group,N] = bf16(sc).
 * w is fp32 [K,N] (N contiguous); group is 32 or 64 and divides K. */
int qlin_requant_w4_sym(const float* w, int K, int N, int group, uint8_t* packed,
                        uint16_t* scale_bf16, void* stream);

/* Per-column W8, replacing requant_w8_row (quant_formats.py:270-275): sc[n] =
 * max(amax over K, 1e-8) / 127 in fp32, q = clamp(round_half_even(w / sc), -127, 127).
 * w is fp32 [K,N]; q int8 [K,N]; scale fp32 [N]. */
int qlin_requant_w8_row(const float* w, int K, int N, int8_t* q, float* scale, void* stream);

/* GPTQ int4 qweight int32 [K/8, N] (8 K-nibbles per word, nibble j = row 8w + j) ->
 * engine packed[K/2, N]: the nibble decode and pair packing of decode_gptq
 * (quant_formats.py:199-208, 369-372, 411-412, 428-429).  K % 8 == 0. */
int qlin_w4_repack_gptq(const int32_t* qweight, int K, int N, uint8_t* packed, void* stream);

/* AWQ int4 qweight int32 [K, N/8] (8 N-nibbles per word in AWQ order) -> engine
 * packed[K/2, N]: decode_awq's nibble decode, de-interleave and pair packing
 * (quant_formats.py:211-220, 442-444, 466).  K even, N % 8 == 0, packed 8-byte aligned. */
int qlin_w4_repack_awq(const int32_t* qweight, int K, int N, uint8_t* packed, void* stream);

/* compressed-tensors pack-quantized symmetric int4 weight_packed int32 [N, W] (8
 * straight-order K nibbles per word, one output feature per row) -> engine packed
 * [K/2, N]: the nibble decode, trim to K and pair packing of the transposed nibbles in
 * decode_ct (quant_formats.py:199-208, 311-316, 348-349).  Even K <= 8 W, N % 16 == 0,
 * packed 16-byte aligned.  The group scales [N, K/G] are transposed by the caller
 * (quant_formats.py:350). */
int qlin_w4_repack_ct(const int32_t* weight_packed, int N, int W, int K, uint8_t* packed, void* stream);

/* qzeros int32 [G, N/8] (8 N-nibbles per word; AWQ order if awq_order) -> uint8
 * zeros[G, N] = nibble + add: GPTQ's effective zero is nibble + 1
 * (quant_formats.py:396-400, 418-424), AWQ's the nibble (quant_formats.py:445-446). */
int qlin_w4_zeros_unpack(const int32_t* qzeros, int G, int N, int awq_order, int add, uint8_t* zeros,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QLIN_H */
