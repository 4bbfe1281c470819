// Device-side helpers for the gfx950 quantized-linear kernels.
//
// The engine's weight layouts are N-contiguous (int8 [K,N], packed nibbles [K/2,N]),
// so a 128-bit load gives one lane 16 adjacent output columns of one K row.  CDNA
// MFMA wants the opposite in each lane: several consecutive K values of ONE output
// column.  The helpers below rebuild MFMA operands in registers with v_perm_b32 byte
// permutes (no LDS round trip):
//
//   * f16 operands: a pair of K values of one column becomes one f16x2 through the
//     exponent-bias trick: 0x6400 | u is the fp16 value 1024 + u for 0 <= u < 1024,
//     so one permute plus one packed fp16 add/fma yields exact small integers.
//   * i8 operands: 4x4 byte transposes (8 permutes per 4 output dwords).
//
// All arithmetic here is exact: every integer weight value in [-128, 127] and every
// nibble difference is representable in fp16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace qlin {

enum ActKind { ACT_F16 = 0, ACT_I8 = 1 };
enum WKind { WK_W8 = 0, WK_W4 = 1 };
enum EpiKind { EPI_STORE = 0, EPI_GATEUP = 1, EPI_GATEUP_Q = 2 };
enum DType { DT_F16 = 1, DT_BF16 = 2, DT_F32 = 3 };

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

template <typename T, typename F>
__device__ __forceinline__ T bitcast(F f) {
  return __builtin_bit_cast(T, f);
}

// Load of a T from global memory through a generic pointer.  A plain dereference of a
// pointer the compiler cannot place (one read from a descriptor in memory) becomes a
// flat load, which counts on the LDS counter as well: every later wait for an LDS
// access then also waits for it, draining a register ring of weight loads.
template <typename T>
__device__ __forceinline__ T ld_global(const void* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}

// The same as a non-temporal load: for weights, which a decode step reads exactly once.
// A plain streaming-read probe reads 6.1 TB/s with it against 5.6 without.
template <typename T>
__device__ __forceinline__ T ld_global_nt(const void* p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) T*)p);
}

// f(std::integral_constant<int, I>{}) for I = B .. E-1, unrolled at compile time.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// ---------------------------------------------------------------------------
// fp16 operands
// ---------------------------------------------------------------------------

// Two int8 weights of the same column from two K rows -> exact f16x2.
// d0/d1: dwords of rows k and k+1 holding the column's byte at position `b`
// (b must fold to a constant after unrolling so the permute selector is an immediate).
// perm gives [d0.b, 0, d1.b, 0]; xor 0x64806480 sets the 0x64 exponent byte and
// flips the sign bit (u = b + 128), so each half is 1024 + 128 + b; subtracting
// 1152 leaves b exactly.
__device__ __forceinline__ uint32_t w8_pair_f16(uint32_t d0, uint32_t d1, int b) {
  const uint32_t sel = 0x0c000c00u | ((4u + (uint32_t)b) << 16) | (uint32_t)b;
  const uint32_t p = perm(d1, d0, sel) ^ 0x64806480u;
  const f16x2 h = bitcast<f16x2>(p) - f16x2{(_Float16)1152.0f, (_Float16)1152.0f};
  return bitcast<uint32_t>(h);
}

// The two nibbles (k even = low nibble, k odd = high nibble) of one packed byte ->
// exact f16x2 (nibble_lo - z, nibble_hi - z).  perm duplicates the byte under two
// 0x64 exponent bytes; the mask keeps the low nibble in half 0 (1024 + lo) and the
// high nibble in place in half 1 (1024 + 16*hi); one packed fma with
// (1, 1/16) and bias = (-1024 - z, -64 - z) finishes both exactly.
__device__ __forceinline__ uint32_t w4_pair_f16(uint32_t d, int b, f16x2 bias) {
  const uint32_t sel = (uint32_t)b | (4u << 8) | ((uint32_t)b << 16) | (4u << 24);
  const uint32_t p = perm(0x64646464u, d, sel) & 0xFFF0FF0Fu;
  const f16x2 h = bitcast<f16x2>(p);
  const f16x2 m = f16x2{(_Float16)1.0f, (_Float16)0.0625f};
  return bitcast<uint32_t>(__builtin_elementwise_fma(h, m, bias));
}

__device__ __forceinline__ f16x2 w4_bias(uint32_t z) {
  return f16x2{(_Float16)(-1024.0f - (float)z), (_Float16)(-64.0f - (float)z)};
}

// The two nibbles of one packed byte -> exact f16x2 (1024 + lo, 64 + hi) in two
// instructions: perm puts the byte under the exponent byte 0x64 in half 0 and 0x54
// in half 1; the mask keeps the low nibble in the unit bits of 0x6400 = 1024 and the
// high nibble in bits 4-7 of 0x5400 = 64, where bit 4 has weight 1.  The caller
// removes the offsets after the MFMA: sum_k x_k * offset_k is one more MFMA of the
// activations against a constant operand, shared by every column.
__device__ __forceinline__ uint32_t w4_pair_offset(uint32_t d, int b) {
  const uint32_t sel = (uint32_t)b | (4u << 8) | ((uint32_t)b << 16) | (5u << 24);
  return perm(0x00005464u, d, sel) & 0x54F0640Fu;
}

// ---------------------------------------------------------------------------
// int8 operands
// ---------------------------------------------------------------------------

// 4x4 byte transpose: out[u].byte[r] = in[r].byte[u].
__device__ __forceinline__ void tr4(const uint32_t in0, const uint32_t in1, const uint32_t in2,
                                    const uint32_t in3, uint32_t out[4]) {
  const uint32_t t0 = perm(in1, in0, 0x05010400u);  // in0.b0 in1.b0 in0.b1 in1.b1
  const uint32_t t1 = perm(in1, in0, 0x07030602u);  // in0.b2 in1.b2 in0.b3 in1.b3
  const uint32_t t2 = perm(in3, in2, 0x05010400u);
  const uint32_t t3 = perm(in3, in2, 0x07030602u);
  out[0] = perm(t2, t0, 0x05040100u);
  out[1] = perm(t2, t0, 0x07060302u);
  out[2] = perm(t3, t1, 0x05040100u);
  out[3] = perm(t3, t1, 0x07060302u);
}

// Packed nibbles -> int8 holding 16 * (nibble - 8): xor 0x88 maps nibble n to the
// 4-bit two's complement of n - 8; moved to the top of the byte it reads as an int8
// equal to 16 * (n - 8).  lo: even-k nibbles, hi: odd-k nibbles.
__device__ __forceinline__ void w4_split_i8x16(uint32_t d, uint32_t& lo, uint32_t& hi) {
  const uint32_t x = d ^ 0x88888888u;
  hi = x & 0xF0F0F0F0u;
  lo = (x << 4) & 0xF0F0F0F0u;
}

// ---------------------------------------------------------------------------
// Split-K partials in the caller's workspace
// ---------------------------------------------------------------------------

// 16-byte loads and stores with the SC1 cache policy: device-coherent, the form that
// agent-scope atomics take on gfx950.  A partial written this way by a workgroup on
// one XCD is read correctly by a workgroup on another, without an L2 writeback or
// invalidate, and the compiler tracks the loads like ordinary ones.
constexpr int kCpolSc1 = 16;

// raw buffer over `bytes` bytes from `base` (gfx9 descriptor word 3)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void st_coherent(const f32x4 v, __amdgpu_buffer_rsrc_t r, unsigned off) {
  __builtin_amdgcn_raw_buffer_store_b128(bitcast<u32x4>(v), r, off, 0, kCpolSc1);
}

__device__ __forceinline__ f32x4 ld_coherent(__amdgpu_buffer_rsrc_t r, unsigned off) {
  return bitcast<f32x4>(__builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolSc1));
}

// Partial-sum slots of the decode units' polling exchange hold an empty mark in every
// word until a unit stores its part: -0.0, which a part never is (every sum starts from
// +0.0, and a rounded sum or fused multiply-add is -0.0 only when its addend is).  With
// FLIP a part is stored with its sign bits flipped, so the mark is a zero word: a slot
// the caller zeroed, or one zeroed again after its tile finished.  A reader polls until
// no word of the slot holds the mark.
__device__ __forceinline__ uint32_t sign_mask() {
  // (made where it is used: a persistent kernel would hoist the constant out of its loop
  // and spill it)
  uint32_t m;
  asm volatile("v_bfrev_b32 %0, 1" : "=v"(m));
  return m;
}

template <bool FLIP>
__device__ __forceinline__ f32x4 part_code(f32x4 v) {
  if constexpr (!FLIP) return v;
  const uint32_t m = sign_mask();
  return bitcast<f32x4>(bitcast<u32x4>(v) ^ u32x4{m, m, m, m});
}

template <bool FLIP>
__device__ __forceinline__ bool part_empty(f32x4 stored) {
  const u32x4 b = bitcast<u32x4>(stored);
  const uint32_t e = FLIP ? 0u : 0x80000000u;
  return b.x == e || b.y == e || b.z == e || b.w == e;
}

template <bool FLIP>
__device__ __forceinline__ f32x4 part_mark() {
  if constexpr (FLIP) return f32x4{0.f, 0.f, 0.f, 0.f};
  const uint32_t m = sign_mask();
  return bitcast<f32x4>(u32x4{m, m, m, m});
}

// ---------------------------------------------------------------------------
// MFMA wrappers (16x16 output; lane l holds D[4*(l/16)+r][l%16], r = 0..3)
// ---------------------------------------------------------------------------

__device__ __forceinline__ f32x4 mfma_f16(const f16x8 a, const f16x8 b, const f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i32x4 mfma_i8(const uint64_t a, const uint64_t b, const i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Element conversions
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return bitcast<float>((uint32_t)b << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN -> quiet NaN), as torch's cast.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = bitcast<uint32_t>(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)0x7FC0;
  return (uint16_t)((u + (((u >> 16) & 1u) + 0x7FFFu)) >> 16);
}

__device__ __forceinline__ float load_scale(const void* p, int dt, long long i) {
  if (dt == DT_F32) return ((const float*)p)[i];
  if (dt == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  return (float)((const _Float16*)p)[i];
}

// Raw bits of 4 consecutive scale values (fp32: 16 bytes; 16-bit types: 8 bytes,
// read twice), loaded without a branch on the dtype: a load issued early and merged
// at a control-flow join is waited for at the join.  idx must be a multiple of 4.
__device__ __forceinline__ u32x4 ld_scale4_raw(const void* p, int dt, long long idx) {
  const bool f32 = dt == DT_F32;
  const uint8_t* base = (const uint8_t*)p + idx * (f32 ? 4 : 2);
  const u32x2 v0 = ld_global<u32x2>(base);
  const u32x2 v1 = ld_global<u32x2>(base + (f32 ? 8 : 0));
  return u32x4{v0.x, v0.y, v1.x, v1.y};
}

__device__ __forceinline__ void cvt_scale4(const u32x4 raw, int dt, float out[4]) {
  if (dt == DT_F32) {
    out[0] = bitcast<float>(raw.x), out[1] = bitcast<float>(raw.y);
    out[2] = bitcast<float>(raw.z), out[3] = bitcast<float>(raw.w);
    return;
  }
  const uint32_t w[2] = {raw.x, raw.y};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    out[e] = (dt == DT_BF16) ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
  }
}

// One scale value as raw bits, loaded without a branch on the dtype: the aligned
// dword holding element idx (for 16-bit types it also holds the neighbour).
__device__ __forceinline__ uint32_t ld_scale1_raw(const void* p, int dt, long long idx) {
  const long long byte = (dt == DT_F32) ? idx * 4 : ((idx * 2) & ~3LL);
  return ld_global<uint32_t>((const uint8_t*)p + byte);
}

// The value of ld_scale1_raw's dword for element idx (only idx's parity is used).
__device__ __forceinline__ float cvt_scale1(uint32_t raw, int dt, long long idx) {
  if (dt == DT_F32) return bitcast<float>(raw);
  const uint16_t h = (uint16_t)(raw >> (16 * (int)(idx & 1)));
  return (dt == DT_BF16) ? bf16_to_f32(h) : (float)bitcast<_Float16>(h);
}

__device__ __forceinline__ float load_act16(const void* p, int dt, long long i) {
  if (dt == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  return (float)((const _Float16*)p)[i];
}

__device__ __forceinline__ uint16_t to_out16(float v, int dt) {
  if (dt == DT_BF16) return f32_to_bf16(v);
  return bitcast<uint16_t>((_Float16)v);
}

// x * sigmoid(x) (kernels/common.py:32-34).
__device__ __forceinline__ float silu(float x) { return x * (1.0f / (1.0f + expf(-x))); }

// Round half away from zero with the add in fp32, truncate, clamp to [-127, 127]
// (kernels/common.py:24-29).
__device__ __forceinline__ int round_i8(float v) {
  const float t = v + (v >= 0.0f ? 0.5f : -0.5f);
  int r = (int)t;
  r = r < -127 ? -127 : r;
  r = r > 127 ? 127 : r;
  return r;
}

}  // namespace qlin
