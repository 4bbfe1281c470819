"""CPU oracle for the quantized-linear path -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
may import this module, and only as the checker (or, in bench.py, as the timed CPU
baseline).  The product path (the `kernels` package and `libqlin.so`) never calls it.

What it restates (numpy, float32 unless stated), each function citing the reference
file:line it follows (paths relative to the reference checkout):

* packed-nibble layout of the engine W4 format and its unpack / dequant;
* the engine W8 format (int8 [K, N] + one scale per output column);
* the fp32 GEMM the reference's CPU path runs after dequantization
  (dequantize, then an fp32 matmul);
* the engine-signature activations `a_q * a_s[k // 64]`;
* the fused epilogues: residual add, three-way column concatenation (proj3),
  `silu(g) * u`, bf16 round trip, per-64-column int8 re-quantization with
  round-half-away-from-zero;
* the load-time producers of the packed layouts (symmetric W4 / per-row W8
  requantization) and the external int4 formats' nibble decode into them (GPTQ
  K-packed words, AWQ N-packed words in AWQ order, their packed zeros).

Pinning (see tests/test_oracle.py): brute force over all 256 byte values, known-answer
bytes, pack/unpack round trips, closed forms (one-hot activations, unit scales,
z == nibble), an fp64 matmul bounding the fp32 oracle's own error, torch's bf16 cast
and silu as library references, and the fused == unfused composition the reference's
own test_fused.py checks.  Every public function here has at least one such check;
none is "parity unpinned".
"""
from __future__ import annotations

import numpy as np

# Activation quantization group along K (kernels/common.py:5-7).
GROUP = 64
# Zero point of the symmetric engine W4 grid (kernels/w4.py:35-37).
W4_ZERO = 8


# ----------------------------------------------------------------------------
# bf16 helpers (numpy has no bfloat16; bf16 values travel as uint16 bit patterns)
# ----------------------------------------------------------------------------

def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit pattern, round-to-nearest-even (torch's `.to(bfloat16)`)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    bias = ((u >> 16) & 1) + 0x7FFF
    r = ((u + bias) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = r.copy()
        r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """fp32 -> bf16 -> fp32 round trip (`h.to(tl.bfloat16).to(tl.float32)`,
    kernels/gemm.py:198-200, kernels/w4.py:285-286)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# ----------------------------------------------------------------------------
# W4 packed-nibble layout
# ----------------------------------------------------------------------------

def pack_pairs(nib) -> np.ndarray:
    """nibbles [K, N] (values 0..15) -> packed uint8 [K//2, N]; even k in the low
    nibble, odd k in the high nibble (quant_formats.py:246-250 `_pairs_from`,
    quant_formats.py:223-229 `_pack_pairs`, kernels/w4.py:5-6)."""
    nib = np.asarray(nib)
    K = nib.shape[0] - (nib.shape[0] % 2)
    lo = nib[0:K:2].astype(np.int32)
    hi = nib[1:K:2].astype(np.int32)
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_w4(packed) -> np.ndarray:
    """packed uint8 [K//2, N] -> nibbles uint8 [K, N] in natural K order
    (kernels/w4.py:51-52 `lo = v & 0x0F`, `hi = (v >> 4) & 0x0F`; w4.py:59-61
    interleave: even k = low nibble, odd k = high nibble)."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty((p.shape[0] * 2,) + p.shape[1:], dtype=np.uint8)
    out[0::2] = p & 0x0F
    out[1::2] = (p >> 4) & 0x0F
    return out


def w4_group(K: int, scale) -> int:
    """Weight-group size from the scale rows: `wgrp = K // b_s.shape[0]`
    (kernels/w4.py:155)."""
    return K // np.asarray(scale).shape[0]


def w4_int(packed, zeros=None, group: int | None = None) -> np.ndarray:
    """Signed integer weights `nibble - z` as int16 [K, N].  `z` is the per-(group,
    column) zero `zeros[k // group, n]` when given, else the constant 8
    (kernels/w4.py:8-11, 53-58, 82-88)."""
    nib = unpack_w4(packed).astype(np.int16)
    if zeros is None:
        return nib - W4_ZERO
    z = np.asarray(zeros, dtype=np.uint8).astype(np.int16)
    if group is None:
        group = nib.shape[0] // z.shape[0]
    return nib - np.repeat(z, group, axis=0)


def scale_to_f32(scale) -> np.ndarray:
    """Scales stored fp16 / fp32 (numpy dtypes) or bf16 (uint16 bit patterns) ->
    float32; the reference kernels load them `.to(tl.float32)` (kernels/w4.py:103)."""
    s = np.asarray(scale)
    if s.dtype == np.uint16:
        return bf16_bits_to_f32(s)
    return s.astype(np.float32)


def dequant_w4_f32(packed, scale, zeros=None) -> np.ndarray:
    """Engine W4 -> fp32 [K, N]: `(nibble - z) * s[k // G, n]` (quant_formats.py:6-8,
    kernels/w4.py:103-104).  Exact in fp32 for fp16 / bf16 scales."""
    s = scale_to_f32(scale)
    K = np.asarray(packed).shape[0] * 2
    G = K // s.shape[0]
    q = w4_int(packed, zeros, G).astype(np.float32)
    return q * np.repeat(s, G, axis=0)


def dequant_w8_f32(w, scale) -> np.ndarray:
    """Engine W8 -> fp32 [K, N]: `W[k, n] * s[n]` (quant_formats.py:9,
    .dev/test_kernels.py:40-41 `b.float() ... * bs[None, :]`)."""
    return np.asarray(w, dtype=np.int8).astype(np.float32) * scale_to_f32(scale)[None, :]


# ----------------------------------------------------------------------------
# A16 core: fp16/fp32 activations, dequantize then fp32 matmul
# ----------------------------------------------------------------------------

def linear_ref(x, w_f32, residual=None) -> np.ndarray:
    """`y = x @ W_dq` in fp32 (the reference CPU path: dequantize, then an fp32
    matmul), with an optional residual added in fp32."""
    y = np.asarray(x, dtype=np.float32) @ np.asarray(w_f32, dtype=np.float32)
    if residual is not None:
        y = y + _as_f32(residual)
    return y.astype(np.float32)


def linear_w8_ref(x, w, scale, residual=None) -> np.ndarray:
    return linear_ref(x, dequant_w8_f32(w, scale), residual)


def linear_w4_ref(x, packed, scale, zeros=None, residual=None) -> np.ndarray:
    return linear_ref(x, dequant_w4_f32(packed, scale, zeros), residual)


def _as_f32(t) -> np.ndarray:
    t = np.asarray(t)
    if t.dtype == np.uint16:          # bf16 bit patterns
        return bf16_bits_to_f32(t)
    return t.astype(np.float32)


# ----------------------------------------------------------------------------
# Engine signature: int8 activations with one fp32 scale per 64 K-elements
# ----------------------------------------------------------------------------

def act_dequant(a_q, a_s) -> np.ndarray:
    """`a_q * a_s.repeat_interleave(64, dim=1)` (.dev/test_kernels.py:40,
    .dev/test_fused.py:18-19)."""
    a_s = np.asarray(a_s, dtype=np.float32)
    return np.asarray(a_q, dtype=np.int8).astype(np.float32) * np.repeat(a_s, GROUP, axis=1)


def gemm_i8_ref(a_q, a_s, b, b_s, residual=None, b_z=None) -> np.ndarray:
    """fp32 result of `gemm_i8` (kernels/gemm.py:60-92): `(a_q * a_s) @ (b * b_s)`
    [+ residual] (.dev/test_kernels.py:40-46).  Dispatches to the W4 form when `b`
    is uint8 packed nibbles (kernels/gemm.py:15-17, 69-72)."""
    b = np.asarray(b)
    if b.dtype == np.uint8:
        return gemm_w4_ref(a_q, a_s, b, b_s, b_z=b_z, residual=residual)
    return linear_ref(act_dequant(a_q, a_s), dequant_w8_f32(b, b_s), residual)


def gemm_w4_ref(a_q, a_s, b, b_s, b_z=None, residual=None) -> np.ndarray:
    """fp32 result of `gemm_w4` (kernels/w4.py:139-166)."""
    return linear_ref(act_dequant(a_q, a_s), dequant_w4_f32(b, b_s, b_z), residual)


def proj3_ref(a_q, a_s, w1, s1, w2, s2, w3, s3, z1=None, z2=None, z3=None) -> np.ndarray:
    """Three projections sharing `(a_q, a_s)`, written side by side as
    `[:, 0:N1] [N1:N1+N2] [N1+N2:NT]` (kernels/gemm.py:238-239, 290-312;
    kernels/w4.py:220-251; .dev/test_kernels.py:49-63).  `None` weights give
    zero columns (gemm.py:296-302)."""
    parts = []
    for w, s, z in ((w1, s1, z1), (w2, s2, z2), (w3, s3, z3)):
        if w is None:
            continue
        parts.append(gemm_i8_ref(a_q, a_s, w, s, b_z=z))
    return np.concatenate(parts, axis=1)


def silu(x) -> np.ndarray:
    """`x * sigmoid(x)` (kernels/common.py:32-34) in fp32."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (x * (np.float32(1.0) / (np.float32(1.0) + np.exp(-x)))).astype(np.float32)


def mlp_gate_up_ref(a_q, a_s, wg, sg, wu, su, zg=None, zu=None) -> np.ndarray:
    """fp32 `silu(gate) * up` before the bf16 store (kernels/gemm.py:95-137,
    kernels/w4.py:284; .dev/test_kernels.py:76-79)."""
    g = gemm_i8_ref(a_q, a_s, wg, sg, b_z=zg)
    u = gemm_i8_ref(a_q, a_s, wu, su, b_z=zu)
    return (silu(g) * u).astype(np.float32)


def round_i8(v) -> np.ndarray:
    """Round half away from zero, clamp to [-127, 127] (kernels/common.py:24-29):
    `r = int32(v + (v >= 0 ? 0.5 : -0.5))` with the add done in fp32 and the cast
    truncating toward zero."""
    v = np.asarray(v, dtype=np.float32)
    half = np.where(v >= np.float32(0.0), np.float32(0.5), np.float32(-0.5)).astype(np.float32)
    with np.errstate(invalid="ignore"):
        r = np.trunc(v + half)
    r = np.clip(r, -127, 127)
    return r.astype(np.int8)


def quant_groups(h) -> tuple[np.ndarray, np.ndarray]:
    """Per-64-column int8 quantization of fp32 rows (kernels/norm.py:15-25,
    kernels/gemm.py:202-211): `sc = max(amax / 127, 1e-8)`, `q = round_i8(h / sc)`.
    Returns (q int8 [M, N], sc fp32 [M, N // 64])."""
    h = np.asarray(h, dtype=np.float32)
    M, N = h.shape
    h3 = h.reshape(M, N // GROUP, GROUP)
    amax = np.abs(h3).max(axis=2)
    sc = np.maximum(amax / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    q = round_i8(h3 / sc[:, :, None]).reshape(M, N)
    return q, sc


def mlp_gate_up_quant_ref(a_q, a_s, wg, sg, wu, su, zg=None, zu=None):
    """Fused gate/up + SiLU*mul + bf16 round trip + per-64 int8 quant
    (kernels/gemm.py:154-231, kernels/w4.py:254-323)."""
    h = round_bf16(mlp_gate_up_ref(a_q, a_s, wg, sg, wu, su, zg, zu))
    return quant_groups(h)


# ----------------------------------------------------------------------------
# Activation producers (kernels/norm.py): 16-bit activations -> int8 codes + per-64
# fp32 scales, the input of every engine-signature linear
#
# The reference computes these in Triton, whose reduction order and rsqrt/exp are
# implementation details; the kernels here fix them, and these functions restate the
# fixed form operation by operation (float32, every operation rounded, no fused
# multiply-add), so the int8 codes can be compared bit for bit.
# ----------------------------------------------------------------------------

# exp(x) = 2^n * exp(r), n = rint(x * log2(e)), r = x - n * ln2 with ln2 split in two
# (Cody and Waite): LN2_HI has 15 significant bits, so n * LN2_HI is exact for |n| <= 127.
LOG2E_F32 = np.float32(float.fromhex("0x1.715476p+0"))
LN2_HI_F32 = np.float32(float.fromhex("0x1.62e4p-1"))
LN2_LO_F32 = np.float32(float.fromhex("0x1.7f7d1cp-20"))
# Taylor coefficients 1/7!, 1/6!, ..., 1/0! rounded to fp32 (Horner order)
EXP_POLY_F32 = [np.float32(float.fromhex(h)) for h in (
    "0x1.a01a02p-13", "0x1.6c16c2p-10", "0x1.111112p-7", "0x1.555556p-5",
    "0x1.555556p-3", "0x1p-1", "0x1p+0", "0x1p+0")]


def exp_f32(x) -> np.ndarray:
    """exp in fp32 as the producer kernels compute it (they need no libm): Cody-Waite
    reduction, the degree-7 Taylor polynomial of exp(r) on |r| <= ln2/2 in Horner
    form, then the exact scaling by 2^n; +inf above 88, 0 below -87 (so no result is
    subnormal).  Stands in for the reference's `tl.exp` / `tl.sigmoid`
    (kernels/norm.py:178, kernels/common.py:32-34)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        n = np.rint(x * LOG2E_F32).astype(np.float32)
        r = ((x - n * LN2_HI_F32) - n * LN2_LO_F32).astype(np.float32)
        p = np.full_like(r, EXP_POLY_F32[0])
        for c in EXP_POLY_F32[1:]:
            p = (p * r).astype(np.float32)
            p = (p + c).astype(np.float32)
        ni = np.where(np.isfinite(n), n, 0).astype(np.int32)
        y = np.ldexp(p, ni).astype(np.float32)
    y = np.where(x > np.float32(88.0), np.float32(np.inf), y)
    y = np.where(x < np.float32(-87.0), np.float32(0.0), y)
    return y.astype(np.float32)


def sigmoid_f32(x) -> np.ndarray:
    """`1 / (1 + exp(-x))` with exp_f32 (tl.sigmoid, kernels/norm.py:178)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", divide="ignore"):
        return (np.float32(1.0) / (np.float32(1.0) + exp_f32(-x))).astype(np.float32)


def silu_f32(x) -> np.ndarray:
    """`x * sigmoid(x)` with exp_f32 (kernels/common.py:32-34, used by
    kernels/norm.py:114)."""
    x = np.asarray(x, dtype=np.float32)
    return (x * sigmoid_f32(x)).astype(np.float32)


def sumsq_lanes(x, lanes: int) -> np.ndarray:
    """Sum of squares of each row of x [M, L] in the kernels' fixed order: 8-element
    chunks; lane l of `lanes` folds chunks l, l + lanes, ... (each chunk's elements
    in order, `acc = acc + v * v`, both operations rounded); then an xor butterfly
    over the lanes (`acc = acc + acc[l ^ m]` for m = lanes/2, ..., 1).  The reference
    writes `tl.sum(x * x, axis=0)` (kernels/norm.py:39, 113) and leaves the order to
    Triton."""
    x = np.asarray(x, dtype=np.float32)
    M, L = x.shape
    assert L % 8 == 0 and lanes & (lanes - 1) == 0
    x2 = (x * x).astype(np.float32)
    nc = L // 8
    P = -(-nc // lanes)
    pad = np.zeros((M, P * lanes * 8), dtype=np.float32)  # + 0.0 leaves a sum of squares unchanged
    pad[:, :L] = x2
    X = pad.reshape(M, P, lanes, 8)
    acc = np.zeros((M, lanes), dtype=np.float32)
    for i in range(P):
        for e in range(8):
            acc = (acc + X[:, i, :, e]).astype(np.float32)
    idx = np.arange(lanes)
    m = lanes // 2
    while m >= 1:
        acc = (acc + acc[:, idx ^ m]).astype(np.float32)
        m //= 2
    return acc[:, 0]


def rms_inv(ss, n: int, eps: float) -> np.ndarray:
    """`rsqrt(ss / n + eps)` as `1 / sqrt(.)`, each operation correctly rounded in
    fp32 (kernels/norm.py:39-40, 113-114 use tl.rsqrt)."""
    ss = np.asarray(ss, dtype=np.float32)
    var = (ss / np.float32(n)).astype(np.float32)
    return (np.float32(1.0) / np.sqrt((var + np.float32(eps)).astype(np.float32))).astype(np.float32)


def rmsnorm_quant_ref(x, w, eps: float = 1e-6, one_plus: bool = True):
    """RMSNorm of each row, then per-64 int8 quant (kernels/norm.py:28-57):
    `y = x * rsqrt(mean(x^2) + eps) * (w + 1 if one_plus else w)`, left to right,
    then `_quant_groups` (norm.py:15-25).  The sum of squares is one 64-lane
    sumsq_lanes.  x: [M, K] values of the 16-bit input; w: [K].
    Returns (q int8 [M, K], s fp32 [M, K // 64])."""
    x = np.asarray(x, dtype=np.float32)
    w = np.asarray(w, dtype=np.float32)
    if one_plus:
        w = (w + np.float32(1.0)).astype(np.float32)
    r = rms_inv(sumsq_lanes(x, 64), x.shape[1], eps)
    y = ((x * r[:, None]).astype(np.float32) * w[None, :]).astype(np.float32)
    return quant_groups(y)


def gate_cols(N: int, hd: int) -> np.ndarray:
    """Column of the gate of activation column k in G [M, heads, 2 hd], the gate
    in the second half of each head (kernels/norm.py:171, 176)."""
    k = np.arange(N)
    return (k // hd) * (2 * hd) + hd + (k % hd)


def gate_mul_quant_ref(a, g, hd: int = 256):
    """`y = a * sigmoid(G[gate column])`, then per-64 int8 quant
    (kernels/norm.py:168-188).  a: [M, N]; g: [M, >= 2 N] gate rows."""
    a = np.asarray(a, dtype=np.float32)
    g = np.asarray(g, dtype=np.float32)
    gv = g[:, gate_cols(a.shape[1], hd)]
    y = (a * sigmoid_f32(gv)).astype(np.float32)
    return quant_groups(y)


def norm_gated_quant_ref(v, z, w, eps: float = 1e-6):
    """Per (row, head) gated RMSNorm, bf16 round trip, per-64 int8 quant
    (kernels/norm.py:95-137): `y = x * rsqrt(mean_head(x^2) + eps) * w * silu(z)`,
    left to right; hd = len(w).  The head's sum of squares is one sumsq_lanes over
    hd / 8 lanes (one 8-element chunk each).  v, z: [T, N] (z already the gate
    columns); w: [hd].  Returns (q int8 [T, N], s fp32 [T, N // 64])."""
    v = np.asarray(v, dtype=np.float32)
    z = np.asarray(z, dtype=np.float32)
    w = np.asarray(w, dtype=np.float32)
    T, N = v.shape
    hd = w.shape[0]
    heads = v.reshape(T * (N // hd), hd)
    r = rms_inv(sumsq_lanes(heads, hd // 8), hd, eps).reshape(T, N // hd)
    rr = np.repeat(r, hd, axis=1)
    ww = np.tile(w, N // hd)
    y = ((v * rr).astype(np.float32) * ww[None, :]).astype(np.float32)
    y = (y * silu_f32(z)).astype(np.float32)
    return quant_groups(round_bf16(y))


# ----------------------------------------------------------------------------
# Load-time producers of the packed layouts (read-only contract)
# ----------------------------------------------------------------------------

def requant_w4_sym(w, group: int = 32):
    """float [K, N] -> (packed uint8 [K//2, N], bf16 scale bits [K//group, N])
    (quant_formats.py:253-267): `sc = amax / 7` in fp32 (clamped at 1e-8),
    `q = clamp(round_half_even(w / sc), -8, 7) + 8`, scale stored as bf16."""
    w = np.asarray(w, dtype=np.float32)
    K, N = w.shape
    q4 = w.reshape(K // group, group, N)
    sc = (np.maximum(np.abs(q4).max(axis=1), np.float32(1e-8)) / np.float32(7.0)).astype(np.float32)
    q = np.clip(np.rint(q4 / sc[:, None, :]), -8, 7) + 8
    return pack_pairs(q.reshape(K, N).astype(np.uint8)), f32_to_bf16_bits(sc)


def requant_w8_row(w):
    """float [K, N] -> (int8 [K, N], fp32 scale [N]) per-column symmetric
    (quant_formats.py:270-275); round half to even like `torch.round`."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.maximum(np.abs(w).max(axis=0), np.float32(1e-8))
    sc = (amax / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.rint(w / sc[None, :]), -127, 127).astype(np.int8)
    return q, sc


def nibbles_i32(qw, bits: int = 4) -> np.ndarray:
    """int32 packed [R, W] -> uint8 nibbles [R, W * 32/bits] in straight bit order:
    element j of word w is bits j*bits .. j*bits+bits-1 (quant_formats.py:199-208)."""
    q = np.asarray(qw).astype(np.int64) & 0xFFFFFFFF
    epf = 32 // bits
    shifts = np.arange(epf, dtype=np.int64) * bits
    n = ((q[..., None] >> shifts) & ((1 << bits) - 1)).astype(np.uint8)
    return n.reshape(n.shape[0], -1)


AWQ_ORDER = np.array([0, 4, 1, 5, 2, 6, 3, 7])


def deinterleave_awq(nib) -> np.ndarray:
    """Restore AutoAWQ's nibble order along the last axis: out[:, c] = in[:, REV[c]]
    per group of 8 with REV = [0, 4, 1, 5, 2, 6, 3, 7] (quant_formats.py:211-220)."""
    nib = np.asarray(nib)
    g = nib.reshape(*nib.shape[:-1], -1, 8)
    return g[..., AWQ_ORDER].reshape(nib.shape)


def gptq_w4_to_engine(qweight) -> np.ndarray:
    """GPTQ int4 qweight int32 [K/8, N] (8 K-nibbles per word, one column) -> engine
    packed [K/2, N] (quant_formats.py:369-372 then 246-250)."""
    qw = np.asarray(qweight)
    R, N = qw.shape
    nib = nibbles_i32(qw).reshape(R, N, 8).transpose(0, 2, 1).reshape(R * 8, N)
    return pack_pairs(nib)


def awq_w4_to_engine(qweight) -> np.ndarray:
    """AWQ int4 qweight int32 [K, N/8] (8 N-nibbles per word in AWQ order) -> engine
    packed [K/2, N] (quant_formats.py:442-444 then 246-250)."""
    nib = deinterleave_awq(nibbles_i32(qweight))
    return pack_pairs(nib)


def ct_w4_to_engine(weight_packed, K: int | None = None) -> np.ndarray:
    """compressed-tensors pack-quantized symmetric int4: weight_packed int32 [N, W]
    (8 K-nibbles per word in straight order along the input dimension, one output
    feature per row) -> engine packed [K/2, N]: the straight-order nibble decode
    (quant_formats.py:199-208, 311), the trim to K (quant_formats.py:315-316, 329),
    then the pair packing of the transposed nibbles (quant_formats.py:348-349,
    246-250).  K defaults to 8 W."""
    qw = np.asarray(weight_packed)
    nib = nibbles_i32(qw)
    if K is not None:
        nib = nib[:, :K]
    return pack_pairs(nib.T)


def ct_scale_to_engine(weight_scale) -> np.ndarray:
    """compressed-tensors group scales [N, K/G] -> engine [K/G, N]
    (quant_formats.py:324-327, 350)."""
    return np.ascontiguousarray(np.asarray(weight_scale).T)


def gptq_zeros(qzeros, plus_one: bool = True) -> np.ndarray:
    """GPTQ qzeros int32 [G, N/8] -> uint8 zeros [G, N], N-packed straight order, with
    the +1 of the effective zero (quant_formats.py:396-400, 418-424)."""
    z = nibbles_i32(qzeros).astype(np.int32) + (1 if plus_one else 0)
    return z.astype(np.uint8)


def awq_zeros(qzeros) -> np.ndarray:
    """AWQ qzeros int32 [G, N/8] -> uint8 zeros [G, N] in natural order, used as is
    (quant_formats.py:445-446, 455)."""
    return deinterleave_awq(nibbles_i32(qzeros)).astype(np.uint8)


# ----------------------------------------------------------------------------
# Error metrics used by the parity tests
# ----------------------------------------------------------------------------

def max_rel_err(y, ref) -> float:
    """`max|y - ref| / max|ref|` -- the normalized maximum error used for the
    ≤ 2e-3 GEMM tolerance."""
    y = _as_f32(y).astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.abs(ref).max()
    if den == 0:
        return float(np.abs(y - ref).max())
    return float(np.abs(y - ref).max() / den)


def rel_l2(y, ref) -> float:
    """`||y - ref|| / ||ref||` (.dev/test_kernels.py:20-23)."""
    y = _as_f32(y).astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(y - ref) / (np.linalg.norm(ref) + 1e-9))
