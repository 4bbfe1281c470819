"""Pins the CPU oracle (oracle/ref_cpu.py) with checks that do not restate its formulas:
brute force over all byte values, known answers, round trips, closed forms, an fp64
recomputation in the reference kernel's own (blocked integer) form, and library
routines (torch's bf16 cast, silu and round).  A few tests plant a plausible mistake
in a copy of an oracle function and show that the pinning check catches it.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ref_cpu as R

RNG = np.random.default_rng(1234)


# ---------------------------------------------------------------- W4 nibble layout

def _unpack_kat_ok(unpack) -> bool:
    """Known answers for the nibble order: byte 0x8F holds k even = 15, k odd = 8."""
    out = unpack(np.array([[0x8F, 0x07, 0xFF, 0x00]], dtype=np.uint8))
    return (out[:, 0].tolist() == [15, 8] and out[:, 1].tolist() == [7, 0]
            and out[:, 2].tolist() == [15, 15] and out[:, 3].tolist() == [0, 0])


def test_unpack_all_bytes_brute_force():
    b = np.arange(256, dtype=np.uint8).reshape(1, 256)
    nib = R.unpack_w4(b)
    for v in range(256):
        hi, lo = divmod(v, 16)
        assert nib[0, v] == lo and nib[1, v] == hi


def test_unpack_known_answers_and_signed_values():
    assert _unpack_kat_ok(R.unpack_w4)
    # symmetric grid z = 8 (kernels/w4.py:37): 0x8F -> (+7, 0), 0x07 -> (-1, -8)
    s = R.w4_int(np.array([[0x8F, 0x07]], dtype=np.uint8))
    assert s[:, 0].tolist() == [7, 0]
    assert s[:, 1].tolist() == [-1, -8]


def test_unpack_planted_mistake_is_caught():
    def swapped(p):  # high nibble taken as the even k
        out = R.unpack_w4(p)
        return out.reshape(-1, 2, *out.shape[1:])[:, ::-1].reshape(out.shape)
    assert not _unpack_kat_ok(swapped)


def test_pack_unpack_round_trips():
    nib = RNG.integers(0, 16, size=(64, 48), dtype=np.uint8)
    assert np.array_equal(R.unpack_w4(R.pack_pairs(nib)), nib)
    packed = RNG.integers(0, 256, size=(32, 48), dtype=np.uint8)
    assert np.array_equal(R.pack_pairs(R.unpack_w4(packed)), packed)


def test_w4_int_with_zeros_closed_forms():
    packed = RNG.integers(0, 256, size=(64, 32), dtype=np.uint8)   # K = 128
    nib = R.unpack_w4(packed)
    G = 32
    # z == nibble of the group's first row -> that row decodes to 0
    z = nib[::G].copy()
    v = R.w4_int(packed, z, G)
    assert np.all(v[::G] == 0)
    # z constant 8 == absent zeros
    assert np.array_equal(R.w4_int(packed, np.full((4, 32), 8, np.uint8), G), R.w4_int(packed))


# ---------------------------------------------------------------- dequant

def test_dequant_w4_group_indexing_closed_form():
    K, N, G = 256, 16, 64
    nib = np.full((K, N), 9, dtype=np.uint8)              # value +1 everywhere
    packed = R.pack_pairs(nib)
    s = np.stack([np.full(N, 2.0 ** -g, np.float16) for g in range(K // G)])
    d = R.dequant_w4_f32(packed, s)
    for k in range(K):
        assert np.all(d[k] == np.float32(2.0 ** -(k // G)))


def test_dequant_w4_exact_vs_fp64():
    K, N, G = 256, 64, 128
    packed = RNG.integers(0, 256, size=(K // 2, N), dtype=np.uint8)
    s = (np.abs(RNG.normal(0, 0.02, size=(K // G, N))) / 7).astype(np.float16)
    z = RNG.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    d32 = R.dequant_w4_f32(packed, s, z)
    nib = R.unpack_w4(packed).astype(np.float64)
    d64 = (nib - np.repeat(z, G, 0)) * np.repeat(s.astype(np.float64), G, 0)
    assert np.array_equal(d32.astype(np.float64), d64)       # exact in fp32
    one = R.dequant_w4_f32(packed, np.ones_like(s), z)        # s = 1 -> integers
    assert np.array_equal(one, (nib - np.repeat(z, G, 0)).astype(np.float32))


def test_dequant_bf16_scales():
    K, N = 64, 16
    packed = RNG.integers(0, 256, size=(K // 2, N), dtype=np.uint8)
    s32 = np.abs(RNG.normal(0, 0.02, size=(1, N))).astype(np.float32)
    bits = torch.from_numpy(s32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    d = R.dequant_w4_f32(packed, bits)
    s_back = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(d, (R.unpack_w4(packed).astype(np.float32) - 8) * s_back)


def test_dequant_w8_closed_form():
    w = RNG.integers(-127, 128, size=(32, 16), dtype=np.int8)
    s = RNG.random(16).astype(np.float32)
    d = R.dequant_w8_f32(w, s)
    # fp32 scales: one correctly rounded product per element
    assert np.array_equal(d, (w.astype(np.float64) * s.astype(np.float64)).astype(np.float32))
    # fp16 scales (11-bit significand) times int8 is exact in fp32
    s16 = s.astype(np.float16)
    d16 = R.dequant_w8_f32(w, s16)
    assert np.array_equal(d16.astype(np.float64), w.astype(np.float64) * s16.astype(np.float64))


# ---------------------------------------------------------------- GEMM

def test_linear_w8_one_hot_selects_row():
    K, N = 128, 32
    w = RNG.integers(-127, 128, size=(K, N), dtype=np.int8)
    s = (np.abs(RNG.normal(0, 0.02, N)) / 127).astype(np.float16)
    for k in (0, 5, K - 1):
        x = np.zeros((1, K), np.float16)
        x[0, k] = 1
        y = R.linear_w8_ref(x, w, s)
        assert np.array_equal(y[0], w[k].astype(np.float32) * s.astype(np.float32))


def test_linear_w8_vs_fp64_and_transpose_guard():
    M, K, N = 3, 512, 96
    x = RNG.normal(size=(M, K)).astype(np.float16)
    w = RNG.integers(-127, 128, size=(K, N), dtype=np.int8)
    s = (np.abs(RNG.normal(0, 0.02, N)) / 127).astype(np.float16)
    y = R.linear_w8_ref(x, w, s)
    y64 = (x.astype(np.float64) @ w.astype(np.float64)) * s.astype(np.float64)
    assert R.max_rel_err(y, y64) < 1e-6
    # a transposed operand (the config's logical [N, K] weight used unflipped) is far off
    wt = np.ascontiguousarray(w[:N, :N].T)
    assert R.max_rel_err(R.linear_w8_ref(x[:, :N], wt, s), y64[:, :N]) > 0.1


def test_linear_w8_common_scale_factors_out():
    M, K, N = 2, 256, 64
    x = RNG.normal(size=(M, K)).astype(np.float16)
    w = RNG.integers(-127, 128, size=(K, N), dtype=np.int8)
    c = np.float16(0.0078125)
    y = R.linear_w8_ref(x, w, np.full(N, c, np.float16))
    y_int = x.astype(np.float64) @ w.astype(np.float64)
    assert R.max_rel_err(y, y_int * float(c)) < 1e-6


def _gemm_i8_blocked_fp64(a_q, a_s, b, b_s):
    """The reference kernel's form (kernels/gemm.py:40-52): exact integer dot per
    64-block, scaled per block, per-column scale at the end -- in fp64."""
    M, K = a_q.shape
    acc = np.zeros((M, b.shape[1]))
    for kb in range(K // 64):
        sl = slice(64 * kb, 64 * kb + 64)
        i32 = a_q[:, sl].astype(np.int64) @ b[sl].astype(np.int64)
        acc += i32 * a_s[:, kb:kb + 1].astype(np.float64)
    return acc * b_s.astype(np.float64)[None, :]


def test_gemm_i8_vs_blocked_integer_form():
    M, K, N = 5, 512, 128
    a_q = RNG.integers(-127, 127, size=(M, K), dtype=np.int8)
    a_s = (RNG.random((M, K // 64)) * 0.02).astype(np.float32)
    b = RNG.integers(-127, 127, size=(K, N), dtype=np.int8)
    b_s = (RNG.random(N) * 0.002).astype(np.float32)
    y = R.gemm_i8_ref(a_q, a_s, b, b_s)
    assert R.max_rel_err(y, _gemm_i8_blocked_fp64(a_q, a_s, b, b_s)) < 1e-6


def test_gemm_i8_planted_scale_index_mistake_is_caught():
    M, K, N = 2, 256, 32
    a_q = RNG.integers(-127, 127, size=(M, K), dtype=np.int8)
    a_s = (RNG.random((M, K // 64)) * 0.02 + 0.001).astype(np.float32)
    b = RNG.integers(-127, 127, size=(K, N), dtype=np.int8)
    b_s = (RNG.random(N) * 0.002 + 1e-4).astype(np.float32)
    ref = _gemm_i8_blocked_fp64(a_q, a_s, b, b_s)
    # scale per 64 columns of K taken with np.tile instead of repeat
    bad = (a_q.astype(np.float32) * np.tile(a_s, (1, 64))) @ R.dequant_w8_f32(b, b_s)
    assert R.max_rel_err(bad, ref) > 1e-2


def _gemm_w4_blocked_fp64(a_q, a_s, b, b_s, b_z=None):
    """kernels/w4.py:64-104 form: per sub-block of min(G, 64) K values, exact integer
    dot, times (a_s * w_s)."""
    M, K = a_q.shape
    N = b.shape[1]
    G = K // b_s.shape[0]
    sub = min(G, 64)
    q = R.w4_int(b, b_z, G).astype(np.int64)
    s = R.scale_to_f32(b_s).astype(np.float64)
    acc = np.zeros((M, N))
    for k0 in range(0, K, sub):
        i32 = a_q[:, k0:k0 + sub].astype(np.int64) @ q[k0:k0 + sub]
        acc += i32 * (a_s[:, k0 // 64][:, None].astype(np.float64) * s[k0 // G][None, :])
    return acc


@pytest.mark.parametrize("G", [32, 64, 128])
def test_gemm_w4_vs_blocked_integer_form(G):
    M, K, N = 4, 256, 64
    a_q = RNG.integers(-127, 127, size=(M, K), dtype=np.int8)
    a_s = (RNG.random((M, K // 64)) * 0.02).astype(np.float32)
    b = RNG.integers(0, 256, size=(K // 2, N), dtype=np.uint8)
    b_s = (np.abs(RNG.normal(0, 0.02, size=(K // G, N))) / 7).astype(np.float16)
    z = RNG.integers(0, 16, size=(K // G, N), dtype=np.uint8)
    for zz in (None, z):
        y = R.gemm_w4_ref(a_q, a_s, b, b_s, b_z=zz)
        assert R.max_rel_err(y, _gemm_w4_blocked_fp64(a_q, a_s, b, b_s, zz)) < 1e-6


def test_proj3_is_column_concatenation():
    M, K = 3, 128
    a_q = RNG.integers(-127, 127, size=(M, K), dtype=np.int8)
    a_s = (RNG.random((M, K // 64)) * 0.02).astype(np.float32)
    ws = [RNG.integers(-127, 127, size=(K, n), dtype=np.int8) for n in (64, 32, 16)]
    ss = [(RNG.random(w.shape[1]) * 0.002).astype(np.float32) for w in ws]
    y = R.proj3_ref(a_q, a_s, ws[0], ss[0], ws[1], ss[1], ws[2], ss[2])
    assert y.shape == (M, 112)
    assert np.array_equal(y[:, 64:96], R.gemm_i8_ref(a_q, a_s, ws[1], ss[1]))
    y2 = R.proj3_ref(a_q, a_s, ws[0], ss[0], ws[1], ss[1], None, None)
    assert np.array_equal(y2, y[:, :96])


# ---------------------------------------------------------------- epilogue pieces

def test_silu_matches_torch():
    x = RNG.normal(0, 4, size=1000).astype(np.float32)
    ref = torch.nn.functional.silu(torch.from_numpy(x)).numpy()
    assert np.allclose(R.silu(x), ref, rtol=2e-6, atol=1e-7)


def test_round_i8_known_answers():
    v = np.array([0.5, -0.5, 1.5, 2.5, -2.5, 0.4, -0.4, 126.5, 127.49, 128.0, 1000.0, -1000.0,
                  0.49999997], dtype=np.float32)
    want = [1, -1, 2, 3, -3, 0, 0, 127, 127, 127, 127, -127, 1]
    assert R.round_i8(v).tolist() == want


def test_round_i8_planted_half_even_is_caught():
    v = np.array([0.5, 2.5, -2.5], dtype=np.float32)
    assert np.rint(v).astype(np.int8).tolist() != R.round_i8(v).tolist()


def test_bf16_cast_matches_torch():
    x = np.concatenate([RNG.normal(size=4096).astype(np.float32),
                        np.array([np.inf, -np.inf, 0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8,
                                  3.4e38, 1e-40], np.float32)])
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(R.f32_to_bf16_bits(x), t)
    nan = R.f32_to_bf16_bits(np.array([np.nan], np.float32))
    assert np.isnan(R.bf16_bits_to_f32(nan))[0]


def test_quant_groups_invariants():
    h = RNG.normal(size=(4, 256)).astype(np.float32)
    h[1, 64:128] = 0.0
    q, s = R.quant_groups(h)
    assert q.dtype == np.int8 and s.shape == (4, 4)
    assert np.abs(q.astype(np.int32)).max() <= 127
    assert s[1, 1] == np.float32(1e-8) and np.all(q[1, 64:128] == 0)
    g = np.abs(q.astype(np.int32)).reshape(4, 4, 64).max(axis=2)
    assert np.all(g[s > 1e-8] == 127)
    err = np.abs(q.astype(np.float32) * np.repeat(s, 64, 1) - h)
    assert np.all(err <= 0.5 * np.repeat(s, 64, 1) * (1 + 1e-5))


def test_gate_up_quant_is_the_unfused_composition():
    M, K, N = 3, 128, 128
    a_q = RNG.integers(-127, 127, size=(M, K), dtype=np.int8)
    a_s = (RNG.random((M, K // 64)) * 0.02).astype(np.float32)
    wg = RNG.integers(-127, 127, size=(K, N), dtype=np.int8)
    wu = RNG.integers(-127, 127, size=(K, N), dtype=np.int8)
    sg = (RNG.random(N) * 0.002).astype(np.float32)
    su = (RNG.random(N) * 0.002).astype(np.float32)
    h = R.mlp_gate_up_ref(a_q, a_s, wg, sg, wu, su)
    g = R.gemm_i8_ref(a_q, a_s, wg, sg)
    u = R.gemm_i8_ref(a_q, a_s, wu, su)
    ref = torch.nn.functional.silu(torch.from_numpy(g)).numpy() * u
    assert np.allclose(h, ref, rtol=1e-5, atol=1e-7)
    q, s = R.mlp_gate_up_quant_ref(a_q, a_s, wg, sg, wu, su)
    q2, s2 = R.quant_groups(R.round_bf16(h))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


# ---------------------------------------------------------------- load-time producers

def test_requant_w4_sym_recovers_exact_grid():
    K, N, G = 64, 16, 32
    q = RNG.integers(1, 16, size=(K, N)).astype(np.uint8)   # |q - 8| <= 7 (amax / 7 grid)
    q[0], q[G] = 15, 1                        # each group reaches |q - 8| = 7
    s = np.full((K // G, N), 2.0 ** -7, np.float32)
    w = (q.astype(np.float32) - 8) * np.repeat(s, G, 0)
    packed, sbits = R.requant_w4_sym(w, G)
    assert np.array_equal(packed, R.pack_pairs(q))
    assert np.array_equal(R.bf16_bits_to_f32(sbits), s)


def test_requant_rounding_matches_torch_round():
    w = np.array([[0.5], [1.5], [2.5], [-2.5], [127.0]], dtype=np.float32) * np.float32(1 / 127)
    q, sc = R.requant_w8_row(w)
    ref = torch.clamp(torch.round(torch.from_numpy(w) / torch.from_numpy(sc)[None, :]), -127, 127)
    assert np.array_equal(q.astype(np.float32), ref.numpy())


# ---------------------------------------------------------------- external int4 formats
#
# Anchors: the bit layout the reference's decoders state (quant_formats.py:199-220:
# straight nibble order inside an int32 word, AWQ's reverse order [0, 4, 1, 5, 2, 6,
# 3, 7]) and the pack order of AutoAWQ's published packer, [0, 2, 4, 6, 1, 3, 5, 7]
# (AutoAWQ is not part of the reference checkout; its order is the inverse of the
# reference's REV, which the round trips below check).

AWQ_PACK_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]


def _words_from_nibbles(nib8):
    """[..., 8] nibbles -> int32 words, nibble p at bits 4p..4p+3."""
    w = np.zeros(nib8.shape[:-1], dtype=np.int64)
    for p in range(8):
        w |= nib8[..., p].astype(np.int64) << (4 * p)
    return w.astype(np.uint32).view(np.int32)


def _gptq_words(nib):
    """natural nibbles [K, N] -> GPTQ qweight [K/8, N]: word w holds rows 8w..8w+7."""
    K, N = nib.shape
    return _words_from_nibbles(nib.reshape(K // 8, 8, N).transpose(0, 2, 1))


def _awq_words(nib, order=AWQ_PACK_ORDER):
    """natural nibbles [R, N] -> AWQ words [R, N/8]: nibble p of word c = column 8c + order[p]."""
    R_, N = nib.shape
    g = nib.reshape(R_, N // 8, 8)
    return _words_from_nibbles(g[..., order])


def test_nibbles_known_answers():
    words = np.array([[0x76543210, np.uint32(0xFEDCBA98).view(np.int32), -1, 0]], dtype=np.int32)
    n = R.nibbles_i32(words)
    assert n.tolist() == [list(range(8)) + list(range(8, 16)) + [15] * 8 + [0] * 8]


def test_gptq_repack_is_the_words_bytes():
    qw = RNG.integers(-2 ** 31, 2 ** 31, size=(16, 24), dtype=np.int64).astype(np.int32)
    p = R.gptq_w4_to_engine(qw)
    u = qw.view(np.uint32)
    for t in range(4):
        assert np.array_equal(p[t::4], ((u >> (8 * t)) & 0xFF).astype(np.uint8))


def test_gptq_repack_round_trip():
    nib = RNG.integers(0, 16, size=(64, 40), dtype=np.uint8)
    assert np.array_equal(R.unpack_w4(R.gptq_w4_to_engine(_gptq_words(nib))), nib)


def test_awq_repack_round_trip_with_published_pack_order():
    nib = RNG.integers(0, 16, size=(32, 64), dtype=np.uint8)
    assert np.array_equal(R.unpack_w4(R.awq_w4_to_engine(_awq_words(nib))), nib)
    # the order is an inverse pair: words packed in straight order do not round-trip
    assert not np.array_equal(R.unpack_w4(R.awq_w4_to_engine(_awq_words(nib, list(range(8))))), nib)


def test_zero_unpack_orders():
    z = RNG.integers(0, 16, size=(4, 32), dtype=np.uint8)
    assert np.array_equal(R.gptq_zeros(_awq_words(z, list(range(8)))), z + 1)
    assert np.array_equal(R.gptq_zeros(_awq_words(z, list(range(8))), plus_one=False), z)
    assert np.array_equal(R.awq_zeros(_awq_words(z)), z)


def _ct_words(nib):
    """nibbles [N, K] (one output feature per row) -> compressed-tensors words [N, K/8]:
    nibble j of word w = element k = 8w + j of the row (straight order)."""
    N, K = nib.shape
    return _words_from_nibbles(nib.reshape(N, K // 8, 8))


def test_ct_repack_known_answer_and_byte_transpose():
    """Word 0x76543210 holds k = 0..7 = 0..7: the engine pair bytes of rows 0..3 are
    0x10, 0x32, 0x54, 0x76, the word's own bytes.  In general the packed matrix is the
    byte transpose of the [N, 4W] byte view of the words."""
    w = np.array([[0x76543210]], dtype=np.int32)
    assert R.ct_w4_to_engine(w)[:, 0].tolist() == [0x10, 0x32, 0x54, 0x76]
    qw = RNG.integers(-2 ** 31, 2 ** 31, size=(24, 10), dtype=np.int64).astype(np.int32)
    assert np.array_equal(R.ct_w4_to_engine(qw), qw.view(np.uint8).reshape(24, 40).T)
    assert np.array_equal(R.ct_w4_to_engine(qw, K=62), qw.view(np.uint8).reshape(24, 40).T[:31])


def test_ct_repack_round_trip_and_planted_mistake():
    nib = RNG.integers(0, 16, size=(40, 64), dtype=np.uint8)
    assert np.array_equal(R.unpack_w4(R.ct_w4_to_engine(_ct_words(nib))), nib.T)
    # a decoder that put the odd K in the low nibble would not round-trip
    swapped = R.ct_w4_to_engine(_ct_words(nib))
    swapped = ((swapped >> 4) | (swapped << 4)).astype(np.uint8)
    assert not np.array_equal(R.unpack_w4(swapped), nib.T)


def test_ct_scale_transpose():
    s = RNG.standard_normal((6, 4)).astype(np.float32)
    assert np.array_equal(R.ct_scale_to_engine(s), s.T)


# ---------------------------------------------------------------- activation producers

def _exp_no_lo(x):
    """exp_f32 with the low part of ln2 dropped (a planted mistake)."""
    x = np.asarray(x, dtype=np.float32)
    n = np.rint(x * R.LOG2E_F32).astype(np.float32)
    r = (x - n * R.LN2_HI_F32).astype(np.float32)
    p = np.full_like(r, R.EXP_POLY_F32[0])
    for c in R.EXP_POLY_F32[1:]:
        p = ((p * r).astype(np.float32) + c).astype(np.float32)
    return np.ldexp(p, n.astype(np.int32)).astype(np.float32)


def _exp_rel_err(f, x):
    y = f(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    return float((np.abs(y - ref) / ref).max())


def test_exp_f32_against_fp64():
    """The producers' exp is within 2 ulp (2^-22 relative) of exp in fp64 over its whole
    finite range; dropping the low part of ln2 breaks that bound."""
    x = np.concatenate([np.linspace(-87.0, 88.0, 400_001, dtype=np.float32),
                        (RNG.standard_normal(200_000) * 8).astype(np.float32)])
    x = x[(x >= -87.0) & (x <= 88.0)]
    assert _exp_rel_err(R.exp_f32, x) <= 2.0 ** -22
    assert _exp_rel_err(_exp_no_lo, x) > 2.0 ** -22
    assert R.exp_f32(np.float32(0.0)) == 1.0
    e = R.exp_f32(np.array([88.5, 1e30, -87.5, -1e30], dtype=np.float32))
    assert np.isinf(e[0]) and np.isinf(e[1]) and e[2] == 0.0 and e[3] == 0.0
    # sigmoid / silu against fp64 (outside the saturated ends)
    z = np.linspace(-60.0, 60.0, 100_001, dtype=np.float32)
    sg = 1.0 / (1.0 + np.exp(-z.astype(np.float64)))
    assert np.abs(R.sigmoid_f32(z) - sg).max() <= 4 * 2.0 ** -24
    assert np.abs(R.silu_f32(z) - z * sg).max() <= 60 * 4 * 2.0 ** -24


def test_sumsq_lanes_sums_every_square():
    """With small integers every partial sum is exact whatever the order, so the fixed
    lane order must give the exact sum of squares; random rows stay within the fp32
    bound of the fp64 sum."""
    for L, lanes in ((2048, 64), (128, 16), (8, 64), (520, 64)):
        xi = RNG.integers(-100, 101, size=(3, L))
        ss = R.sumsq_lanes(xi.astype(np.float32), lanes)
        assert (ss == (xi.astype(np.int64) ** 2).sum(axis=1)).all()
    x = RNG.standard_normal((4, 4096)).astype(np.float32)
    ref = (x.astype(np.float64) ** 2).sum(axis=1)
    assert (np.abs(R.sumsq_lanes(x, 64) - ref) <= 4096 * 2.0 ** -24 * ref).all()


def _bf16(a):
    return R.round_bf16(np.asarray(a, dtype=np.float32))


def _codes_vs_fp64(q, s, y64, tie_margin=1e-3):
    """Whether the codes equal the fp64 computation away from rounding ties and differ
    by at most 1 near them, and the scales agree to a few fp32 ulp."""
    M, K = y64.shape
    g = y64.reshape(M, K // 64, 64)
    s64 = np.maximum(np.abs(g).max(axis=2) / 127.0, 1e-8)
    if not np.allclose(s, s64, rtol=4 * 2.0 ** -24, atol=0):
        return False
    v = g / s64[:, :, None]
    q64 = np.clip(np.trunc(v + np.where(v >= 0, 0.5, -0.5)), -127, 127).reshape(M, K)
    qi = q.astype(np.int64)
    far = (np.abs(np.abs(v - np.trunc(v)) - 0.5) > tie_margin).reshape(M, K)
    return bool(np.abs(qi - q64).max() <= 1 and (qi[far] == q64[far]).all())


def _rms_y64(x, w, eps, one_plus):
    x64 = x.astype(np.float64)
    w64 = w.astype(np.float64) + (1.0 if one_plus else 0.0)
    r = 1.0 / np.sqrt((x64 ** 2).mean(axis=1) + eps)
    return x64 * r[:, None] * w64[None, :]


def test_rmsnorm_quant_against_fp64_and_planted_mistakes():
    """rmsnorm_quant codes equal an fp64 RMSNorm + quant away from rounding ties; a
    variance over K - 1 and a forgotten `w + 1` both change codes."""
    M, K = 6, 2048
    x = _bf16(RNG.standard_normal((M, K)) * 3)
    w = _bf16(RNG.standard_normal(K) * 0.1)
    for one_plus in (True, False):
        q, s = R.rmsnorm_quant_ref(x, w, 1e-6, one_plus)
        assert _codes_vs_fp64(q, s, _rms_y64(x, w, 1e-6, one_plus))
    q, s = R.rmsnorm_quant_ref(x, w, 1e-6, True)
    wrong_n = _rms_y64(x, w, 1e-6, True) * np.sqrt((K - 1) / K)  # var = sum / (K - 1)
    qn = np.clip(np.trunc(wrong_n / np.repeat(s, 64, axis=1) + 0.5 * np.sign(wrong_n)), -127, 127)
    assert not (qn == q).all()
    assert not _codes_vs_fp64(q, s, _rms_y64(x, w, 1e-6, False))


def test_rmsnorm_quant_closed_forms():
    """A constant row with a zero weight and one_plus normalizes to +-1 everywhere: every
    code is +-127 and every scale (1/sqrt(1 + eps/c^2))/127; a zero row gives the
    scale floor 1e-8 and zero codes."""
    K = 256
    x = np.stack([np.full(K, 3.0), np.full(K, -0.5), np.zeros(K)]).astype(np.float32)
    q, s = R.rmsnorm_quant_ref(x, np.zeros(K, np.float32), 1e-6, True)
    assert (q[0] == 127).all() and (q[1] == -127).all() and (q[2] == 0).all()
    assert np.allclose(s[0], 1.0 / np.sqrt(1 + 1e-6 / 9) / 127, rtol=1e-6)
    assert (s[2] == np.float32(1e-8)).all()


def test_gate_mul_head_layout_and_fp64():
    """With gates +100 in the second half of every head and -100 in the first,
    sigmoid is exactly 1 on the gates the kernel must read, so y == a and the codes are
    quant_groups(a); reading the first half instead gives zeros.  Random gates agree
    with fp64 away from ties."""
    M, N, hd = 3, 512, 64
    a = _bf16(RNG.standard_normal((M, N)))
    g = np.full((M, N // hd, 2 * hd), -100.0, dtype=np.float32)
    g[:, :, hd:] = 100.0
    g = g.reshape(M, 2 * N)
    q, s = R.gate_mul_quant_ref(a, g, hd)
    qa, sa = R.quant_groups(a)
    assert (q == qa).all() and (s == sa).all()
    first_half = np.repeat(np.arange(N // hd) * 2 * hd, hd) + np.tile(np.arange(hd), N // hd)
    y_wrong = a * R.sigmoid_f32(g[:, first_half])
    assert not (R.quant_groups(y_wrong)[0] == q).all()
    g = _bf16(RNG.standard_normal((M, 2 * N)) * 2)
    q, s = R.gate_mul_quant_ref(a, g, hd)
    gv = g[:, R.gate_cols(N, hd)].astype(np.float64)
    assert _codes_vs_fp64(q, s, a.astype(np.float64) / (1.0 + np.exp(-gv)))


def test_norm_gated_quant_per_head_and_fp64():
    """Per-head norm: with eps = 0, scaling one head's v by 4 leaves every code and
    scale unchanged (power-of-two scaling is exact through the sum, the division and
    the sqrt); a norm over the whole row would not.  Random inputs agree with fp64
    (bf16 rounding before the quant: codes within 1, scales within a bf16 step)."""
    T, hd, NV = 3, 128, 4
    N = hd * NV
    v = _bf16(RNG.standard_normal((T, N)))
    z = _bf16(RNG.standard_normal((T, N)) * 2)
    w = _bf16(RNG.standard_normal(hd) * 0.5 + 1.0)
    q, s = R.norm_gated_quant_ref(v, z, w, 0.0)
    v2 = v.copy()
    v2[:, hd:2 * hd] *= 4
    q2, s2 = R.norm_gated_quant_ref(v2, z, w, 0.0)
    assert (q2 == q).all() and (s2 == s).all()

    def whole_row(v_):
        r = R.rms_inv(R.sumsq_lanes(v_, 64), N, 0.0)
        y = (v_ * r[:, None]).astype(np.float32) * np.tile(w, NV)[None, :]
        return R.quant_groups(R.round_bf16((y * R.silu_f32(z)).astype(np.float32)))[0]
    assert not (whole_row(v2) == whole_row(v)).all()
    q, s = R.norm_gated_quant_ref(v, z, w, 1e-6)
    v64 = v.astype(np.float64).reshape(T, NV, hd)
    r = 1.0 / np.sqrt((v64 ** 2).mean(axis=2) + 1e-6)
    z64 = z.astype(np.float64)
    y64 = (v64 * r[:, :, None]).reshape(T, N) * np.tile(w, NV) * (z64 / (1.0 + np.exp(-z64)))
    y64 = _bf16(y64).astype(np.float64)  # the reference's bf16 round trip (kernels/norm.py:116)
    g = y64.reshape(T, N // 64, 64)
    s64 = np.maximum(np.abs(g).max(axis=2) / 127.0, 1e-8)
    assert np.allclose(s, s64, rtol=2.0 ** -8, atol=0)
    v_ = g / s64[:, :, None]
    q64 = np.clip(np.trunc(v_ + np.where(v_ >= 0, 0.5, -0.5)), -127, 127).reshape(T, N)
    assert np.abs(q.astype(np.int64) - q64).max() <= 1
    assert (q.astype(np.int64) != q64).mean() < 0.005
