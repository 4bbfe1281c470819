"""GPU parity of the layout kernels and the A16 (fp16-activation) linears against the
CPU oracle, on the workload shapes (decode rows M <= 4 and mid-range M).

Bar: unpack / dequant bit-exact; GEMM |y - y_ref| <= 2e-3 * max|y_ref| against the
oracle's fp32 result (y_ref = dequantize, then fp32 matmul), plus half an ulp of the
16-bit output type for the final rounding (helpers.assert_out_close).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

pytestmark = pytest.mark.gpu



def _k():
    from qwen35_amd.kernels import layout, linear
    return layout, linear


# ---------------------------------------------------------------- layout, bit-exact

@pytest.mark.parametrize("K,N", [(256, 16), (2048, 512), (4096, 1040)])
def test_w4_unpack_bit_exact(K, N):
    layout, _ = _k()
    packed, _, _ = H.w4(K, N, seed=11)
    nib = layout.w4_unpack(packed.cuda()).cpu().numpy()
    assert np.array_equal(nib, R.unpack_w4(packed.numpy()))


def test_w4_unpack_all_bytes():
    layout, _ = _k()
    packed = torch.arange(256, dtype=torch.int32).to(torch.uint8).reshape(1, 256).repeat(2, 1)
    nib = layout.w4_unpack(packed.cuda()).cpu().numpy()
    assert np.array_equal(nib, R.unpack_w4(packed.numpy()))


@pytest.mark.parametrize("group,zeros,sdt", [(128, "none", torch.float16), (32, "random", torch.float16),
                                             (64, "random", torch.bfloat16), (128, "eight", torch.float32)])
def test_w4_dequant_bit_exact(group, zeros, sdt):
    layout, _ = _k()
    K, N = 1024, 256
    packed, s, z = H.w4(K, N, seed=12, group=group, zeros=zeros)
    s = s.to(sdt)
    d = layout.w4_dequant_f32(packed.cuda(), s.cuda(), None if z is None else z.cuda()).cpu().numpy()
    ref = R.dequant_w4_f32(packed.numpy(), H.np_(s), None if z is None else z.numpy())
    assert np.array_equal(d, ref)


@pytest.mark.parametrize("sdt", [torch.float16, torch.float32])
def test_w8_dequant_bit_exact(sdt):
    layout, _ = _k()
    w, s = H.w8(512, 256, seed=13)
    s = s.to(sdt)
    d = layout.w8_dequant_f32(w.cuda(), s.cuda()).cpu().numpy()
    assert np.array_equal(d, R.dequant_w8_f32(w.numpy(), H.np_(s)))


def _requant_input(K, N, seed, grid_amax, group):
    """Normal weights plus the edge cases of the producers: an all-zero column block
    (amax clamped at 1e-8), a column holding -0.0, and a column whose blocks hit an
    exact scale (amax = grid_amax * 2^-4, so sc = 2^-4) with every half-step tie."""
    w = (torch.randn((K, N), generator=H.gen(seed)) * 0.02).numpy()
    w[:group, 0] = 0.0
    w[:, 1] = -0.0
    rows = np.arange(K)
    ties = ((rows % (2 * grid_amax + 1)) - grid_amax + 0.5) / 16.0
    w[:, 2] = np.clip(ties, -grid_amax / 16.0, grid_amax / 16.0)
    w[::group, 2] = grid_amax / 16.0  # every block reaches the exact amax
    return torch.from_numpy(w.astype(np.float32))


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("K,N", [(256, 40), (2048, 1040)])
def test_requant_w4_sym_bit_exact(group, K, N):
    """GPU requant_w4_sym (quant_formats.py:253-267) equals the oracle bit for bit:
    packed codes and bf16 scales, ties rounded half to even."""
    layout, _ = _k()
    w = _requant_input(K, N, seed=14, grid_amax=7, group=group)
    packed, scale = layout.requant_w4_sym(w.cuda(), group)
    assert packed.dtype == torch.uint8 and scale.dtype == torch.bfloat16
    ref_p, ref_s = R.requant_w4_sym(w.numpy(), group)
    assert np.array_equal(packed.cpu().numpy(), ref_p)
    assert np.array_equal(scale.cpu().view(torch.int16).numpy().view(np.uint16), ref_s)


@pytest.mark.parametrize("K,N", [(64, 24), (2048, 1040), (6144, 2048)])
def test_requant_w8_row_bit_exact(K, N):
    """GPU requant_w8_row (quant_formats.py:270-275) equals the oracle bit for bit."""
    layout, _ = _k()
    w = _requant_input(K, N, seed=15, grid_amax=127, group=K)
    q, sc = layout.requant_w8_row(w.cuda())
    assert q.dtype == torch.int8 and sc.dtype == torch.float32
    ref_q, ref_sc = R.requant_w8_row(w.numpy())
    assert np.array_equal(q.cpu().numpy(), ref_q)
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), ref_sc.view(np.uint32))


def test_requant_round_trip_full_size():
    """At a full layer size: requantize on the GPU, dequantize with the GEMM layout
    kernels, and every weight is back within half a step of its scale (the codes'
    rounding bound), for W8 per column and W4 g32."""
    layout, _ = _k()
    K, N = 4096, 6144
    w = (torch.randn((K, N), generator=H.gen(16)) * 0.02).cuda()
    q, sc = layout.requant_w8_row(w)
    err = (layout.w8_dequant_f32(q, sc) - w).abs()
    assert bool((err <= sc[None, :] * 0.5 + w.abs() * 2.0 ** -22).all())
    packed, s4 = layout.requant_w4_sym(w, 32)
    d4 = layout.w4_dequant_f32(packed, s4)
    s_rows = s4.float().repeat_interleave(32, dim=0)
    # the codes were rounded with the fp32 scale; bf16 storage of the scale adds up to
    # 2^-9 relative per step of 8
    assert bool(((d4 - w).abs() <= s_rows * (0.5 + 8 * 2.0 ** -8) + w.abs() * 2.0 ** -22).all())


def _rand_words(rows, cols, seed):
    g = np.random.default_rng(seed)
    return torch.from_numpy(g.integers(-2 ** 31, 2 ** 31, size=(rows, cols), dtype=np.int64).astype(np.int32))


@pytest.mark.parametrize("K,N", [(64, 24), (4096, 1040), (12288, 4096)])
def test_w4_repack_gptq_bit_exact(K, N):
    """GPTQ qweight int32 [K/8, N] -> engine packed [K/2, N] equals the oracle bit for bit."""
    layout, _ = _k()
    qw = _rand_words(K // 8, N, seed=17)
    p = layout.gptq_w4_to_engine(qw.cuda())
    assert p.shape == (K // 2, N) and p.dtype == torch.uint8
    assert np.array_equal(p.cpu().numpy(), R.gptq_w4_to_engine(qw.numpy()))


@pytest.mark.parametrize("K,N", [(2, 8), (4096, 1040), (4096, 12288)])
def test_w4_repack_awq_bit_exact(K, N):
    """AWQ qweight int32 [K, N/8] (AWQ nibble order) -> engine packed [K/2, N]."""
    layout, _ = _k()
    qw = _rand_words(K, N // 8, seed=18)
    p = layout.awq_w4_to_engine(qw.cuda())
    assert p.shape == (K // 2, N) and p.dtype == torch.uint8
    assert np.array_equal(p.cpu().numpy(), R.awq_w4_to_engine(qw.numpy()))


def test_w4_zeros_unpack_bit_exact():
    layout, _ = _k()
    qz = _rand_words(32, 128, seed=19)
    assert np.array_equal(layout.gptq_zeros(qz.cuda()).cpu().numpy(), R.gptq_zeros(qz.numpy()))
    assert np.array_equal(layout.gptq_zeros(qz.cuda(), plus_one=False).cpu().numpy(),
                          R.gptq_zeros(qz.numpy(), plus_one=False))
    assert np.array_equal(layout.awq_zeros(qz.cuda()).cpu().numpy(), R.awq_zeros(qz.numpy()))


def test_repacked_gptq_feeds_the_gemm():
    """A GPTQ-packed symmetric checkpoint, repacked on the GPU, runs through the W4
    decode GEMM and matches the oracle's dequantize + fp32 matmul of the same codes."""
    layout, _ = _k()
    K, N = 2048, 1024
    qw = _rand_words(K // 8, N, seed=20)
    packed = layout.gptq_w4_to_engine(qw.cuda())
    s = (torch.rand((K // 128, N), generator=H.gen(21)) * 1e-3).to(torch.float16)
    x = H.act_f16(4, K, seed=22)
    y = _run_w4(x, packed.cpu(), s, None)
    ref = H.linear_w4_ref_cols(x, torch.from_numpy(R.gptq_w4_to_engine(qw.numpy())), s, None, np.arange(N))
    H.assert_out_close(y, ref)


@pytest.mark.parametrize("N,W,K", [(48, 25, 200), (64, 8, 62), (6144, 256, 2048), (4096, 1536, 12288)])
def test_w4_repack_ct_bit_exact(N, W, K):
    """compressed-tensors weight_packed int32 [N, W] -> engine packed [K/2, N] equals the
    oracle bit for bit, partial tiles and a K short of 8 W included."""
    layout, _ = _k()
    qw = _rand_words(N, W, seed=23)
    p = layout.ct_w4_to_engine(qw.cuda(), K=K)
    assert p.shape == (K // 2, N) and p.dtype == torch.uint8
    assert np.array_equal(p.cpu().numpy(), R.ct_w4_to_engine(qw.numpy(), K=K))


def test_repacked_ct_feeds_the_gemm():
    """A compressed-tensors symmetric int4 checkpoint (zero point 8, group 128),
    decoded on the GPU, runs through the W4 GEMMs: decode (M = 4) and prefill tiles
    (M = 96), against the oracle's dequantize + fp32 matmul of the same codes."""
    layout, _ = _k()
    K, N = 2048, 1024
    qw = _rand_words(N, K // 8, seed=24)
    s_ct = (torch.rand((N, K // 128), generator=H.gen(25)) * 1e-3).to(torch.bfloat16)
    packed, s = layout.ct_w4_to_engine(qw.cuda(), K=K, weight_scale=s_ct.cuda())
    assert torch.equal(s.cpu(), s_ct.t())
    ref_packed = torch.from_numpy(R.ct_w4_to_engine(qw.numpy(), K=K))
    for M in (4, 96):
        x = H.act_f16(M, K, seed=26 + M)
        y = _run_w4(x, packed.cpu(), s.cpu(), None)
        H.assert_out_close(y, H.linear_w4_ref_cols(x, ref_packed, s_ct.t().contiguous(), None, np.arange(N)))


def test_repack_bad_arguments_raise():
    layout, _ = _k()
    with pytest.raises(ValueError):
        layout.awq_w4_to_engine(torch.zeros((3, 2), dtype=torch.int32, device="cuda"))  # odd K
    with pytest.raises(ValueError):
        layout.gptq_w4_to_engine(torch.zeros((4, 8), dtype=torch.int64, device="cuda"))  # not int32


# ---------------------------------------------------------------- A16 linears

def _run_w8(x, w, s, out_dtype=torch.float16, residual=None):
    _, linear = _k()
    M, N = x.shape[0], w.shape[1]
    out = torch.empty((M, N), dtype=out_dtype, device="cuda")
    linear.linear_w8(x.cuda(), w.cuda(), s.cuda(), out,
                     residual=None if residual is None else residual.cuda())
    torch.cuda.synchronize()
    return out


def _run_w4(x, packed, s, z, out_dtype=torch.float16, residual=None):
    _, linear = _k()
    M, N = x.shape[0], packed.shape[1]
    out = torch.empty((M, N), dtype=out_dtype, device="cuda")
    linear.linear_w4(x.cuda(), packed.cuda(), s.cuda(), out,
                     w_zero=None if z is None else z.cuda(),
                     residual=None if residual is None else residual.cuda())
    torch.cuda.synchronize()
    return out


def test_linear_w8_plumbing_case():
    """M=1, K=2048, N=6144 int8 per-channel, fp16 out (the single-linear CPU case)."""
    x = H.act_f16(1, 2048, seed=0)
    w, s = H.w8(2048, 6144, seed=0)
    y = _run_w8(x, w, s)
    ref = H.linear_w8_ref_cols(x, w, s, np.arange(6144))
    H.assert_out_close(y, ref)
    assert R.rel_l2(H.to_f32(y), ref) < 1e-3


DECODE_SHAPES = [(2048, 2048), (2048, 512), (2048, 6144), (6144, 2048), (2048, 4096), (4096, 2048)]


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("K,N", DECODE_SHAPES)
def test_linear_w8_decode_shapes(M, K, N):
    x = H.act_f16(M, K, seed=100 + M)
    w, s = H.w8(K, N, seed=K + N)
    y = _run_w8(x, w, s)
    ref = H.linear_w8_ref_cols(x, w, s, np.arange(N))
    H.assert_out_close(y, ref)


@pytest.mark.parametrize("M", [1, 4])
def test_linear_w8_vocab_head(M):
    K, N = 2048, 248320
    x = H.act_f16(M, K, seed=7)
    w, s = H.w8(K, N, seed=8)
    y = _run_w8(x, w, s)
    cols = H.sample_cols(N, 8192)
    ref = H.linear_w8_ref_cols(x, w, s, cols)
    H.assert_out_close(y.cpu()[:, cols], ref)


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("K,N", DECODE_SHAPES)
def test_linear_w4_decode_shapes(M, K, N):
    x = H.act_f16(M, K, seed=200 + M)
    packed, s, z = H.w4(K, N, seed=K * 3 + N)
    y = _run_w4(x, packed, s, z)
    ref = H.linear_w4_ref_cols(x, packed, s, z, np.arange(N))
    H.assert_out_close(y, ref)


def test_linear_w4_explicit_zero_eight_is_identical():
    x = H.act_f16(4, 2048, seed=21)
    packed, s, _ = H.w4(2048, 2048, seed=22)
    z8 = torch.full((2048 // 128, 2048), 8, dtype=torch.uint8)
    y0 = _run_w4(x, packed, s, None)
    y1 = _run_w4(x, packed, s, z8)
    assert torch.equal(y0, y1)


@pytest.mark.parametrize("group", [32, 64, 128, 256])
@pytest.mark.parametrize("zeros", ["none", "random"])
def test_linear_w4_groups_and_zeros(group, zeros):
    M, K, N = 3, 1024, 768
    x = H.act_f16(M, K, seed=31)
    packed, s, z = H.w4(K, N, seed=32, group=group, zeros=zeros)
    y = _run_w4(x, packed, s, z)
    ref = H.linear_w4_ref_cols(x, packed, s, z, np.arange(N))
    H.assert_out_close(y, ref)


@pytest.mark.parametrize("M", [1, 4])
def test_linear_w4_vocab_head(M):
    K, N = 2048, 248320
    x = H.act_f16(M, K, seed=41)
    packed, s, z = H.w4(K, N, seed=42)
    y = _run_w4(x, packed, s, z)
    cols = H.sample_cols(N, 8192)
    ref = H.linear_w4_ref_cols(x, packed, s, z, cols)
    H.assert_out_close(y.cpu()[:, cols], ref)


@pytest.mark.parametrize("M", [5, 16, 17, 40])
def test_linear_mid_range_rows(M):
    K, N = 2048, 1024
    x = H.act_f16(M, K, seed=50 + M)
    w, s = H.w8(K, N, seed=51)
    y = _run_w8(x, w, s)
    H.assert_out_close(y, H.linear_w8_ref_cols(x, w, s, np.arange(N)))
    packed, s4, z = H.w4(K, N, seed=52, zeros="random")
    y4 = _run_w4(x, packed, s4, z)
    H.assert_out_close(y4, H.linear_w4_ref_cols(x, packed, s4, z, np.arange(N)))


def test_linear_residual_and_bf16_out():
    M, K, N = 4, 2048, 2048
    x = H.act_f16(M, K, seed=61)
    w, s = H.w8(K, N, seed=62)
    res = torch.randn((M, N), generator=H.gen(63)).to(torch.bfloat16)
    y = _run_w8(x, w, s, out_dtype=torch.bfloat16, residual=res)
    ref = H.linear_w8_ref_cols(x, w, s, np.arange(N), residual=res)
    H.assert_out_close(y, ref)


@pytest.mark.parametrize("K,N", [(2048, 6144), (6144, 2048)])
def test_rows_independent_of_batch(K, N):
    """Row m of an M=16 call is bit-identical to the same row run alone (every plan
    choice depends on K and N only): one-pass tiles (K=2048) and split-K (K=6144)."""
    x = H.act_f16(16, K, seed=71)
    w, s = H.w8(K, N, seed=72)
    packed, s4, _ = H.w4(K, N, seed=73)
    y = _run_w8(x, w, s)
    y4 = _run_w4(x, packed, s4, None)
    for m in (0, 5, 15):
        assert torch.equal(_run_w8(x[m:m + 1], w, s)[0], y[m])
        assert torch.equal(_run_w4(x[m:m + 1], packed, s4, None)[0], y4[m])


@pytest.mark.parametrize("plan", ["4,8,0", "8,8,0", "8,4,0", "16,4,0"])
@pytest.mark.parametrize("K,N", [(2048, 2048), (6144, 1024)])
def test_decode_forced_plans(plan, K, N, monkeypatch):
    """Every decode plan family on the same shapes, whatever the default picks:
    one-pass 64-column tiles (4 columns per lane), split-K over 128- and 256-column
    tiles.  Oracle parity for W8 (+ residual) and W4 with zeros, M = 1, 4, 16, and
    rows independent of M within the plan."""
    monkeypatch.setenv("QLIN_SKINNY_PLAN", plan)
    x = H.act_f16(16, K, seed=90)
    w, s = H.w8(K, N, seed=91)
    packed, s4, z = H.w4(K, N, seed=92, zeros="random")
    res = torch.randn((16, N), generator=H.gen(93)).to(torch.float16)
    for M in (1, 4, 16):
        y = _run_w8(x[:M], w, s, residual=res[:M])
        H.assert_out_close(y, H.linear_w8_ref_cols(x[:M], w, s, np.arange(N), residual=res[:M]))
        y4 = _run_w4(x[:M], packed, s4, z)
        H.assert_out_close(y4, H.linear_w4_ref_cols(x[:M], packed, s4, z, np.arange(N)))
        if M == 16:
            assert torch.equal(_run_w8(x[3:4], w, s, residual=res[3:4])[0], y[3])
            assert torch.equal(_run_w4(x[3:4], packed, s4, z)[0], y4[3])


@pytest.mark.parametrize("upw", [1, 2, 3, 5, 8, 9, 12, 13])
@pytest.mark.parametrize("K,N", [(2048, 1024), (6144, 512)])
def test_decode_w8_wave_depths(upw, K, N, monkeypatch):
    """fp16 W8 waves issue each 32-row step's loads once: short K ranges test every
    load, long ones run a straight-line main loop and test only their last steps.
    Forced K depths of 1-13 steps per wave (the last wave of a tile shorter, some
    waves empty) cover both paths and the boundary between them, split-K or not;
    oracle parity with a residual at M = 1, 4, 16, rows independent of M."""
    monkeypatch.setenv("QLIN_SKINNY_PLAN", f"8,8,{upw}")
    x = H.act_f16(16, K, seed=94)
    w, s = H.w8(K, N, seed=95)
    res = torch.randn((16, N), generator=H.gen(96)).to(torch.float16)
    for M in (1, 4, 16):
        y = _run_w8(x[:M], w, s, residual=res[:M])
        H.assert_out_close(y, H.linear_w8_ref_cols(x[:M], w, s, np.arange(N), residual=res[:M]))
        if M == 16:
            assert torch.equal(_run_w8(x[5:6], w, s, residual=res[5:6])[0], y[5])


def test_repeat_calls_are_deterministic():
    """Split-K partials are summed in a fixed order, so repeated calls agree bit for bit."""
    K, N = 6144, 2048
    x = H.act_f16(2, K, seed=81)
    w, s = H.w8(K, N, seed=82)
    ys = [_run_w8(x, w, s) for _ in range(3)]
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[1], ys[2])


# ---------------------------------------------------------------- prefill (M > 16): tiled MFMA path
#
# The library picks the LDS-tiled MFMA kernel for M > 16 when its time model says it
# beats row tiles; QLIN_PREFILL=tiled forces it (and QLIN_PREFILL_SHAPE its workgroup
# tile: 0 = 128x128, 1 = 256x256, 2 = 128x128 with two wave groups splitting each K
# tile) so these small cases exercise every tile shape, edge tiles in M and N
# included.

def _force_tiled(monkeypatch, shape):
    monkeypatch.setenv("QLIN_PREFILL", "tiled")
    monkeypatch.setenv("QLIN_PREFILL_SHAPE", str(shape))


@pytest.mark.parametrize("shape", [0, 1, 2])
@pytest.mark.parametrize("M", [17, 300])
@pytest.mark.parametrize("K,N", [(2048, 1024), (512, 2064)])
def test_prefill_w8(M, K, N, shape, monkeypatch):
    _force_tiled(monkeypatch, shape)
    x = H.act_f16(M, K, seed=300 + M)
    w, s = H.w8(K, N, seed=301)
    res = torch.randn((M, N), generator=H.gen(302)).to(torch.float16)
    H.assert_out_close(_run_w8(x, w, s), H.linear_w8_ref_cols(x, w, s, np.arange(N)))
    H.assert_out_close(_run_w8(x, w, s, residual=res),
                       H.linear_w8_ref_cols(x, w, s, np.arange(N), residual=res))


@pytest.mark.parametrize("shape", [0, 1, 2])
@pytest.mark.parametrize("M", [40, 256])
@pytest.mark.parametrize("group,zeros,sdt", [(128, "none", torch.float16), (32, "random", torch.float16),
                                             (64, "random", torch.bfloat16), (128, "eight", torch.float32),
                                             (128, "none", torch.bfloat16), (64, "none", torch.float32)])
def test_prefill_w4(M, group, zeros, sdt, shape, monkeypatch):
    """W4 prefill folds the group scale into the fp16 weight (one fp16 rounding per
    weight), so it is held to the GEMM tolerance, not bit-exactness.  The kernels are
    built per scale dtype, each with and without a zeros tensor: all six are run."""
    _force_tiled(monkeypatch, shape)
    K, N = 1024, 1280
    x = H.act_f16(M, K, seed=310 + M)
    packed, s, z = H.w4(K, N, seed=311, group=group, zeros=zeros)
    s = s.to(sdt)
    y = _run_w4(x, packed, s, z, out_dtype=torch.bfloat16)
    H.assert_out_close(y, H.linear_w4_ref_cols(x, packed, s.float() if sdt == torch.bfloat16 else s, z,
                                               np.arange(N)))


@pytest.mark.parametrize("shapes", [(0, 1)])
def test_prefill_tile_shapes_agree(shapes, monkeypatch):
    """The single-group workgroup tiles (128x128, 256x256) accumulate each output
    element over the same K order, so they give bit-identical results (W8 and W4
    with zeros).  The two-group shape sums its groups' substeps separately (another
    rounding order) and is checked against the oracle in the tests above."""
    M, K, N = 300, 1024, 1280
    x = H.act_f16(M, K, seed=340)
    w, s = H.w8(K, N, seed=341)
    packed, s4, z = H.w4(K, N, seed=342, group=64, zeros="random")
    outs = []
    for shape in shapes:
        _force_tiled(monkeypatch, shape)
        outs.append((_run_w8(x, w, s), _run_w4(x, packed, s4, z)))
    for o in outs[1:]:
        assert torch.equal(o[0], outs[0][0]) and torch.equal(o[1], outs[0][1])


@pytest.mark.parametrize("shape,splits", [(0, 2), (0, 16), (1, 4), (1, 8), (2, 4), (2, 16)])
def test_prefill_split_k(shape, splits, monkeypatch):
    """Split-K: each of `splits` workgroups per tile covers K/splits; the last to
    arrive sums the fp32 partials in split order.  Checked against the oracle (W8
    with residual, W4 with zeros and bf16 out) and for bit-identical repeat calls
    (the arrival order must not matter)."""
    _force_tiled(monkeypatch, shape)
    monkeypatch.setenv("QLIN_PREFILL_SPLITS", str(splits))
    M, K, N = 300, 1024, 1280
    x = H.act_f16(M, K, seed=360 + splits)
    w, s = H.w8(K, N, seed=361)
    res = torch.randn((M, N), generator=H.gen(362)).to(torch.float16)
    y = _run_w8(x, w, s, residual=res)
    H.assert_out_close(y, H.linear_w8_ref_cols(x, w, s, np.arange(N), residual=res))
    for _ in range(2):
        assert torch.equal(_run_w8(x, w, s, residual=res), y)
    packed, s4, z = H.w4(K, N, seed=363, group=128, zeros="random")
    y4 = _run_w4(x, packed, s4, z, out_dtype=torch.bfloat16)
    H.assert_out_close(y4, H.linear_w4_ref_cols(x, packed, s4, z, np.arange(N)))
    assert torch.equal(_run_w4(x, packed, s4, z, out_dtype=torch.bfloat16), y4)


@pytest.mark.parametrize("shape,sk", [(1, 16), (1, 24), (1, 31), (1, 37), (1, 40), (0, 24), (2, 31), (2, 37)])
def test_prefill_balanced(shape, sk, monkeypatch):
    """Balanced schedule: workgroup i covers the (tile, K tile) units
    [i*sk, (i+1)*sk) in order, so it may finish one tile and go on to the next; a
    tile shared by two workgroups is finished by the last to arrive, which adds the
    other's partial.  With 32 K tiles per tile: sk=16 halves every tile, sk=31 leaves
    one-K-tile pieces, sk=37 gives some workgroups three pieces, and sk=40 (8
    workgroups) and the 128x128 case (40) take the XCD-ordered ranges.  Checked against the
    oracle (W8 with residual, W4 with zeros and bf16 out) and for bit-identical
    repeat calls."""
    _force_tiled(monkeypatch, shape)
    monkeypatch.setenv("QLIN_PREFILL_SK", str(sk))
    M, K, N = 300, 2048, 1280
    x = H.act_f16(M, K, seed=370 + sk)
    w, s = H.w8(K, N, seed=371)
    res = torch.randn((M, N), generator=H.gen(372)).to(torch.float16)
    y = _run_w8(x, w, s, residual=res)
    H.assert_out_close(y, H.linear_w8_ref_cols(x, w, s, np.arange(N), residual=res))
    for _ in range(2):
        assert torch.equal(_run_w8(x, w, s, residual=res), y)
    packed, s4, z = H.w4(K, N, seed=373, group=128, zeros="random")
    y4 = _run_w4(x, packed, s4, z, out_dtype=torch.bfloat16)
    H.assert_out_close(y4, H.linear_w4_ref_cols(x, packed, s4, z, np.arange(N)))
    assert torch.equal(_run_w4(x, packed, s4, z, out_dtype=torch.bfloat16), y4)


@pytest.mark.parametrize("shape,splits", [(0, 1), (1, 1), (1, 4), (2, 2)])
def test_prefill_tile_order_does_not_change_results(shape, splits, monkeypatch):
    """The XCD-aware tile order (each XCD runs a contiguous run of the order, gm row
    tiles per group) only places workgroups: every gm, and the earlier order
    (QLIN_PREFILL_GM=0), gives the same bits, with and without split-K (W8 with
    residual, W4 with zeros).  M = 300 gives a partial last row tile and a
    workgroup count that is not a multiple of 8 for some shapes."""
    _force_tiled(monkeypatch, shape)
    monkeypatch.setenv("QLIN_PREFILL_SPLITS", str(splits))
    M, K, N = 300, 1024, 1280
    x = H.act_f16(M, K, seed=390 + shape)
    w, s = H.w8(K, N, seed=391)
    res = torch.randn((M, N), generator=H.gen(392)).to(torch.float16)
    packed, s4, z = H.w4(K, N, seed=393, group=128, zeros="random")
    outs = []
    for gm in ("0", "1", "2", "8", ""):
        monkeypatch.setenv("QLIN_PREFILL_GM", gm)
        outs.append((_run_w8(x, w, s, residual=res), _run_w4(x, packed, s4, z, out_dtype=torch.bfloat16)))
    H.assert_out_close(outs[0][0], H.linear_w8_ref_cols(x, w, s, np.arange(N), residual=res))
    for o in outs[1:]:
        assert torch.equal(o[0], outs[0][0]) and torch.equal(o[1], outs[0][1])


def test_prefill_balanced_rejects_three_way_tiles(monkeypatch):
    """sk=12 would spread a 32-K-tile output tile over three workgroups: refused."""
    _force_tiled(monkeypatch, 1)
    monkeypatch.setenv("QLIN_PREFILL_SK", "12")
    x = H.act_f16(300, 2048, seed=380)
    w, s = H.w8(2048, 1280, seed=381)
    with pytest.raises(ValueError, match="QLIN_PREFILL_SK"):
        _run_w8(x, w, s)


@pytest.mark.parametrize("shape", [0, 1, 2])
def test_prefill_rows_independent_of_chunking(shape, monkeypatch):
    """Rows computed in one M=300 call equal the same rows computed as an M=100
    chunk (the tiled kernel's per-row arithmetic does not depend on M)."""
    _force_tiled(monkeypatch, shape)
    K, N = 2048, 1024
    x = H.act_f16(300, K, seed=320)
    w, s = H.w8(K, N, seed=321)
    y = _run_w8(x, w, s)
    yc = _run_w8(x[100:200].contiguous(), w, s)
    assert torch.equal(y[100:200], yc)


@pytest.mark.parametrize("M,K,N", [(512, 512, 4096), (1024, 256, 8192)])
def test_prefill_default_dispatch(M, K, N):
    """Sizes where the library itself picks the tiled kernel (128x128 and 256x256
    tiles), checked on sampled columns against the oracle."""
    x = H.act_f16(M, K, seed=350 + M)
    w, s = H.w8(K, N, seed=351)
    packed, s4, z = H.w4(K, N, seed=352, group=128, zeros="random")
    cols = H.sample_cols(N, 512, seed=353)
    H.assert_out_close(_run_w8(x, w, s).cpu()[:, cols], H.linear_w8_ref_cols(x, w, s, cols))
    H.assert_out_close(_run_w4(x, packed, s4, z).cpu()[:, cols], H.linear_w4_ref_cols(x, packed, s4, z, cols))


# ---------------------------------------------------------------- the configs at full size
#
# Config 3 (prefill, M = 2048) and config 4 (9B-class W4 chain shapes) at their real
# sizes, checked against the oracle on sampled columns, plus a size-independent
# property: scaling the activations by 2 scales every output by exactly 2 (fp32 sums
# and the 16-bit rounding commute with a power of two when nothing overflows or
# underflows), so the whole output is checked bit for bit, not only the sample.


def _assert_doubled(y, y2):
    """y2 == 2 * y bit for bit where y is a normal fp16 number above the smallest one;
    where the sum v lies in the subnormal range (fixed spacing 2**-24, so also where
    round(v) = 2**-14 exactly) rounding 2v and doubling round(v) may differ by one
    step of 2**-24."""
    a, b = y.float().cpu(), y2.float().cpu()
    normal = a.abs() > 2.0 ** -14
    assert torch.equal(b[normal], 2 * a[normal])
    if (~normal).any():
        assert float((b[~normal] - 2 * a[~normal]).abs().max()) <= 2.0 ** -24


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("K,N", [(2048, 6144), (6144, 2048), (2048, 2048)])
@pytest.mark.parametrize("M", [128, 512, 2048])
def test_config3_prefill_full_size(kind, K, N, M):
    """Every config-3 case (M = 128, 512, 2048 on its three shapes, W8 and W4-g128)
    under the planner's own choice of tile shape, split-K and schedule."""
    x = H.act_f16(M, K, seed=500 + K + M)
    cols = H.sample_cols(N, 256, seed=501)
    if kind == "w8":
        w, s = H.w8(K, N, seed=502)
        y = _run_w8(x, w, s)
        y2 = _run_w8((x * 2).to(torch.float16), w, s)
        ref = H.linear_w8_ref_cols(x, w, s, cols)
    else:
        packed, s, z = H.w4(K, N, seed=502)
        y = _run_w4(x, packed, s, z)
        y2 = _run_w4((x * 2).to(torch.float16), packed, s, z)
        ref = H.linear_w4_ref_cols(x, packed, s, z, cols)
    H.assert_out_close(y.cpu()[:, cols], ref)
    _assert_doubled(y, y2)


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_prefill_balanced_default_plan_full_size(kind):
    """M = 2048 on the 9B-class gate shape (4096 x 12288): 384 tiles of 256x256 would
    take one and a half rounds of the chip, so the planner picks the balanced
    schedule (96 K tiles per workgroup, every other tile shared by two workgroups).
    Sampled columns against the oracle, and the activation-doubling property over the
    whole output."""
    M, K, N = 2048, 4096, 12288
    x = H.act_f16(M, K, seed=520)
    cols = H.sample_cols(N, 256, seed=521)
    if kind == "w8":
        w, s = H.w8(K, N, seed=522)
        y, y2 = _run_w8(x, w, s), _run_w8((x * 2).to(torch.float16), w, s)
        ref = H.linear_w8_ref_cols(x, w, s, cols)
    else:
        packed, s, z = H.w4(K, N, seed=522)
        y, y2 = _run_w4(x, packed, s, z), _run_w4((x * 2).to(torch.float16), packed, s, z)
        ref = H.linear_w4_ref_cols(x, packed, s, z, cols)
    H.assert_out_close(y.cpu()[:, cols], ref)
    _assert_doubled(y, y2)


@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("K,N", [(4096, 12288), (12288, 4096), (4096, 4096), (4096, 1024), (4096, 248320)])
def test_config4_chain_shapes_full_size(M, K, N):
    x = H.act_f16(M, K, seed=510 + M)
    packed, s, z = H.w4(K, N, seed=511 + K // 1024)
    y = _run_w4(x, packed, s, z)
    cols = H.sample_cols(N, 4096, seed=512)
    H.assert_out_close(y.cpu()[:, cols], H.linear_w4_ref_cols(x, packed, s, z, cols))
    y2 = _run_w4((x * 2).to(torch.float16), packed, s, z)
    _assert_doubled(y, y2)


@pytest.mark.parametrize("scale", [1e-5, 8.0])
@pytest.mark.parametrize("M", [4, 64, 300])
def test_w4_extreme_group_scales(scale, M):
    """bf16 group scales near 1e-5 (below fp16's normal range on their own) and near 8,
    through the decode path (M = 4, scales applied in fp32) and the prefill tiles
    (M = 64, 300: the scale times 2^8 is folded into the fp16 weight), against the
    oracle."""
    K, N = 1024, 1024
    x = H.act_f16(M, K, seed=900 + M)
    packed, s, z = H.w4(K, N, seed=901, group=128, zeros="random")
    s = (torch.rand(s.shape, generator=H.gen(902)) * scale + scale / 2).to(torch.bfloat16)
    y = _run_w4(x, packed, s, z)
    ref = H.linear_w4_ref_cols(x, packed, s, z, np.arange(N))
    if scale >= 1.0:  # keep the fp16 output in range
        assert np.abs(ref).max() < 6e4
    H.assert_out_close(y.cpu(), ref)
