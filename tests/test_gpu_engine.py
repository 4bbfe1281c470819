"""GPU parity of the engine-signature entry points (gemm_i8 / gemm_w4 / proj3(_w4) /
mlp_gate_up / mlp_gate_up_quant(_w4)) against the CPU oracle, at the shapes the
reference's own kernel tests use (.dev/test_kernels.py:31-80, .dev/test_fused.py:22-46)
and at the engine's decode shapes.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

pytestmark = pytest.mark.gpu



def _g():
    from qwen35_amd.kernels import gemm, w4
    return gemm, w4


def _bf16(t):
    return H.np_(t.cpu())


def _w4_engine(K, N, seed, group=128, zeros="none"):
    """Engine W4: packed nibbles + bf16 group scales (weights.py:297-305)."""
    packed, s, z = H.w4(K, N, seed, group=group, zeros=zeros)
    return packed, s.to(torch.bfloat16), z


@pytest.mark.parametrize("M,N,K", [(1, 3584, 1024), (37, 3584, 1024), (37, 2048, 1024),
                                   (1, 248320, 1024), (4, 6144, 2048), (8, 2048, 6144)])
@pytest.mark.parametrize("with_res", [False, True])
def test_gemm_i8(M, N, K, with_res):
    gemm, _ = _g()
    a, as_ = H.engine_act(M, K, seed=M + K)
    b, bs = H.engine_w8(K, N, seed=N)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    res = torch.randn((M, N), generator=H.gen(5)).to(torch.bfloat16) if with_res else None
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out,
                 residual=None if res is None else res.cuda(), block_k=64)
    cols = H.sample_cols(N, 8192)
    ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy()[:, cols], bs.numpy()[cols],
                        residual=None if res is None else _bf16(res)[:, cols])
    H.assert_out_close(out.cpu()[:, cols], ref)
    assert R.rel_l2(H.to_f32(out)[:, cols], ref) < 3e-3


def test_gemm_i8_in_place_residual():
    """`out is residual` (engine.py:238-240): each element read once before written."""
    gemm, _ = _g()
    M, K, N = 4, 2048, 2048
    a, as_ = H.engine_act(M, K, seed=1)
    b, bs = H.engine_w8(K, N, seed=2)
    hid = torch.randn((M, N), generator=H.gen(3)).to(torch.bfloat16)
    ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy(), bs.numpy(), residual=_bf16(hid))
    h = hid.cuda()
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), h, residual=h)
    H.assert_out_close(h, ref)


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("zeros", ["none", "random"])
@pytest.mark.parametrize("M", [1, 4, 37])
def test_gemm_w4(group, zeros, M):
    gemm, _ = _g()
    K, N = 2048, 2048
    a, as_ = H.engine_act(M, K, seed=M)
    b, bs, bz = _w4_engine(K, N, seed=group, group=group, zeros=zeros)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    res = torch.randn((M, N), generator=H.gen(9)).to(torch.bfloat16)
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out, residual=res.cuda(),
                 b_z=None if bz is None else bz.cuda())
    ref = R.gemm_w4_ref(a.numpy(), as_.numpy(), b.numpy(), _bf16(bs),
                        None if bz is None else bz.numpy(), residual=_bf16(res))
    H.assert_out_close(out, ref)


def test_gemm_w4_explicit_zero_eight_is_identical():
    _, w4 = _g()
    M, K, N = 4, 2048, 1024
    a, as_ = H.engine_act(M, K, seed=3)
    b, bs, _ = _w4_engine(K, N, seed=4)
    z8 = torch.full((K // 128, N), 8, dtype=torch.uint8, device="cuda")
    o0 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    o1 = torch.empty_like(o0)
    w4.gemm_w4(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), o0)
    w4.gemm_w4(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), o1, b_z=z8)
    assert torch.equal(o0, o1)


@pytest.mark.parametrize("M", [1, 4, 37])
def test_proj3_w8(M):
    """lin_qkv + lin_z shape (6144 + 2048) and q/k/v (4096 + 512 + 512)."""
    gemm, _ = _g()
    K = 2048
    a, as_ = H.engine_act(M, K, seed=11)
    w1, s1 = H.engine_w8(K, 6144, seed=12)
    w2, s2 = H.engine_w8(K, 2048, seed=13)
    out = torch.full((M, 8192 + 64), 7.0, dtype=torch.bfloat16, device="cuda")
    gemm.proj3(a.cuda(), as_.cuda(), w1.cuda(), s1.cuda(), w2.cuda(), s2.cuda(), None, None, out)
    ref = R.proj3_ref(a.numpy(), as_.numpy(), w1.numpy(), s1.numpy(), w2.numpy(), s2.numpy(), None, None)
    H.assert_out_close(out[:, :8192], ref)
    assert np.all(H.to_f32(out)[:, 8192:] == 7.0)       # columns beyond NT untouched
    q, sq = H.engine_w8(K, 4096, seed=14)
    k, sk = H.engine_w8(K, 512, seed=15)
    v, sv = H.engine_w8(K, 512, seed=16)
    out2 = torch.empty((M, 5120), dtype=torch.bfloat16, device="cuda")
    gemm.proj3(a.cuda(), as_.cuda(), q.cuda(), sq.cuda(), k.cuda(), sk.cuda(), v.cuda(), sv.cuda(), out2)
    ref2 = R.proj3_ref(a.numpy(), as_.numpy(), q.numpy(), sq.numpy(), k.numpy(), sk.numpy(), v.numpy(), sv.numpy())
    H.assert_out_close(out2, ref2)


@pytest.mark.parametrize("zeros", ["none", "random"])
@pytest.mark.parametrize("M", [1, 4, 37])
def test_proj3_w4(zeros, M):
    gemm, _ = _g()
    K = 2048
    a, as_ = H.engine_act(M, K, seed=21)
    ws = [_w4_engine(K, n, seed=22 + i, zeros=zeros) for i, n in enumerate((4096, 512, 512))]
    out = torch.empty((M, 5120), dtype=torch.bfloat16, device="cuda")
    cu = lambda t: None if t is None else t.cuda()
    gemm.proj3(a.cuda(), as_.cuda(), cu(ws[0][0]), cu(ws[0][1]), cu(ws[1][0]), cu(ws[1][1]),
               cu(ws[2][0]), cu(ws[2][1]), out, z1=cu(ws[0][2]), z2=cu(ws[1][2]), z3=cu(ws[2][2]))
    npz = lambda t: None if t is None else t.numpy()
    ref = R.proj3_ref(a.numpy(), as_.numpy(), ws[0][0].numpy(), _bf16(ws[0][1]), ws[1][0].numpy(),
                      _bf16(ws[1][1]), ws[2][0].numpy(), _bf16(ws[2][1]),
                      npz(ws[0][2]), npz(ws[1][2]), npz(ws[2][2]))
    H.assert_out_close(out, ref)


@pytest.mark.parametrize("M", [1, 16, 37])
def test_mlp_gate_up(M):
    gemm, _ = _g()
    K, N = 1024, 3584
    a, as_ = H.engine_act(M, K, seed=31)
    wg, sg = H.engine_w8(K, N, seed=32)
    wu, su = H.engine_w8(K, N, seed=33)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gemm.mlp_gate_up(a.cuda(), as_.cuda(), wg.cuda(), sg.cuda(), wu.cuda(), su.cuda(), out)
    ref = R.mlp_gate_up_ref(a.numpy(), as_.numpy(), wg.numpy(), sg.numpy(), wu.numpy(), su.numpy())
    H.assert_out_close(out, ref)


def _fused_vs_unfused(M, w4_=False, zeros="none", group=128):
    """.dev/test_fused.py:22-46: the fused int8 output must equal quant_row applied to
    the unfused bf16 h -- here bit for bit, since both kernels share the
    accumulation and the oracle's quant_groups is the reference's quantizer."""
    gemm, w4 = _g()
    K, N = 2048, 6144
    a, as_ = H.engine_act(M, K, seed=41 + M)
    if w4_:
        wg, sg, zg = _w4_engine(K, N, seed=42, group=group, zeros=zeros)
        wu, su, zu = _w4_engine(K, N, seed=43, group=group, zeros=zeros)
    else:
        (wg, sg), (wu, su) = H.engine_w8(K, N, seed=42), H.engine_w8(K, N, seed=43)
        zg = zu = None
    cu = lambda t: None if t is None else t.cuda()
    h = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    q1 = torch.empty((M, N), dtype=torch.int8, device="cuda")
    s1 = torch.empty((M, N // 64), dtype=torch.float32, device="cuda")
    if w4_:
        w4.mlp_gate_up_w4(cu(a), cu(as_), cu(wg), cu(sg), cu(wu), cu(su), h, zg=cu(zg), zu=cu(zu))
    else:
        gemm.mlp_gate_up(cu(a), cu(as_), cu(wg), cu(sg), cu(wu), cu(su), h)
    gemm.mlp_gate_up_quant(cu(a), cu(as_), cu(wg), cu(sg), cu(wu), cu(su), q1, s1, zg=cu(zg), zu=cu(zu))
    q0, s0 = R.quant_groups(H.to_f32(h))
    assert np.array_equal(q1.cpu().numpy(), q0)
    assert np.array_equal(s1.cpu().numpy(), s0)
    # and against the oracle's fused path: dequantized values within tolerance,
    # int8 codes equal except where bf16 rounding of h differs
    npz = lambda t: None if t is None else (H.np_(t) if t.dtype == torch.bfloat16 else t.numpy())
    qr, sr = R.mlp_gate_up_quant_ref(a.numpy(), as_.numpy(), npz(wg), npz(sg), npz(wu), npz(su),
                                     npz(zg), npz(zu))
    deq = q1.cpu().numpy().astype(np.float32) * np.repeat(s1.cpu().numpy(), 64, 1)
    deq_r = qr.astype(np.float32) * np.repeat(sr, 64, 1)
    assert R.max_rel_err(deq, deq_r) <= 1e-2
    assert (q1.cpu().numpy() == qr).mean() > 0.99


@pytest.mark.parametrize("M", [1, 16, 37])
def test_mlp_gate_up_quant_w8(M):
    _fused_vs_unfused(M)


@pytest.mark.parametrize("M,zeros,group", [(1, "none", 128), (4, "random", 128), (16, "none", 32),
                                           (37, "random", 64)])
def test_mlp_gate_up_quant_w4(M, zeros, group):
    _fused_vs_unfused(M, w4_=True, zeros=zeros, group=group)


@pytest.mark.parametrize("plan", ["4,8,0", "8,4,0"])
@pytest.mark.parametrize("M", [1, 2, 4])
def test_engine_decode_forced_plans(plan, M, monkeypatch):
    """The skinny decode plans (QLIN_ENGINE_DECODE=skinny; by default decode-sized
    engine calls run the engine decode work units): one-pass 64-column tiles and
    split-K 128-column tiles for every engine call kind (store + residual, proj3,
    gate/up + quant; W8 and W4), whatever the default plan is for the shape."""
    monkeypatch.setenv("QLIN_ENGINE_DECODE", "skinny")
    monkeypatch.setenv("QLIN_SKINNY_PLAN", plan)
    gemm, w4 = _g()
    K, N = 2048, 2048
    a, as_ = H.engine_act(M, K, seed=60 + M)
    b, bs = H.engine_w8(K, N, seed=61)
    res = torch.randn((M, N), generator=H.gen(62)).to(torch.bfloat16)
    out = res.clone().cuda()
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out, residual=out)
    H.assert_out_close(out, R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy(), bs.numpy(), residual=_bf16(res)))
    packed, s4, z = _w4_engine(K, N, seed=63, zeros="random")
    out4 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    w4.gemm_w4(a.cuda(), as_.cuda(), packed.cuda(), s4.cuda(), out4, b_z=z.cuda())
    H.assert_out_close(out4, R.gemm_w4_ref(a.numpy(), as_.numpy(), packed.numpy(), H.np_(s4), z.numpy()))
    _fused_vs_unfused(M)
    _fused_vs_unfused(M, w4_=True, zeros="random")


def test_engine_rows_independent_of_batch():
    gemm, _ = _g()
    K, N = 2048, 6144
    a, as_ = H.engine_act(4, K, seed=51)
    b, bs = H.engine_w8(K, N, seed=52)
    out = torch.empty((4, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out)
    for m in range(4):
        o1 = torch.empty((1, N), dtype=torch.bfloat16, device="cuda")
        gemm.gemm_i8(a[m:m + 1].cuda(), as_[m:m + 1].cuda(), b.cuda(), bs.cuda(), o1)
        assert torch.equal(o1[0], out[m])


def test_bad_arguments_raise_before_launch():
    gemm, _ = _g()
    a, as_ = H.engine_act(2, 96, seed=1)          # K not a multiple of 64
    b, bs = H.engine_w8(96, 64, seed=2)
    out = torch.empty((2, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        gemm.gemm_i8(a.cuda(), as_[:, :1].contiguous().cuda(), b.cuda(), bs.cuda(), out)


# ---------------------------------------------------------------- prefill-sized M (tiled int8 kernel)
#
# Engine-signature stores with more than 16 rows can run on the tiled int8 MFMA
# kernel when K % 64 == 0, every projection is a multiple of 128 columns and W4
# groups are at least 64; a time model picks it or the 16-row tiles.  The tests
# force it with QLIN_ENGINE_PREFILL=tiled (=skinny forces the row tiles).


@pytest.fixture
def tiled(monkeypatch):
    monkeypatch.setenv("QLIN_ENGINE_PREFILL", "tiled")
    return monkeypatch

@pytest.mark.parametrize("M", [17, 130, 300])
@pytest.mark.parametrize("K", [64, 192, 2048])
def test_gemm_i8_prefill_tiled(M, K, tiled):
    gemm, _ = _g()
    N = 1024
    a, as_ = H.engine_act(M, K, seed=400 + M + K)
    b, bs = H.engine_w8(K, N, seed=401)
    hid = torch.randn((M, N), generator=H.gen(402)).to(torch.bfloat16)
    ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy(), bs.numpy(), residual=_bf16(hid))
    h = hid.cuda()
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), h, residual=h)   # in place (engine.py:238-240)
    H.assert_out_close(h, ref)
    assert R.rel_l2(H.to_f32(h), ref) < 3e-3


@pytest.mark.parametrize("group,zeros", [(64, "none"), (128, "random"), (128, "eight"), (256, "random")])
@pytest.mark.parametrize("M", [40, 256])
def test_gemm_w4_prefill_tiled(group, zeros, M, tiled):
    gemm, _ = _g()
    K, N = 1024, 1280
    a, as_ = H.engine_act(M, K, seed=410 + M)
    b, bs, bz = _w4_engine(K, N, seed=411, group=group, zeros=zeros)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    res = torch.randn((M, N), generator=H.gen(412)).to(torch.bfloat16)
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out, residual=res.cuda(),
                 b_z=None if bz is None else bz.cuda())
    ref = R.gemm_w4_ref(a.numpy(), as_.numpy(), b.numpy(), _bf16(bs),
                        None if bz is None else bz.numpy(), residual=_bf16(res))
    H.assert_out_close(out, ref)


@pytest.mark.parametrize("M", [1, 4])
def test_decode_w4_explicit_zero_eight_is_identical(M):
    """Engine decode units (1-8 rows): a W4 call with an explicit zero tensor of all 8s
    gives the bits of the same call with none, for gemm_w4 with a residual (K split over
    units) and the fused gate/up + quant."""
    _, w4 = _g()
    K, N = 2048, 1024
    a, as_ = H.engine_act(M, K, seed=430 + M)
    b, bs, _ = _w4_engine(K, N, seed=431)
    z8 = torch.full((K // 128, N), 8, dtype=torch.uint8, device="cuda")
    res = torch.randn((M, N), generator=H.gen(432)).to(torch.bfloat16).cuda()
    o0 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    o1 = torch.empty_like(o0)
    w4.gemm_w4(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), o0, residual=res)
    w4.gemm_w4(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), o1, residual=res, b_z=z8)
    assert torch.equal(o0, o1)
    bu, bsu, _ = _w4_engine(K, N, seed=433)
    q0 = torch.empty((M, N), dtype=torch.int8, device="cuda")
    s0 = torch.empty((M, N // 64), dtype=torch.float32, device="cuda")
    q1, s1 = torch.empty_like(q0), torch.empty_like(s0)
    w4.mlp_gate_up_quant_w4(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), bu.cuda(), bsu.cuda(), q0, s0)
    w4.mlp_gate_up_quant_w4(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), bu.cuda(), bsu.cuda(), q1, s1, zg=z8, zu=z8)
    assert torch.equal(q0, q1) and torch.equal(s0, s1)


def test_prefill_tiled_w4_explicit_zero_eight_is_identical(tiled):
    _, w4 = _g()
    M, K, N = 64, 1024, 1024
    a, as_ = H.engine_act(M, K, seed=420)
    b, bs, _ = _w4_engine(K, N, seed=421)
    z8 = torch.full((K // 128, N), 8, dtype=torch.uint8, device="cuda")
    o0 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    o1 = torch.empty_like(o0)
    w4.gemm_w4(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), o0)
    w4.gemm_w4(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), o1, b_z=z8)
    assert torch.equal(o0, o1)


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_prefill_tiled_rows_independent_of_chunking(kind, tiled):
    """Rows of an M=300 call equal the same rows computed as an M=100 chunk: the
    tiled kernel's K order does not depend on M (chunked prefill, ENGINEERING.md:453-455)."""
    gemm, _ = _g()
    K, N = 2048, 1024
    a, as_ = H.engine_act(300, K, seed=430)
    if kind == "w8":
        b, bs = H.engine_w8(K, N, seed=431)
        bz = None
    else:
        b, bs, bz = _w4_engine(K, N, seed=431, zeros="random")
    cu = lambda t: None if t is None else t.cuda()
    y = torch.empty((300, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), y, b_z=cu(bz))
    yc = torch.empty((100, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a[100:200].contiguous().cuda(), as_[100:200].contiguous().cuda(), b.cuda(), bs.cuda(), yc, b_z=cu(bz))
    assert torch.equal(y[100:200], yc)


def test_prefill_tiled_matches_row_tiles(tiled):
    """The tiled kernel and the 16-row skinny kernel fold K in the same order (two
    interleaved lanes per split, splits in order): identical bits."""
    gemm, _ = _g()
    M, K, N = 96, 2048, 2048
    a, as_ = H.engine_act(M, K, seed=440)
    b, bs = H.engine_w8(K, N, seed=441)
    y0 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), y0)
    tiled.setenv("QLIN_ENGINE_PREFILL", "skinny")
    y1 = torch.empty_like(y0)
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), y1)
    assert torch.equal(y0, y1)


@pytest.mark.parametrize("N,group", [(1040, 128), (1024, 32)])
def test_prefill_outside_tiled_kernel(N, group, tiled):
    """Column counts that are not a multiple of 128 and W4 group 32 stay on the
    16-row tiles; still checked against the oracle."""
    gemm, _ = _g()
    M, K = 40, 1024
    a, as_ = H.engine_act(M, K, seed=450)
    b, bs, bz = _w4_engine(K, N, seed=451, group=group, zeros="random")
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out, b_z=bz.cuda())
    ref = R.gemm_w4_ref(a.numpy(), as_.numpy(), b.numpy(), _bf16(bs), bz.numpy())
    H.assert_out_close(out, ref)


@pytest.mark.parametrize("splits", [2, 4, 8])
@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_gemm_prefill_tiled_split_k(kind, splits, tiled):
    """Split-K on the tiled int8 kernel (store epilogue): each of `splits` workgroups
    per tile covers K/splits, and the last to arrive sums the fp32 partials in split
    order.  W8 with the residual in place, W4 with zeros; against the oracle and
    bit-identical on repeat calls (the arrival order must not matter)."""
    gemm, _ = _g()
    tiled.setenv("QLIN_ENGINE_SPLITS", str(splits))
    M, K, N = 300, 2048, 1024
    a, as_ = H.engine_act(M, K, seed=480 + splits)
    hid = torch.randn((M, N), generator=H.gen(481)).to(torch.bfloat16)
    if kind == "w8":
        b, bs = H.engine_w8(K, N, seed=482)
        bz = None
        ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy(), bs.numpy(), residual=_bf16(hid))
    else:
        b, bs, bz = _w4_engine(K, N, seed=482, zeros="random")
        ref = R.gemm_w4_ref(a.numpy(), as_.numpy(), b.numpy(), _bf16(bs), bz.numpy(), residual=_bf16(hid))
    cu = lambda t: None if t is None else t.cuda()
    outs = []
    for _ in range(3):
        h = hid.cuda()
        gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), h, residual=h, b_z=cu(bz))
        outs.append(h)
    H.assert_out_close(outs[0], ref)
    assert torch.equal(outs[1], outs[0]) and torch.equal(outs[2], outs[0])


def test_proj3_prefill_tiled_split_k(tiled):
    """proj3 (three column segments in one launch) with split-K on the tiled kernel."""
    gemm, _ = _g()
    tiled.setenv("QLIN_ENGINE_SPLITS", "4")
    M, K = 200, 1024
    a, as_ = H.engine_act(M, K, seed=485)
    ws = [H.engine_w8(K, n, seed=486 + i) for i, n in enumerate((1024, 256, 256))]
    out = torch.empty((M, 1536), dtype=torch.bfloat16, device="cuda")
    gemm.proj3(a.cuda(), as_.cuda(), *(t.cuda() for w in ws for t in w), out)
    ref = R.proj3_ref(a.numpy(), as_.numpy(), *(t.numpy() for w in ws for t in w))
    H.assert_out_close(out, ref)


def test_prefill_tiled_split_k_rows_independent_of_chunking(tiled):
    """With a fixed split count the K order of a row does not depend on M either."""
    gemm, _ = _g()
    tiled.setenv("QLIN_ENGINE_SPLITS", "4")
    K, N = 2048, 1024
    a, as_ = H.engine_act(300, K, seed=487)
    b, bs = H.engine_w8(K, N, seed=488)
    y = torch.empty((300, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), y)
    yc = torch.empty((100, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a[100:200].contiguous().cuda(), as_[100:200].contiguous().cuda(), b.cuda(), bs.cuda(), yc)
    assert torch.equal(y[100:200], yc)


@pytest.mark.parametrize("splits", [1, 4])
def test_prefill_tiled_tile_order_does_not_change_results(splits, tiled):
    """The XCD-aware tile order of the tiled int8 kernel only places workgroups: every
    gm, and the earlier order (QLIN_I8_GM=0), gives the same bits for gemm_i8 with the
    residual and for gate/up + requant (codes and scales), with and without split-K."""
    gemm, _ = _g()
    tiled.setenv("QLIN_ENGINE_SPLITS", str(splits))
    M, K, N = 300, 2048, 1280
    a, as_ = H.engine_act(M, K, seed=495 + splits)
    b, bs = H.engine_w8(K, N, seed=496)
    (wg, sg), (wu, su) = H.engine_w8(K, N, seed=497), H.engine_w8(K, N, seed=498)
    hid = torch.randn((M, N), generator=H.gen(499)).to(torch.bfloat16).cuda()
    outs = []
    for gm in ("0", "1", "2", "8", ""):
        tiled.setenv("QLIN_I8_GM", gm)
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), y, residual=hid)
        q = torch.empty((M, N), dtype=torch.int8, device="cuda")
        s = torch.empty((M, N // 64), dtype=torch.float32, device="cuda")
        gemm.mlp_gate_up_quant(a.cuda(), as_.cuda(), wg.cuda(), sg.cuda(), wu.cuda(), su.cuda(), q, s)
        outs.append((y.cpu(), q.cpu(), s.cpu()))
    ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy(), bs.numpy(), residual=_bf16(hid.cpu()))
    H.assert_out_close(outs[0][0], ref)
    for o in outs[1:]:
        assert all(torch.equal(u, v) for u, v in zip(o, outs[0]))


@pytest.mark.parametrize("splits,K", [(1, 2048), (2, 2048), (4, 2048), (1, 1984)])
def test_prefill_tiled_dma_tile_same_bits(splits, K, tiled):
    """The 4-wave 128 x 64 DMA tile (QLIN_I8_DMA=1) and the 8-wave 128 x 128 tile (the
    default) fold every output in the same order: gemm_i8 with the residual and proj3
    (three column segments) give the same bits on both, also with an odd number of
    64-wide blocks (the last stage holds one block)."""
    gemm, _ = _g()
    tiled.setenv("QLIN_ENGINE_SPLITS", str(splits))
    M = 300
    a, as_ = H.engine_act(M, K, seed=520 + splits)
    b, bs = H.engine_w8(K, 1280, seed=521)
    ws = [H.engine_w8(K, n, seed=522 + i) for i, n in enumerate((1024, 256, 256))]
    hid = torch.randn((M, 1280), generator=H.gen(525)).to(torch.bfloat16).cuda()
    outs = []
    for dma in ("1", "0"):
        tiled.setenv("QLIN_I8_DMA", dma)
        y = torch.empty((M, 1280), dtype=torch.bfloat16, device="cuda")
        gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), y, residual=hid)
        p3 = torch.empty((M, 1536), dtype=torch.bfloat16, device="cuda")
        gemm.proj3(a.cuda(), as_.cuda(), *(t.cuda() for w in ws for t in w), p3)
        outs.append((y.cpu(), p3.cpu()))
    ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy(), bs.numpy(), residual=_bf16(hid.cpu()))
    H.assert_out_close(outs[0][0], ref)
    for o in outs[1:]:
        assert torch.equal(outs[0][0], o[0]) and torch.equal(outs[0][1], o[1])


def test_prefill_tiled_bad_split_raises(tiled):
    gemm, _ = _g()
    tiled.setenv("QLIN_ENGINE_SPLITS", "3")  # 32 blocks of 64 do not split three ways
    a, as_ = H.engine_act(64, 2048, seed=489)
    b, bs = H.engine_w8(2048, 1024, seed=489)
    out = torch.empty((64, 1024), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="K splits"):
        gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out)


@pytest.mark.parametrize("M,K,N", [(512, 2048, 6144), (512, 6144, 2048), (512, 2048, 2048), (384, 6144, 2048),
                                   (100, 6144, 2048)])
def test_engine_prefill_default_dispatch(M, K, N):
    """Engine prefill chunk sizes with the library's own choice of kernel (tiled int8,
    split over K for the narrow shapes at M = 384 and 512; row tiles at M = 100),
    sampled columns."""
    gemm, _ = _g()
    a, as_ = H.engine_act(M, K, seed=460)
    b, bs = H.engine_w8(K, N, seed=461)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out)
    cols = H.sample_cols(N, 512, seed=462)
    ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy()[:, cols], bs.numpy()[cols])
    H.assert_out_close(out.cpu()[:, cols], ref)


@pytest.mark.parametrize("M", [17, 200])
def test_mlp_gate_up_prefill_tiled(M, tiled):
    """Fused gate/up (bf16 h) on the tiled int8 kernel, against the oracle."""
    gemm, _ = _g()
    K, N = 1024, 1280
    a, as_ = H.engine_act(M, K, seed=470 + M)
    wg, sg = H.engine_w8(K, N, seed=471)
    wu, su = H.engine_w8(K, N, seed=472)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gemm.mlp_gate_up(a.cuda(), as_.cuda(), wg.cuda(), sg.cuda(), wu.cuda(), su.cuda(), out)
    ref = R.mlp_gate_up_ref(a.numpy(), as_.numpy(), wg.numpy(), sg.numpy(), wu.numpy(), su.numpy())
    H.assert_out_close(out, ref)


@pytest.mark.parametrize("M", [17, 200])
def test_mlp_gate_up_quant_w8_prefill_tiled(M, tiled):
    """mlp_gate_up_quant on the tiled kernel: bit-identical to quantizing its own
    bf16 h, and within tolerance of the oracle."""
    _fused_vs_unfused(M)


@pytest.mark.parametrize("zeros,group", [("none", 128), ("random", 64)])
def test_mlp_gate_up_quant_w4_prefill_tiled(zeros, group, tiled):
    _fused_vs_unfused(96, w4_=True, zeros=zeros, group=group)


@pytest.mark.parametrize("splits", [2, 4])
@pytest.mark.parametrize("w4_,zeros,group", [(False, "none", 128), (True, "random", 128)])
def test_mlp_gate_up_quant_prefill_tiled_split_k(splits, w4_, zeros, group, tiled):
    """Split-K on the tiled kernel's gate/up epilogue: each split stores both weight
    sets' partials and the last to arrive sums them in split order before silu(g) * u
    and the requantization -- bit-identical to quantizing its own bf16 h, within
    tolerance of the oracle."""
    tiled.setenv("QLIN_ENGINE_SPLITS", str(splits))
    _fused_vs_unfused(200, w4_=w4_, zeros=zeros, group=group)


@pytest.mark.parametrize("splits", [1, 2])
def test_gate_up_quant_tiled_matches_row_tiles(splits, tiled):
    """gate/up + requant: the tiled kernel and the 16-row tiles give identical codes and
    scales for the same split count (the K order depends on the split count only)."""
    gemm, _ = _g()
    M, K, N = 96, 2048, 1280
    a, as_ = H.engine_act(M, K, seed=450)
    (wg, sg), (wu, su) = H.engine_w8(K, N, seed=451), H.engine_w8(K, N, seed=452)
    cu = lambda t: t.cuda()
    tiled.setenv("QLIN_ENGINE_SPLITS", str(splits))
    out = []
    for fam in ("tiled", "skinny"):
        tiled.setenv("QLIN_ENGINE_PREFILL", fam)
        q = torch.empty((M, N), dtype=torch.int8, device="cuda")
        s = torch.empty((M, N // 64), dtype=torch.float32, device="cuda")
        gemm.mlp_gate_up_quant(cu(a), cu(as_), cu(wg), cu(sg), cu(wu), cu(su), q, s)
        out.append((q.cpu(), s.cpu()))
    assert torch.equal(out[0][0], out[1][0]) and torch.equal(out[0][1], out[1][1])


@pytest.mark.parametrize("M,K,N", [(1, 2048, 6144), (4, 2048, 6144), (512, 2048, 6144), (512, 6144, 2048)])
def test_engine_scale_property_full_size(M, K, N):
    """Doubling the per-64 activation scales doubles every bf16 output exactly (the
    int32 dots are unchanged and the fp32 fold, the split-K sum and the rounding
    commute with 2), over the whole output at decode and prefill-chunk sizes."""
    gemm, _ = _g()
    a, as_ = H.engine_act(M, K, seed=490 + M)
    b, bs = H.engine_w8(K, N, seed=491)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    y2 = torch.empty_like(y)
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), y)
    gemm.gemm_i8(a.cuda(), (as_ * 2).cuda(), b.cuda(), bs.cuda(), y2)
    assert torch.equal(y2, (y.float() * 2).to(torch.bfloat16))


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_wide_decode_residual_edge_tile(kind):
    """A wide decode launch (N >= 131072 takes one-wave 256-column tiles for W4, 128 for
    W8) whose last tile is partial, with a residual and 4 rows: the epilogue's later
    passes read the residual only inside the row."""
    gemm, _ = _g()
    M, K, N = 4, 1024, 131072 + 144
    a, as_ = H.engine_act(M, K, seed=920)
    if kind == "w8":
        b, bs = H.engine_w8(K, N, seed=921)
        bz = None
    else:
        b, bs, bz = _w4_engine(K, N, seed=921, zeros="random")
    hid = torch.randn((M, N), generator=H.gen(922)).to(torch.bfloat16)
    h = hid.cuda()
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), h, residual=h, b_z=None if bz is None else bz.cuda())
    cols = np.concatenate([np.arange(N - 512, N), H.sample_cols(N - 512, 1024, seed=923)])
    if kind == "w8":
        ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy()[:, cols], bs.numpy()[cols],
                            residual=_bf16(hid)[:, cols])
    else:
        ref = R.gemm_w4_ref(a.numpy(), as_.numpy(), b.numpy()[:, cols], _bf16(bs)[:, cols], bz.numpy()[:, cols],
                            residual=_bf16(hid)[:, cols])
    H.assert_out_close(h.cpu()[:, cols], ref)


def test_two_streams_use_separate_workspaces():
    """Split-K decode calls issued on two streams at once: each stream has its own
    workspace (arrival counters and partials), so both results equal the same calls
    made on one stream."""
    gemm, _ = _g()
    from qwen35_amd.kernels import qlin as C
    M, K, N = 4, 6144, 2048                     # a split-K decode plan
    a, as_ = H.engine_act(M, K, seed=930)
    b, bs = H.engine_w8(K, N, seed=931)
    a2, as2 = H.engine_act(M, K, seed=932)
    a, as_, a2, as2, b, bs = a.cuda(), as_.cuda(), a2.cuda(), as2.cuda(), b.cuda(), bs.cuda()
    ref1 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ref2 = torch.empty_like(ref1)
    gemm.gemm_i8(a, as_, b, bs, ref1)
    gemm.gemm_i8(a2, as2, b, bs, ref2)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs1 = [torch.empty_like(ref1) for _ in range(20)]
    outs2 = [torch.empty_like(ref1) for _ in range(20)]
    torch.cuda.synchronize()
    for o1, o2 in zip(outs1, outs2):
        with torch.cuda.stream(s1):
            gemm.gemm_i8(a, as_, b, bs, o1)
        with torch.cuda.stream(s2):
            gemm.gemm_i8(a2, as2, b, bs, o2)
    torch.cuda.synchronize()
    assert C.workspace(ref1.device, s1.cuda_stream).data_ptr() != C.workspace(ref1.device, s2.cuda_stream).data_ptr()
    for o1, o2 in zip(outs1, outs2):
        assert torch.equal(o1, ref1)
        assert torch.equal(o2, ref2)


@pytest.mark.parametrize("M", [1, 4, 8])
@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_decode_polling_exchange_same_bits_and_slots_left_zero(kind, M, monkeypatch):
    """Decode-sized engine calls whose units are all resident finish their split tiles
    by polling the partners' slots in the workspace's slot region (parts stored with
    flipped sign bits, zero = empty); QLIN_ECALL_POLL=0 takes the arrival counters.
    Both give the same bits for gemm + residual, proj3 and gate/up + requant (K = 2048
    and 6144: 4 and 12 splits), call after call, and the slot region is zero after
    every call (the next call's finisher would read a leftover part as data)."""
    from qwen35_amd.kernels import qlin
    gemm, w4 = _g()
    K1, N1, K2, N2 = 2048, 6144, 6144, 2048
    a1, s1 = H.engine_act(M, K1, seed=71)
    a2, s2 = H.engine_act(M, K2, seed=72)
    if kind == "w8":
        wg, sg = H.engine_w8(K1, N1, seed=73)
        wu, su = H.engine_w8(K1, N1, seed=74)
        wd, sd = H.engine_w8(K2, N2, seed=75)
        zg = zu = zd = None
    else:
        wg, sg, zg = _w4_engine(K1, N1, seed=73, zeros="random")
        wu, su, zu = _w4_engine(K1, N1, seed=74, zeros="random")
        wd, sd, zd = _w4_engine(K2, N2, seed=75)
    cu = lambda t: None if t is None else t.cuda()
    res = torch.randn((M, N2), dtype=torch.float32).to(torch.bfloat16).cuda()

    def calls():
        outs = {}
        q = torch.empty((M, N1), dtype=torch.int8, device="cuda")
        qs = torch.empty((M, N1 // 64), dtype=torch.float32, device="cuda")
        gemm.mlp_gate_up_quant(cu(a1), cu(s1), cu(wg), cu(sg), cu(wu), cu(su), q, qs, zg=cu(zg), zu=cu(zu))
        outs["q"], outs["qs"] = q.cpu(), qs.cpu()
        d = res.clone()
        if kind == "w8":
            gemm.gemm_i8(cu(a2), cu(s2), cu(wd), cu(sd), d, residual=d)
        else:
            w4.gemm_w4(cu(a2), cu(s2), cu(wd), cu(sd), d, residual=d, b_z=cu(zd))
        outs["d"] = d.cpu()
        p = torch.empty((M, 512 + 1024 + 1536), dtype=torch.bfloat16, device="cuda")
        if kind == "w8":
            gemm.proj3(cu(a1), cu(s1), cu(wg[:, :512].contiguous()), cu(sg[:512].contiguous()),
                       cu(wu[:, :1024].contiguous()), cu(su[:1024].contiguous()),
                       cu(wg[:, 512:2048].contiguous()), cu(sg[512:2048].contiguous()), p)
            outs["p"] = p.cpu()
        torch.cuda.synchronize()
        return outs

    slots = lambda: qlin.workspace(torch.device("cuda", torch.cuda.current_device()))[1 << 20:5 << 20]
    monkeypatch.setenv("QLIN_ECALL_POLL", "0")
    ref = calls()
    assert int(slots().count_nonzero()) == 0
    monkeypatch.setenv("QLIN_ECALL_POLL", "1")
    for _ in range(3):
        got = calls()
        assert int(slots().count_nonzero()) == 0
        for k in ref:
            assert torch.equal(ref[k], got[k]), k
