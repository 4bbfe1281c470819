"""GPU parity of the activation producers (kernels/norm.py:28-57, 95-137, 168-188) and of
the linears that run them in their own launch.

* The standalone producers (rmsnorm_quant, gate_mul_quant, norm_gated_quant) and the
  producers' exp must equal the oracle bit for bit: int8 codes and fp32 scales.
* A fused call (`kernels/fused.py`) must equal the two-call sequence it replaces --
  the standalone producer, then the engine-signature linear -- bit for bit, for every
  plan family: the decode work units (M = 1-8, the producer in every unit's
  prologue), two-wave row tiles (M = 9-16), the tiled prefill kernel (the producer
  then runs as a launch of its own), with and without the optional code outputs.
* The fused result is also within the GEMM tolerance of the oracle's fp32 result on
  the oracle's codes.
Shapes are the engine's 2B-class layer (hidden 2048; engine.py:218-279).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

pytestmark = pytest.mark.gpu

MS = [1, 2, 4, 8, 16, 40, 512]


def _k():
    from qwen35_amd.kernels import fused, gemm, norm, qlin
    return fused, gemm, norm, qlin


def _f32(t):
    return t.detach().float().cpu().numpy()


def _act(shape, seed, dtype=torch.bfloat16, scale=1.0):
    return (torch.randn(shape, generator=H.gen(seed)) * scale).to(dtype)


def _codes(M, K):
    return (torch.empty((M, K), dtype=torch.int8, device="cuda"),
            torch.empty((M, K // 64), dtype=torch.float32, device="cuda"))


def _assert_codes(q, s, ref):
    rq, rs = ref
    gq, gs = q.cpu().numpy(), s.cpu().numpy()
    if not (gq == rq).all():
        i = np.argwhere(gq != rq)[0]
        raise AssertionError(f"{int((gq != rq).sum())} codes differ; first at {tuple(i)}: "
                             f"gpu {gq[tuple(i)]} oracle {rq[tuple(i)]}")
    assert (gs.view(np.uint32) == rs.astype(np.float32).view(np.uint32)).all(), "scales differ"


def test_pro_exp_bit_exact():
    _, _, _, C = _k()
    x = np.concatenate([np.linspace(-100.0, 100.0, 1_000_001, dtype=np.float32),
                        (np.random.default_rng(0).standard_normal(500_000) * 30).astype(np.float32),
                        np.array([0.0, -0.0, 88.0, 88.000008, -87.0, -87.00001, 1e-30, -1e-30], np.float32)])
    xt = torch.from_numpy(x).cuda()
    y = torch.empty_like(xt)
    C.call("qlin_pro_exp_f32", C.ptr(xt), C.ptr(y), x.size, C.stream_of(xt))
    ref = R.exp_f32(x)
    got = y.cpu().numpy()
    same = got.view(np.uint32) == ref.view(np.uint32)
    assert same.all(), f"{int((~same).sum())} values differ, first x={x[~same][0]!r}"


@pytest.mark.parametrize("M", [1, 4, 37])
@pytest.mark.parametrize("K", [2048, 4096])
@pytest.mark.parametrize("xdt,wdt,one_plus", [(torch.bfloat16, torch.bfloat16, True),
                                              (torch.float16, torch.float32, False)])
def test_rmsnorm_quant_bit_exact(M, K, xdt, wdt, one_plus):
    _, _, N_, _ = _k()
    xf = _act((M, K + 64), seed=M + K, dtype=xdt, scale=2.0)
    x = xf[:, :K]
    w = (torch.randn(K, generator=H.gen(7)) * 0.1).to(wdt)
    q, s = _codes(M, K)
    xg = xf.cuda()[:, :K]                                            # row stride K + 64
    assert xg.stride(0) == K + 64
    N_.rmsnorm_quant(xg, w.cuda(), q, s, eps=1e-6, one_plus=one_plus)
    _assert_codes(q, s, R.rmsnorm_quant_ref(x.float().numpy(), w.float().numpy(), 1e-6, one_plus))


@pytest.mark.parametrize("M", [1, 4, 33])
@pytest.mark.parametrize("N,hd", [(2048, 256), (4096, 128)])
def test_gate_mul_quant_bit_exact(M, N, hd):
    _, _, N_, _ = _k()
    a = _act((M, N), seed=M, scale=3.0)
    g = _act((M, 2 * N + 1024), seed=M + 1, scale=4.0)   # the engine's proj buffer: q | gate, then k, v
    q, s = _codes(M, N)
    N_.gate_mul_quant(a.cuda(), g.cuda(), q, s, hd=hd)
    _assert_codes(q, s, R.gate_mul_quant_ref(a.float().numpy(), g.float().numpy(), hd))


@pytest.mark.parametrize("T", [1, 4, 19])
@pytest.mark.parametrize("N,hd", [(2048, 128), (4096, 256)])
def test_norm_gated_quant_bit_exact(T, N, hd):
    _, _, N_, _ = _k()
    v = _act((T, N), seed=T, scale=0.5)
    proj = _act((T, 6144 + N), seed=T + 2, scale=2.0)     # z = proj[:, conv_dim:] (engine.py:236)
    z = proj[:, 6144:]
    w = (torch.randn(hd, generator=H.gen(3)) * 0.3 + 1.0).to(torch.bfloat16)
    q, s = _codes(T, N)
    N_.norm_gated_quant(v.cuda(), proj.cuda()[:, 6144:], w.cuda(), q, s, eps=1e-6)
    _assert_codes(q, s, R.norm_gated_quant_ref(v.float().numpy(), z.float().numpy(), w.float().numpy(), 1e-6))


# ---------------------------------------------------------------- fused == two calls

def _w8(K, N, seed):
    b, bs = H.engine_w8(K, N, seed)
    return b.cuda(), bs.cuda()


def _w4(K, N, seed, zeros=True):
    packed, sc, z = H.w4(K, N, seed, group=128, zeros="random" if zeros else "none")
    return packed.cuda(), sc.to(torch.bfloat16).cuda(), (z.cuda() if z is not None else None)


def _rms_inputs(M, K, seed):
    x = _act((M, K), seed=seed, scale=2.0).cuda()
    nw = (torch.randn(K, generator=H.gen(seed + 1)) * 0.1).to(torch.bfloat16).cuda()
    return x, nw


@pytest.mark.parametrize("M", MS)
@pytest.mark.parametrize("wk", ["w8", "w4"])
@pytest.mark.parametrize("keep", [True, False])
def test_rmsnorm_proj3_equals_two_calls(M, wk, keep):
    """rmsnorm_quant + proj3 (engine.py:220-226: lin_qkv 2048->6144 + lin_z ->2048)."""
    FU, G, N_, _ = _k()
    K = 2048
    x, nw = _rms_inputs(M, K, seed=M)
    if wk == "w8":
        (w1, s1), (w2, s2) = _w8(K, 6144, 11), _w8(K, 2048, 12)
        z1 = z2 = None
    else:
        w1, s1, z1 = _w4(K, 6144, 11)
        w2, s2, z2 = _w4(K, 2048, 12)
    q0, s0 = _codes(M, K)
    N_.rmsnorm_quant(x, nw, q0, s0, 1e-6)
    ref = torch.empty((M, 8192), dtype=torch.bfloat16, device="cuda")
    G.proj3(q0, s0, w1, s1, w2, s2, None, None, ref, z1=z1, z2=z2)
    out = torch.zeros_like(ref)
    q1, s1c = _codes(M, K) if keep else (None, None)
    pro = FU.Producer.rmsnorm(x, nw, 1e-6, q=q1, s=s1c)
    FU.pro_proj3(pro, w1, s1, w2, s2, None, None, out, z1=z1, z2=z2)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    if keep:
        assert torch.equal(q1, q0) and torch.equal(s1c.view(torch.int32), s0.view(torch.int32))


@pytest.mark.parametrize("M", MS)
@pytest.mark.parametrize("wk", ["w8", "w4"])
def test_rmsnorm_gate_up_quant_equals_two_calls(M, wk):
    """rmsnorm_quant + mlp_gate_up_quant (engine.py:272-276: gate/up 2048->6144)."""
    FU, G, N_, _ = _k()
    K, N = 2048, 6144
    x, nw = _rms_inputs(M, K, seed=M + 100)
    if wk == "w8":
        (wg, sg), (wu, su) = _w8(K, N, 21), _w8(K, N, 22)
        zg = zu = None
    else:
        wg, sg, zg = _w4(K, N, 21)
        wu, su, zu = _w4(K, N, 22)
    q0, s0 = _codes(M, K)
    N_.rmsnorm_quant(x, nw, q0, s0, 1e-6)
    hq0, hs0 = _codes(M, N)
    G.mlp_gate_up_quant(q0, s0, wg, sg, wu, su, hq0, hs0, zg=zg, zu=zu)
    hq1, hs1 = _codes(M, N)
    FU.pro_mlp_gate_up_quant(FU.Producer.rmsnorm(x, nw, 1e-6), wg, sg, wu, su, hq1, hs1, zg=zg, zu=zu)
    torch.cuda.synchronize()
    assert torch.equal(hq1, hq0) and torch.equal(hs1.view(torch.int32), hs0.view(torch.int32))


@pytest.mark.parametrize("M", MS)
@pytest.mark.parametrize("wk", ["w8", "w4"])
def test_gate_mul_o_proj_equals_two_calls(M, wk):
    """gate_mul_quant + gemm_i8 with the residual in place (engine.py:265-268)."""
    FU, G, N_, _ = _k()
    K, N, hd = 2048, 2048, 256
    a = _act((M, K), seed=M + 200, scale=3.0).cuda()
    proj = _act((M, 5120), seed=M + 201, scale=4.0).cuda()     # q | gate (4096), k, v
    if wk == "w8":
        b, bs = _w8(K, N, 31)
        bz = None
    else:
        b, bs, bz = _w4(K, N, 31)
    hid = _act((M, N), seed=M + 202).cuda()
    q0, s0 = _codes(M, K)
    N_.gate_mul_quant(a, proj, q0, s0, hd=hd)
    ref = hid.clone()
    G.gemm_i8(q0, s0, b, bs, ref, residual=ref, b_z=bz)
    out = hid.clone()
    FU.pro_gemm_i8(FU.Producer.gate_mul(a, proj, hd=hd), b, bs, out, residual=out, b_z=bz)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M", MS)
@pytest.mark.parametrize("wk", ["w8", "w4"])
def test_norm_gated_lin_out_equals_two_calls(M, wk):
    """norm_gated_quant + gemm_i8 with the residual in place (engine.py:236-240)."""
    FU, G, N_, _ = _k()
    K, N, hd = 2048, 2048, 128
    v = _act((M, K), seed=M + 300, scale=0.5).cuda()
    proj = _act((M, 6144 + K), seed=M + 301, scale=2.0).cuda()
    z = proj[:, 6144:]
    w = (torch.randn(hd, generator=H.gen(302)) * 0.3 + 1.0).to(torch.bfloat16).cuda()
    if wk == "w8":
        b, bs = _w8(K, N, 41)
        bz = None
    else:
        b, bs, bz = _w4(K, N, 41)
    hid = _act((M, N), seed=M + 303).cuda()
    q0, s0 = _codes(M, K)
    N_.norm_gated_quant(v, z, w, q0, s0, eps=1e-6)
    ref = hid.clone()
    G.gemm_i8(q0, s0, b, bs, ref, residual=ref, b_z=bz)
    out = hid.clone()
    FU.pro_gemm_i8(FU.Producer.norm_gated(v, z, w, 1e-6), b, bs, out, residual=out, b_z=bz)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M", [1, 4])
def test_rmsnorm_vocab_head_equals_two_calls(M):
    """The final norm + vocab head (engine.py:371-374, 468-470): a wide launch, which
    makes its codes with a producer launch of its own first."""
    FU, G, N_, _ = _k()
    K, N = 2048, 248320
    x, nw = _rms_inputs(M, K, seed=M + 400)
    b, bs = _w8(K, N, 51)
    q0, s0 = _codes(M, K)
    N_.rmsnorm_quant(x, nw, q0, s0, 1e-6)
    ref = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    G.gemm_i8(q0, s0, b, bs, ref, block_n=512, block_k=64)
    out = torch.empty_like(ref)
    FU.pro_gemm_i8(FU.Producer.rmsnorm(x, nw, 1e-6), b, bs, out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M", [1, 4, 16])
def test_fused_against_oracle(M):
    """The fused rmsnorm + proj3 result is within the GEMM tolerance of the oracle's
    fp32 linear on the oracle's codes (sampled columns)."""
    FU, _, _, _ = _k()
    K = 2048
    x, nw = _rms_inputs(M, K, seed=M + 500)
    (w1, s1), (w2, s2) = _w8(K, 6144, 61), _w8(K, 2048, 62)
    out = torch.empty((M, 8192), dtype=torch.bfloat16, device="cuda")
    FU.pro_proj3(FU.Producer.rmsnorm(x, nw, 1e-6), w1, s1, w2, s2, None, None, out)
    qr, sr = R.rmsnorm_quant_ref(x.float().cpu().numpy(), nw.float().cpu().numpy(), 1e-6, True)
    cols = H.sample_cols(6144, 2048)
    ref = R.gemm_i8_ref(qr, sr, w1.cpu().numpy()[:, cols], s1.cpu().numpy()[cols])
    H.assert_out_close(out.cpu()[:, cols], ref)
