"""GPU parity of W4 calls whose weights give zeros only in part (kernels/w4.py
fill_zeros: the reference's rule, kernels/w4.py:235-241 and 309-314, where each missing
zero tensor is the first given one read with the weight's own strides).

Every such call equals the same call with the filled zero tensors passed explicitly,
bit for bit, and the oracle applied to those zeros within the GEMM tolerance:
proj3 and gate/up + requant as single calls (decode rows and a prefill chunk), fused
with their producer, and as engine-chain jobs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

pytestmark = pytest.mark.gpu

K = 2048
ROWS = K // 128  # group-128 zero rows


def _k():
    from qwen35_amd.kernels import echain, fused, gemm
    return echain, fused, gemm


def _w4e(N, seed, zeros):
    packed, s, z = H.w4(K, N, seed, group=128, zeros=zeros)
    return packed.cuda(), s.to(torch.bfloat16).cuda(), (None if z is None else z.cuda())


def _as_grid(fill, n):
    """The [ROWS, n] zeros the reference's kernel reads from `fill` for a weight of n columns."""
    return fill.reshape(-1)[: ROWS * n].view(ROWS, n)


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def _np(t):
    return H.np_(t.cpu()) if t.dtype == torch.bfloat16 else t.cpu().numpy()


@pytest.mark.parametrize("M", [1, 4, 37])
def test_proj3_partial_zeros(M):
    _, _, gemm = _k()
    a, as_ = H.engine_act(M, K, seed=70 + M)
    a, as_ = a.cuda(), as_.cuda()
    w1, s1, z1 = _w4e(4096, 71, "random")
    w2, s2, _ = _w4e(512, 72, "none")
    w3, s3, _ = _w4e(512, 73, "none")
    out = torch.empty((M, 5120), dtype=torch.bfloat16, device="cuda")
    gemm.proj3(a, as_, w1, s1, w2, s2, w3, s3, out, z1=z1)
    z2, z3 = _as_grid(z1, 512), _as_grid(z1, 512)
    exp = torch.empty_like(out)
    gemm.proj3(a, as_, w1, s1, w2, s2, w3, s3, exp, z1=z1, z2=z2.clone(), z3=z3.clone())
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(exp))
    ref = R.proj3_ref(_np(a), _np(as_), _np(w1), _np(s1), _np(w2), _np(s2), _np(w3), _np(s3),
                      _np(z1), _np(z2), _np(z3))
    H.assert_out_close(out, ref)


def test_proj3_zeros_too_small_for_a_missing_grid_are_refused():
    _, _, gemm = _k()
    a, as_ = H.engine_act(1, K, seed=74)
    w1, s1, _ = _w4e(4096, 75, "none")
    w2, s2, z2 = _w4e(512, 76, "random")
    out = torch.zeros((1, 4608), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="cannot stand in"):
        gemm.proj3(a.cuda(), as_.cuda(), w1, s1, w2, s2, None, None, out, z2=z2)
    assert not out.any()


@pytest.mark.parametrize("M", [1, 4, 37])
@pytest.mark.parametrize("given", ["gate", "up"])
def test_gate_up_quant_one_zero_tensor(M, given):
    _, _, gemm = _k()
    N = 6144
    a, as_ = H.engine_act(M, K, seed=80 + M)
    a, as_ = a.cuda(), as_.cuda()
    wg, sg, zg = _w4e(N, 81, "random")
    wu, su, zu = _w4e(N, 82, "random")
    z = zg if given == "gate" else zu
    q1 = torch.empty((M, N), dtype=torch.int8, device="cuda")
    s1 = torch.empty((M, N // 64), dtype=torch.float32, device="cuda")
    gemm.mlp_gate_up_quant(a, as_, wg, sg, wu, su, q1, s1, zg=z if given == "gate" else None,
                           zu=z if given == "up" else None)
    q2, s2 = torch.empty_like(q1), torch.empty_like(s1)
    gemm.mlp_gate_up_quant(a, as_, wg, sg, wu, su, q2, s2, zg=z, zu=z.clone())
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(_bits(s1), _bits(s2))
    qr, sr = R.mlp_gate_up_quant_ref(_np(a), _np(as_), _np(wg), _np(sg), _np(wu), _np(su), _np(z), _np(z))
    deq = q1.cpu().numpy().astype(np.float32) * np.repeat(s1.cpu().numpy(), 64, 1)
    deq_r = qr.astype(np.float32) * np.repeat(sr, 64, 1)
    assert R.max_rel_err(deq, deq_r) <= 1e-2
    assert (q1.cpu().numpy() == qr).mean() > 0.99


@pytest.mark.parametrize("M", [1, 4])
def test_fused_and_chain_partial_zeros(M):
    EC, FU, gemm = _k()
    g = H.gen(90 + M)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
    nw = (torch.rand(K, generator=g) * 0.1 + 0.95).to(torch.bfloat16).cuda()
    w1, s1, z1 = _w4e(6144, 91, "random")
    w2, s2, _ = _w4e(2048, 92, "none")
    wg, sg, zg = _w4e(6144, 93, "random")
    wu, su, _ = _w4e(6144, 94, "none")
    z2 = _as_grid(z1, 2048).clone()
    pro = lambda: FU.Producer.rmsnorm(x, nw, 1e-6)

    exp_p = torch.empty((M, 8192), dtype=torch.bfloat16, device="cuda")
    FU.pro_proj3(pro(), w1, s1, w2, s2, None, None, exp_p, z1=z1, z2=z2)
    out_p = torch.empty_like(exp_p)
    FU.pro_proj3(pro(), w1, s1, w2, s2, None, None, out_p, z1=z1)
    exp_q = torch.empty((M, 6144), dtype=torch.int8, device="cuda")
    exp_s = torch.empty((M, 96), dtype=torch.float32, device="cuda")
    FU.pro_mlp_gate_up_quant(pro(), wg, sg, wu, su, exp_q, exp_s, zg=zg, zu=zg.clone())
    out_q, out_s = torch.empty_like(exp_q), torch.empty_like(exp_s)
    FU.pro_mlp_gate_up_quant(pro(), wg, sg, wu, su, out_q, out_s, zg=zg)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out_p), _bits(exp_p))
    assert torch.equal(out_q, exp_q) and torch.equal(_bits(out_s), _bits(exp_s))

    ch_p = torch.zeros_like(exp_p)
    ch_q, ch_s = torch.zeros_like(exp_q), torch.zeros_like(exp_s)
    ch = EC.EngineChain(M)
    ch.proj3(None, None, w1, s1, w2, s2, None, None, ch_p, z1=z1, pro=pro(), level=0)
    ch.mlp_gate_up_quant(None, None, wg, sg, wu, su, ch_q, ch_s, zg=zg, pro=pro(), level=0)
    ch.build().run()
    torch.cuda.synchronize()
    assert ch.wait_error() == 0
    assert torch.equal(_bits(ch_p), _bits(exp_p))
    assert torch.equal(ch_q, exp_q) and torch.equal(_bits(ch_s), _bits(exp_s))
