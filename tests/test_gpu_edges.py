"""GPU parity of engine-signature calls outside the fast kernels' layout rules: any N
and pointers aligned only to their element size, as the reference's masked kernels
take them (kernels/gemm.py:50-57, kernels/w4.py:75-104).  Such calls run on the edge
kernel (csrc/edge.hip).

* Every call kind (gemm_i8 / gemm_w4 with and without a residual, proj3 W8 / W4,
  mlp_gate_up, mlp_gate_up_quant W8 / W4, the fused producer forms) is within the
  GEMM tolerance of the oracle for N not a multiple of 16, and for weights, codes,
  outputs and residuals at addresses off the 16-byte grid.
* Rows do not depend on the batch: rows of a 4-row call equal single-row calls and a
  37-row call equals its 20 + 17 row chunks, bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

pytestmark = pytest.mark.gpu

K = 2048


def _k():
    from qwen35_amd.kernels import fused, gemm, norm, w4
    return fused, gemm, norm, w4


def _off(t, elems):
    """A contiguous copy of t starting `elems` elements past an allocation's start (so
    off the 16-byte grid for elems * itemsize not a multiple of 16)."""
    flat = torch.empty(t.numel() + elems, dtype=t.dtype, device="cuda")
    v = flat[elems:].view(t.shape)
    v.copy_(t.cuda() if not t.is_cuda else t)
    return v


def _w4e(N, seed, zeros="random", group=128):
    packed, s, z = H.w4(K, N, seed, group=group, zeros=zeros)
    return packed, s.to(torch.bfloat16), z


def _np(t):
    if t is None:
        return None
    return H.np_(t.cpu()) if t.dtype == torch.bfloat16 else t.cpu().numpy()


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("N", [1000, 4001])
@pytest.mark.parametrize("M", [1, 4, 37])
@pytest.mark.parametrize("with_res", [False, True])
def test_gemm_i8_any_n(N, M, with_res):
    _, gemm, _, _ = _k()
    a, as_ = H.engine_act(M, K, seed=100 + M)
    b, bs = H.engine_w8(K, N, seed=101)
    res = torch.randn((M, N), generator=H.gen(102)).to(torch.bfloat16) if with_res else None
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out, residual=None if res is None else res.cuda())
    ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy(), bs.numpy(), residual=None if res is None else _np(res))
    H.assert_out_close(out, ref)


@pytest.mark.parametrize("group,zeros", [(128, "random"), (32, "none"), (64, "random")])
@pytest.mark.parametrize("M", [1, 37])
def test_gemm_w4_any_n(group, zeros, M):
    _, gemm, _, _ = _k()
    N = 1000
    a, as_ = H.engine_act(M, K, seed=110 + M)
    packed, s, z = _w4e(N, 111, zeros, group)
    res = torch.randn((M, N), generator=H.gen(112)).to(torch.bfloat16)
    out = res.clone().cuda()
    gemm.gemm_i8(a.cuda(), as_.cuda(), packed.cuda(), s.cuda(), out, residual=out,
                 b_z=None if z is None else z.cuda())
    ref = R.gemm_w4_ref(a.numpy(), as_.numpy(), packed.numpy(), _np(s), _np(z), residual=_np(res))
    H.assert_out_close(out, ref)


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("M", [1, 37])
def test_proj3_any_n(kind, M):
    _, gemm, _, _ = _k()
    a, as_ = H.engine_act(M, K, seed=120 + M)
    ns = (1000, 200, 56)
    if kind == "w8":
        ws = [H.engine_w8(K, n, seed=121 + i) + (None,) for i, n in enumerate(ns)]
    else:
        ws = [_w4e(n, 121 + i) for i, n in enumerate(ns)]
    cu = lambda t: None if t is None else t.cuda()
    out = torch.empty((M, sum(ns)), dtype=torch.bfloat16, device="cuda")
    kw = {} if kind == "w8" else dict(z1=cu(ws[0][2]), z2=cu(ws[1][2]), z3=cu(ws[2][2]))
    gemm.proj3(a.cuda(), as_.cuda(), cu(ws[0][0]), cu(ws[0][1]), cu(ws[1][0]), cu(ws[1][1]), cu(ws[2][0]),
               cu(ws[2][1]), out, **kw)
    ref = R.proj3_ref(a.numpy(), as_.numpy(), *[_np(t) for w in ws for t in w[:2]],
                      *([_np(w[2]) for w in ws] if kind == "w4" else []))
    H.assert_out_close(out, ref)


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_off_grid_pointers(kind):
    """Weights, codes, output and residual each one element past the 16-byte grid."""
    _, gemm, _, _ = _k()
    M, N = 4, 2048
    a, as_ = H.engine_act(M, K, seed=130)
    if kind == "w8":
        b, bs = H.engine_w8(K, N, seed=131)
        z = None
    else:
        b, bs, z = _w4e(N, 131)
    res = torch.randn((M, N), generator=H.gen(132)).to(torch.bfloat16)
    ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), _np(b), _np(bs), residual=_np(res), b_z=_np(z))
    cases = {"weight": dict(b=_off(b, 1)), "codes": dict(a=_off(a, 3)), "out": dict(out=1),
             "residual": dict(res=1), "scale": dict(bs=_off(bs, 1))}
    for what, c in cases.items():
        out = _off(torch.zeros((M, N), dtype=torch.bfloat16), c["out"]) if "out" in c else \
            torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        r = _off(res, c["res"]) if "res" in c else res.cuda()
        gemm.gemm_i8(c.get("a", a.cuda()), as_.cuda(), c.get("b", b.cuda()), c.get("bs", bs.cuda()), out,
                      residual=r, b_z=None if z is None else z.cuda())
        try:
            H.assert_out_close(out, ref)
        except AssertionError as e:
            raise AssertionError(f"{what} off the grid: {e}") from None


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_gate_up_any_n_and_off_grid(kind):
    _, gemm, _, w4 = _k()
    M = 5
    a, as_ = H.engine_act(M, K, seed=140)
    if kind == "w8":
        (wg, sg), (wu, su) = H.engine_w8(K, 1000, seed=141), H.engine_w8(K, 1000, seed=142)
        zg = zu = None
    else:
        wg, sg, zg = _w4e(1000, 141)
        wu, su, zu = _w4e(1000, 142)
    cu = lambda t: None if t is None else t.cuda()
    # bf16 h for N = 1000 (mlp_gate_up has no per-64 groups)
    h = torch.empty((M, 1000), dtype=torch.bfloat16, device="cuda")
    if kind == "w8":
        gemm.mlp_gate_up(cu(a), cu(as_), cu(wg), cu(sg), cu(wu), cu(su), h)
    else:
        w4.mlp_gate_up_w4(cu(a), cu(as_), cu(wg), cu(sg), cu(wu), cu(su), h, zg=cu(zg), zu=cu(zu))
    H.assert_out_close(h, R.mlp_gate_up_ref(a.numpy(), as_.numpy(), _np(wg), _np(sg), _np(wu), _np(su),
                                            _np(zg), _np(zu)))
    # gate/up + requant (N a multiple of 64) with the weights off the grid
    N = 640
    if kind == "w8":
        (wg, sg), (wu, su) = H.engine_w8(K, N, seed=143), H.engine_w8(K, N, seed=144)
    else:
        wg, sg, zg = _w4e(N, 143)
        wu, su, zu = _w4e(N, 144)
    q = torch.empty((M, N), dtype=torch.int8, device="cuda")
    s = torch.empty((M, N // 64), dtype=torch.float32, device="cuda")
    gemm.mlp_gate_up_quant(cu(a), cu(as_), _off(wg, 1), cu(sg), _off(wu, 5), cu(su), q, s, zg=cu(zg), zu=cu(zu))
    qr, sr = R.mlp_gate_up_quant_ref(a.numpy(), as_.numpy(), _np(wg), _np(sg), _np(wu), _np(su), _np(zg), _np(zu))
    deq = q.cpu().numpy().astype(np.float32) * np.repeat(s.cpu().numpy(), 64, 1)
    deq_r = qr.astype(np.float32) * np.repeat(sr, 64, 1)
    assert R.max_rel_err(deq, deq_r) <= 1e-2
    assert (q.cpu().numpy() == qr).mean() > 0.99


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_rows_independent_of_batch(kind):
    _, gemm, _, _ = _k()
    N = 1000
    a, as_ = H.engine_act(37, K, seed=150)
    a, as_ = a.cuda(), as_.cuda()
    if kind == "w8":
        b, bs = H.engine_w8(K, N, seed=151)
        z = None
    else:
        b, bs, z = _w4e(N, 151)
    b, bs, z = b.cuda(), bs.cuda(), None if z is None else z.cuda()

    def run(rows):
        out = torch.empty((rows.stop - rows.start, N), dtype=torch.bfloat16, device="cuda")
        gemm.gemm_i8(a[rows].contiguous(), as_[rows].contiguous(), b, bs, out, b_z=z)
        return out

    full = run(slice(0, 37))
    assert torch.equal(_bits(torch.cat([run(slice(0, 20)), run(slice(20, 37))])), _bits(full))
    four = run(slice(0, 4))
    for m in range(4):
        assert torch.equal(_bits(run(slice(m, m + 1))[0]), _bits(four[m]))


def test_fused_producer_any_n():
    """A fused producer call with N = 1000 equals the standalone producer followed by the
    linear, bit for bit (the producer runs as its own launch before the edge kernel)."""
    fused, gemm, norm, _ = _k()
    M, N = 4, 1000
    g = H.gen(160)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16).cuda()
    nw = (torch.rand(K, generator=g) * 0.1 + 0.95).to(torch.bfloat16).cuda()
    b, bs = H.engine_w8(K, N, seed=161)
    b, bs = b.cuda(), bs.cuda()
    q = torch.empty((M, K), dtype=torch.int8, device="cuda")
    s = torch.empty((M, K // 64), dtype=torch.float32, device="cuda")
    norm.rmsnorm_quant(x, nw, q, s, 1e-6)
    exp = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(q, s, b, bs, exp)
    out = torch.empty_like(exp)
    fused.pro_gemm_i8(fused.Producer.rmsnorm(x, nw, 1e-6), b, bs, out)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(exp))
