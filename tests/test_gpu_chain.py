"""GPU parity of the decode chain (many A16 linears in one persistent launch) against the
CPU oracle: the config-1 and config-4 layer shapes with their vocabulary heads, a
chain whose jobs consume each other's outputs (dependency levels), residuals added in
place, rows independent of M, repeated launches, and HIP-graph replay.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

pytestmark = pytest.mark.gpu

CONFIG1 = [(2048, 2048), (2048, 512), (2048, 512), (2048, 2048), (2048, 6144), (2048, 6144), (6144, 2048),
           (2048, 4096), (4096, 2048)]
CONFIG4 = [(4096, 4096), (4096, 1024), (4096, 1024), (4096, 4096), (4096, 12288), (4096, 12288), (12288, 4096)]


def _chain(M):
    from qwen35_amd.kernels.chain import DecodeChain
    return DecodeChain(M)


def _weights(kind, K, N, seed, zeros="none"):
    if kind == "w8":
        w, s = H.w8(K, N, seed)
        return w, s, None
    return H.w4(K, N, seed, group=128, zeros=zeros)


def _ref(kind, x, w, s, z, cols, residual=None):
    if kind == "w8":
        return H.linear_w8_ref_cols(x, w, s, cols, residual=residual)
    return H.linear_w4_ref_cols(x, w, s, z, cols, residual=residual)


def _cu(t):
    return None if t is None else t.cuda()


@pytest.mark.parametrize("kind,shapes,head_k", [("w8", CONFIG1, 2048), ("w4", CONFIG1, 2048),
                                                ("w4", CONFIG4, 4096)])
@pytest.mark.parametrize("M", [1, 2, 4])
def test_layer_and_head_in_one_launch(kind, shapes, head_k, M):
    """Every linear of one layer plus the vocabulary head as one chain (level 0: the
    sweep's shapes are independent), each output against the oracle."""
    if head_k == 4096 and M == 2:
        pytest.skip("config 4 runs M = 1 and 4")
    xs = {K: H.act_f16(M, K, seed=800 + K + M) for K in {K for K, _ in shapes} | {head_k}}
    ch = _chain(M)
    jobs = []
    for i, (K, N) in enumerate(shapes + [(head_k, 248320)]):
        w, s, z = _weights(kind, K, N, seed=810 + i, zeros="random" if i % 2 else "none")
        out = torch.empty((M, N), dtype=torch.float16, device="cuda")
        ch.add(_cu(xs[K]), _cu(w), _cu(s), out, zero=_cu(z))
        jobs.append((K, N, w, s, z, out))
    ch.build()
    ch.run()
    torch.cuda.synchronize()
    assert ch.wait_error() == 0
    for K, N, w, s, z, out in jobs:
        cols = H.sample_cols(N, 2048, seed=K + N)
        H.assert_out_close(out.cpu()[:, cols], _ref(kind, xs[K], w, s, z, cols))


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_dependent_levels_consume_outputs(kind):
    """x -> A (2048 -> 6144) -> B reads A's output (6144 -> 2048) and adds it in place
    to h, which level 0 also wrote (job C) -> D reads h (2048 -> 2048).  Every job is
    checked against the oracle applied to the GPU's own inputs, so a job that read its
    input before the producer finished would fail."""
    M = 4
    x = H.act_f16(M, 2048, seed=830)
    (wa, sa, za), (wb, sb, zb), (wc, sc, zc), (wd, sd, zd) = (
        _weights(kind, 2048, 6144, 831), _weights(kind, 6144, 2048, 832, zeros="random"),
        _weights(kind, 2048, 2048, 833), _weights(kind, 2048, 2048, 834))
    a = torch.empty((M, 6144), dtype=torch.float16, device="cuda")
    h = torch.empty((M, 2048), dtype=torch.float16, device="cuda")
    d = torch.empty((M, 2048), dtype=torch.float16, device="cuda")
    # scale A's output down so that B's sum stays in fp16 range
    sa = (sa.float() / 64).to(torch.float16) if kind == "w8" else (sa.float() / 64).to(torch.float16)
    ch = _chain(M)
    ch.add(_cu(x), _cu(wa), _cu(sa), a, zero=_cu(za), level=0)
    ch.add(_cu(x), _cu(wc), _cu(sc), h, zero=_cu(zc), level=0)
    ch.add(a, _cu(wb), _cu(sb), h, zero=_cu(zb), residual=h, level=1)
    ch.add(h, _cu(wd), _cu(sd), d, zero=_cu(zd), level=2)
    ch.build()
    for rep in range(2):   # a second launch of the same plan (counters reset)
        ch.run()
        torch.cuda.synchronize()
        assert ch.wait_error() == 0
        all_cols = np.arange(2048)
        ref_a = _ref(kind, x, wa, sa, za, np.arange(6144))
        H.assert_out_close(a.cpu(), ref_a)
        ref_c = _ref(kind, x, wc, sc, zc, all_cols)
        h_c = torch.from_numpy(ref_c).to(torch.float16)      # what C wrote (to the tolerance)
        ref_h = _ref(kind, a.cpu(), wb, sb, zb, all_cols, residual=h_c)
        H.assert_out_close(h.cpu(), ref_h, tol=4e-3)
        H.assert_out_close(d.cpu(), _ref(kind, h.cpu(), wd, sd, zd, all_cols))


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_rows_equal_across_M(kind):
    """Row m of an M = 4 (and 16) chain equals an M = 1 chain of row m, bit for bit."""
    shapes = [(2048, 2048), (6144, 2048), (2048, 6144)]
    ws = [_weights(kind, K, N, 840 + i, zeros="random") for i, (K, N) in enumerate(shapes)]
    X = {K: H.act_f16(16, K, seed=845 + K) for K, _ in shapes}
    res = {}
    for M in (16, 4, 1):
        ch = _chain(M)
        outs = []
        for (K, N), (w, s, z) in zip(shapes, ws):
            o = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            ch.add(X[K][:M].cuda(), _cu(w), _cu(s), o, zero=_cu(z))
            outs.append(o)
        ch.build()
        ch.run()
        torch.cuda.synchronize()
        res[M] = [o.cpu() for o in outs]
    for i in range(len(shapes)):
        assert torch.equal(res[4][i][0], res[1][i][0])
        assert torch.equal(res[16][i][:4], res[4][i])


@pytest.mark.parametrize("M", [1, 4])
def test_w4_explicit_zero_eight_is_identical(M):
    """A W4 job with an explicit zero tensor of all 8s gives the bits of the same job with
    none (z = 8 implied), at M = 1 (per-row group fold) and M = 4 (one-load cycles, one
    row per lane group), whole-K and K-split units."""
    outs = {}
    for zeros in ("none", "eight"):
        ch = _chain(M)
        res = []
        for i, (K, N) in enumerate([(2048, 2048), (6144, 1024)]):
            w, s, z = _weights("w4", K, N, 890 + i, zeros=zeros)
            o = torch.empty((M, N), dtype=torch.float16, device="cuda")
            ch.add(H.act_f16(M, K, seed=895 + i).cuda(), w.cuda(), s.cuda(), o, zero=_cu(z), level=0)
            res.append(o)
        ch.build()
        ch.run()
        torch.cuda.synchronize()
        assert ch.wait_error() == 0
        outs[zeros] = [o.cpu() for o in res]
    for a, b in zip(outs["none"], outs["eight"]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_graph_replay_matches_eager(kind):
    """run() captured in a HIP graph, replayed three times with eager work in between;
    every replay equals the eager launch (M = 2: the one-load activation cycles)."""
    M = 2
    ch = _chain(M)
    outs = []
    for i, (K, N) in enumerate([(2048, 2048), (6144, 2048), (2048, 512)]):
        w, s, z = _weights(kind, K, N, 850 + i, zeros="random" if i == 1 else "none")
        o = torch.empty((M, N), dtype=torch.float16, device="cuda")
        ch.add(H.act_f16(M, K, seed=855 + i).cuda(), w.cuda(), s.cuda(), o, zero=_cu(z), level=0)
        outs.append(o)
    ch.build()
    ch.run()
    torch.cuda.synchronize()
    ref = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            ch.run()
    torch.cuda.synchronize()
    for _ in range(3):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r)
    assert ch.wait_error() == 0


def test_bf16_and_fp32_scales_bf16_outputs_residual():
    """fp32 W8 scales and bf16 W4 scales, bf16 outputs, a residual added in place; a
    chain holds one weight kind (W8 and W4 jobs together are refused)."""
    M = 3
    x = H.act_f16(M, 2048, seed=860)
    w8, s8 = H.w8(2048, 1024, 861)
    p4, s4, z4 = H.w4(2048, 1024, 862, group=128, zeros="random")
    s8f = s8.float()
    s4b = s4.to(torch.bfloat16)
    res = torch.randn((M, 1024), generator=H.gen(863)).to(torch.bfloat16)
    o8 = res.clone().cuda()
    o4 = torch.empty((M, 1024), dtype=torch.bfloat16, device="cuda")
    _chain(M).add(x.cuda(), w8.cuda(), s8f.cuda(), o8, residual=o8).build().run()
    _chain(M).add(x.cuda(), p4.cuda(), s4b.cuda(), o4, zero=z4.cuda()).build().run()
    torch.cuda.synchronize()
    cols = np.arange(1024)
    H.assert_out_close(o8.cpu(), H.linear_w8_ref_cols(x, w8, s8f, cols, residual=res))
    H.assert_out_close(o4.cpu(), H.linear_w4_ref_cols(x, p4, s4b, z4, cols))
    mixed = _chain(M).add(x.cuda(), w8.cuda(), s8f.cuda(), o8).add(x.cuda(), p4.cuda(), s4b.cuda(), o4)
    with pytest.raises(ValueError, match="not both"):
        mixed.build()


def test_bad_levels_rejected():
    from qwen35_amd.kernels.chain import DecodeChain
    M = 1
    w, s = H.w8(2048, 512, 870)
    ch = DecodeChain(M)
    x = H.act_f16(M, 2048, 871).cuda()
    o = torch.empty((M, 512), dtype=torch.float16, device="cuda")
    ch.add(x, w.cuda(), s.cuda(), o, level=0)
    ch.add(x, w.cuda(), s.cuda(), o, level=2)
    with pytest.raises(ValueError, match="level"):
        ch.build()


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("M", [2, 3, 4])
def test_one_load_activation_cycles_same_bits(kind, M, monkeypatch):
    """Chains at M = 2-4 load a ring cycle's activations with one load and permute them
    to the MFMA lanes; QLIN_CHAIN_XC=0 takes one load per step instead.  The same plan
    gives the same bits both ways, W8 and W4 (the K-split job with explicit zeros):
    whole-K units (2048 deep), K-split units (6144 deep) and a dependent level that
    reads a level-0 output, and a K of 2176 whose last split holds waves with no steps.
    Three outputs are also checked against the oracle."""
    shapes = [(2048, 2048), (6144, 2048), (2048, 6144), (2176, 1024)]
    ws = [_weights(kind, K, N, 870 + i, zeros="random" if i == 1 else "none") for i, (K, N) in enumerate(shapes)]
    X = {K: H.act_f16(M, K, seed=875 + K).cuda() for K, _ in shapes}
    outs = [torch.empty((M, N), dtype=torch.float16, device="cuda") for _, N in shapes]
    w4k, s4k, z4k = _weights(kind, 6144, 2048, 879)
    s4k = (s4k.float() / 64).to(torch.float16)
    dep = torch.empty((M, 2048), dtype=torch.float16, device="cuda")
    ch = _chain(M)
    for (K, N), (w, s, z), o in zip(shapes, ws, outs):
        ch.add(X[K], _cu(w), _cu(s), o, zero=_cu(z), level=0)
    ch.add(outs[2], _cu(w4k), _cu(s4k), dep, zero=_cu(z4k), level=1)
    ch.build()
    res = {}
    for xc in ("1", "0"):
        monkeypatch.setenv("QLIN_CHAIN_XC", xc)
        for o in outs + [dep]:
            o.zero_()
        ch.run()
        torch.cuda.synchronize()
        assert ch.wait_error() == 0
        res[xc] = [o.cpu() for o in outs + [dep]]
    for a, b in zip(res["1"], res["0"]):
        assert torch.equal(a, b)
    w0, s0, z0 = ws[0]
    H.assert_out_close(res["1"][0], _ref(kind, X[2048].cpu(), w0, s0, z0, np.arange(2048)))
    w1, s1, z1 = ws[1]
    H.assert_out_close(res["1"][1], _ref(kind, X[6144].cpu(), w1, s1, z1, np.arange(2048)))
    w3, s3, z3 = ws[3]
    H.assert_out_close(res["1"][3], _ref(kind, X[2176].cpu(), w3, s3, z3, np.arange(1024)))
