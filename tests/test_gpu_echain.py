"""GPU parity of the engine decode chain (`kernels/echain.py`, csrc/echain.hip): the
engine-signature linears between two mixer kernels, with their activation producers,
in one persistent launch.

* A chain of one 2B-class layer's body equals the engine's call sequence (standalone
  producers, then the reference-signature linears; engine.py:236-279, 265-268,
  272-279, 218-226) bit for bit -- hidden state updated in place twice, the gate/up
  codes, the next layer's projections and its kept codes -- for W8 and W4 (g128 with
  zeros), M = 1 and 4, the attention (gate_mul) and linear-attention (norm_gated)
  o-projections; launched again and replayed from a HIP graph.
* Each stage of the chain is within the GEMM tolerance of the oracle applied to that
  stage's inputs, and every producer's codes equal the oracle's bit for bit.
* Rows of an 8-row call (best-of candidates, engine.py:392) equal single-row calls
  bit for bit, for every call kind.
* The engine's per-layer calls captured in a HIP graph on a non-default stream replay
  bit for bit like the eager calls.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

pytestmark = pytest.mark.gpu

K, NI, HD_ATTN, HD_LIN = 2048, 6144, 256, 128
EPS = 1e-6


def _k():
    from qwen35_amd.kernels import echain, fused, gemm, norm, qlin
    return echain, fused, gemm, norm, qlin


def _w4mod():
    from qwen35_amd.kernels import w4
    return w4


def _act(shape, seed, scale=1.0):
    return (torch.randn(shape, generator=H.gen(seed)) * scale).to(torch.bfloat16)


def _codes(M, n):
    return (torch.zeros((M, n), dtype=torch.int8, device="cuda"),
            torch.zeros((M, n // 64), dtype=torch.float32, device="cuda"))


def _w(kind, k, n, seed):
    """(weight, scale, zeros) in the engine layout: W8 int8 [K,N] + fp32 [N]; W4 g128
    packed + bf16 scales + uint8 zeros."""
    if kind == "w8":
        b, s = H.engine_w8(k, n, seed)
        return b.cuda(), s.cuda(), None
    packed, s, z = H.w4(k, n, seed, group=128, zeros="random")
    return packed.cuda(), s.to(torch.bfloat16).cuda(), z.cuda()


class Layer:
    """One 2B-class layer body's weights and inputs (hidden 2048, intermediate 6144;
    the next layer's proj3 is attention q|gate 4096 + k 512 + v 512, or linear
    attention qkv 6144 + z 2048)."""

    def __init__(self, kind, M, mixer, seed=0):
        self.kind, self.M, self.mixer = kind, M, mixer
        self.o = _w(kind, K, K, seed + 1)
        self.g = _w(kind, K, NI, seed + 2)
        self.u = _w(kind, K, NI, seed + 3)
        self.d = _w(kind, NI, K, seed + 4)
        if mixer == "attn":
            self.p = [_w(kind, K, n, seed + 5 + i) for i, n in enumerate((4096, 512, 512))]
        else:
            self.p = [_w(kind, K, n, seed + 5 + i) for i, n in enumerate((6144, 2048))]
        self.np_ = sum(w.shape[1] for w, _, _ in self.p)
        self.hidden = _act((M, K), seed + 10, 1.0).cuda()
        self.post = (torch.randn(K, generator=H.gen(seed + 11)) * 0.1).to(torch.bfloat16).cuda()
        self.inn = (torch.randn(K, generator=H.gen(seed + 12)) * 0.1).to(torch.bfloat16).cuda()
        if mixer == "attn":
            self.aout = _act((M, K), seed + 13, 3.0).cuda()
            self.gates = _act((M, 5120), seed + 14, 4.0).cuda()   # proj: q | gate (4096), k, v
        else:
            self.dout = _act((M, K), seed + 13, 0.5).cuda()
            self.projz = _act((M, 6144 + K), seed + 14, 2.0).cuda()  # z = proj[:, conv_dim:]
            self.lnw = (torch.randn(HD_LIN, generator=H.gen(seed + 15)) * 0.3 + 1.0).to(torch.bfloat16).cuda()

    def o_producer(self, FU, q=None, s=None):
        if self.mixer == "attn":
            return FU.Producer.gate_mul(self.aout, self.gates, hd=HD_ATTN, q=q, s=s)
        return FU.Producer.norm_gated(self.dout, self.projz[:, 6144:], self.lnw, EPS, q=q, s=s)

    def proj_args(self):
        args = []
        for i in range(3):
            if i < len(self.p):
                w, s, _ = self.p[i]
                args += [w, s]
            else:
                args += [None, None]
        zs = [self.p[i][2] if i < len(self.p) else None for i in range(3)]
        return args, zs


def run_calls(L, hidden, xq3, xs3):
    """The engine's call sequence (standalone producers + reference-signature linears).
    Returns (hq, hs, proj)."""
    _, FU, G, N_, _ = _k()
    M = L.M
    q1, s1 = _codes(M, K)
    if L.mixer == "attn":
        N_.gate_mul_quant(L.aout, L.gates, q1, s1, hd=HD_ATTN)
    else:
        N_.norm_gated_quant(L.dout, L.projz[:, 6144:], L.lnw, q1, s1, eps=EPS)
    G.gemm_i8(q1, s1, L.o[0], L.o[1], hidden, residual=hidden, b_z=L.o[2])
    q2, s2 = _codes(M, K)
    N_.rmsnorm_quant(hidden, L.post, q2, s2, EPS)
    hq, hs = _codes(M, NI)
    G.mlp_gate_up_quant(q2, s2, L.g[0], L.g[1], L.u[0], L.u[1], hq, hs, zg=L.g[2], zu=L.u[2])
    G.gemm_i8(hq, hs, L.d[0], L.d[1], hidden, residual=hidden, b_z=L.d[2])
    N_.rmsnorm_quant(hidden, L.inn, xq3, xs3, EPS)
    proj = torch.zeros((M, L.np_), dtype=torch.bfloat16, device="cuda")
    pa, zs = L.proj_args()
    G.proj3(xq3, xs3, *pa, proj, z1=zs[0], z2=zs[1], z3=zs[2])
    return hq, hs, proj


def build_chain(L, hidden, hq, hs, proj, xq3, xs3):
    EC, FU, _, _, _ = _k()
    ch = EC.EngineChain(L.M)
    ch.gemm_i8(None, None, L.o[0], L.o[1], hidden, residual=hidden, b_z=L.o[2], pro=L.o_producer(FU), level=0)
    ch.mlp_gate_up_quant(None, None, L.g[0], L.g[1], L.u[0], L.u[1], hq, hs, zg=L.g[2], zu=L.u[2],
                         pro=FU.Producer.rmsnorm(hidden, L.post, EPS), level=1)
    ch.gemm_i8(hq, hs, L.d[0], L.d[1], hidden, residual=hidden, b_z=L.d[2], level=2)
    pa, zs = L.proj_args()
    ch.proj3(None, None, *pa, proj, z1=zs[0], z2=zs[1], z3=zs[2],
             pro=FU.Producer.rmsnorm(hidden, L.inn, EPS, q=xq3, s=xs3), level=3)
    return ch.build()


def _eq16(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def _eq32(a, b):
    return torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("mixer", ["attn", "lin"])
def test_layer_chain_equals_call_sequence(kind, M, mixer):
    L = Layer(kind, M, mixer, seed=100 * M + (7 if mixer == "lin" else 0))
    h_ref = L.hidden.clone()
    xq_r, xs_r = _codes(M, K)
    hq_r, hs_r, proj_r = run_calls(L, h_ref, xq_r, xs_r)

    h = L.hidden.clone()
    hq, hs = _codes(M, NI)
    proj = torch.zeros((M, L.np_), dtype=torch.bfloat16, device="cuda")
    xq, xs = _codes(M, K)
    ch = build_chain(L, h, hq, hs, proj, xq, xs)
    for rep in range(2):                         # the plan resets itself after a launch
        h.copy_(L.hidden)
        hq.zero_(), proj.zero_(), xq.zero_()
        ch.run()
        torch.cuda.synchronize()
        assert ch.wait_error() == 0
        assert _eq16(h, h_ref), f"hidden differs (launch {rep})"
        assert torch.equal(hq, hq_r) and _eq32(hs, hs_r), f"gate/up codes differ (launch {rep})"
        assert _eq16(proj, proj_r), f"next layer's projections differ (launch {rep})"
        assert torch.equal(xq, xq_r) and _eq32(xs, xs_r), f"kept codes differ (launch {rep})"


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_layer_chain_graph_replay(kind):
    """The chain launch captured in a HIP graph on a non-default stream, replayed three
    times with eager work between the replays: every replay equals the eager launch."""
    EC, FU, _, _, C = _k()
    M = 4
    L = Layer(kind, M, "attn", seed=900)
    h_ref = L.hidden.clone()
    xq_r, xs_r = _codes(M, K)
    hq_r, hs_r, proj_r = run_calls(L, h_ref, xq_r, xs_r)
    h = L.hidden.clone()
    hq, hs = _codes(M, NI)
    proj = torch.zeros((M, L.np_), dtype=torch.bfloat16, device="cuda")
    xq, xs = _codes(M, K)
    ch = build_chain(L, h, hq, hs, proj, xq, xs)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with C.capture(g, stream=s):
        ch.run()
    torch.cuda.synchronize()
    for rep in range(3):
        h.copy_(L.hidden)
        hq.zero_(), proj.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert ch.wait_error() == 0
        assert _eq16(h, h_ref) and torch.equal(hq, hq_r) and _eq32(hs, hs_r) and _eq16(proj, proj_r), \
            f"replay {rep} differs"
        torch.empty(1 << 20, device="cuda").normal_()   # eager work between replays


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("mixer", ["attn", "lin"])
def test_chain_stages_against_oracle(kind, mixer):
    """Every stage of a chain against the oracle applied to that stage's own inputs:
    separate outputs (no in-place residual) and kept codes make each input visible.
    Codes are bit-exact, linears within the GEMM tolerance."""
    EC, FU, _, _, _ = _k()
    M = 4
    L = Layer(kind, M, mixer, seed=300 + (5 if mixer == "lin" else 0))
    h_mid = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
    h_fin = torch.zeros_like(h_mid)
    q1, s1 = _codes(M, K)
    q2, s2 = _codes(M, K)
    hq, hs = _codes(M, NI)
    q3, s3 = _codes(M, K)
    proj = torch.zeros((M, L.np_), dtype=torch.bfloat16, device="cuda")
    ch = EC.EngineChain(M)
    ch.gemm_i8(None, None, L.o[0], L.o[1], h_mid, residual=L.hidden, b_z=L.o[2], pro=L.o_producer(FU, q1, s1))
    ch.mlp_gate_up_quant(None, None, L.g[0], L.g[1], L.u[0], L.u[1], hq, hs, zg=L.g[2], zu=L.u[2],
                         pro=FU.Producer.rmsnorm(h_mid, L.post, EPS, q=q2, s=s2), level=1)
    ch.gemm_i8(hq, hs, L.d[0], L.d[1], h_fin, residual=h_mid, b_z=L.d[2], level=2)
    pa, zs = L.proj_args()
    ch.proj3(None, None, *pa, proj, z1=zs[0], z2=zs[1], z3=zs[2],
             pro=FU.Producer.rmsnorm(h_fin, L.inn, EPS, q=q3, s=s3), level=3)
    ch.build().run()
    torch.cuda.synchronize()
    assert ch.wait_error() == 0

    f = lambda t: t.detach().float().cpu().numpy()
    n = lambda t: None if t is None else t.cpu().numpy()
    sc = lambda t: H.np_(t.cpu())

    def codes_equal(q, s, ref, what):
        assert (q.cpu().numpy() == ref[0]).all(), f"{what}: codes differ from the oracle"
        assert (s.cpu().numpy().view(np.uint32) == ref[1].astype(np.float32).view(np.uint32)).all(), \
            f"{what}: scales differ from the oracle"

    if mixer == "attn":
        codes_equal(q1, s1, R.gate_mul_quant_ref(f(L.aout), f(L.gates), HD_ATTN), "gate_mul_quant")
    else:
        codes_equal(q1, s1, R.norm_gated_quant_ref(f(L.dout), f(L.projz[:, 6144:]), f(L.lnw), EPS),
                    "norm_gated_quant")
    res = H.np_(L.hidden.cpu())
    if kind == "w8":
        ref_o = R.gemm_i8_ref(q1.cpu().numpy(), s1.cpu().numpy(), n(L.o[0]), n(L.o[1]), residual=res)
    else:
        ref_o = R.gemm_w4_ref(q1.cpu().numpy(), s1.cpu().numpy(), n(L.o[0]), sc(L.o[1]), n(L.o[2]), residual=res)
    H.assert_out_close(h_mid.cpu(), ref_o)
    codes_equal(q2, s2, R.rmsnorm_quant_ref(f(h_mid), f(L.post), EPS, True), "rmsnorm_quant (post)")
    if kind == "w8":
        ref_h = R.mlp_gate_up_quant_ref(q2.cpu().numpy(), s2.cpu().numpy(), n(L.g[0]), n(L.g[1]), n(L.u[0]),
                                        n(L.u[1]))
    else:
        ref_h = R.mlp_gate_up_quant_ref(q2.cpu().numpy(), s2.cpu().numpy(), n(L.g[0]), sc(L.g[1]), n(L.u[0]),
                                        sc(L.u[1]), n(L.g[2]), n(L.u[2]))
    # requantized codes: equal except where the bf16 rounding of h differs; the
    # dequantized values within tolerance (as tests/test_gpu_engine.py checks the call)
    y = hq.cpu().numpy().astype(np.float32) * np.repeat(hs.cpu().numpy(), 64, axis=1)
    yr = ref_h[0].astype(np.float32) * np.repeat(ref_h[1], 64, axis=1)
    assert R.max_rel_err(y, yr) <= 1e-2
    assert (hq.cpu().numpy() == ref_h[0]).mean() > 0.99
    res2 = H.np_(h_mid.cpu())
    if kind == "w8":
        ref_d = R.gemm_i8_ref(hq.cpu().numpy(), hs.cpu().numpy(), n(L.d[0]), n(L.d[1]), residual=res2)
    else:
        ref_d = R.gemm_w4_ref(hq.cpu().numpy(), hs.cpu().numpy(), n(L.d[0]), sc(L.d[1]), n(L.d[2]), residual=res2)
    H.assert_out_close(h_fin.cpu(), ref_d)
    codes_equal(q3, s3, R.rmsnorm_quant_ref(f(h_fin), f(L.inn), EPS, True), "rmsnorm_quant (next layer)")
    col = 0
    for w, s, z in L.p:
        nn = w.shape[1]
        if kind == "w8":
            ref_p = R.gemm_i8_ref(q3.cpu().numpy(), s3.cpu().numpy(), n(w), n(s))
        else:
            ref_p = R.gemm_w4_ref(q3.cpu().numpy(), s3.cpu().numpy(), n(w), sc(s), n(z))
        H.assert_out_close(proj.cpu()[:, col:col + nn], ref_p)
        col += nn


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_rows_of_an_8_row_call_equal_single_rows(kind):
    """Best-of decode (engine.py:392 allows B <= 8): every row of an 8-row call equals
    the 1-row call of that row, bit for bit, for gemm (+ residual), proj3 and gate/up +
    quant."""
    _, _, G, _, _ = _k()
    M = 8
    a, as_ = H.engine_act(M, K, seed=71)
    a, as_ = a.cuda(), as_.cuda()
    o = _w(kind, K, 2048, 72)
    res = _act((M, 2048), 73).cuda()
    out = res.clone()
    G.gemm_i8(a, as_, o[0], o[1], out, residual=out, b_z=o[2])
    p1, p2 = _w(kind, K, 4096, 74), _w(kind, K, 1024, 75)
    pr = torch.zeros((M, 5120), dtype=torch.bfloat16, device="cuda")
    G.proj3(a, as_, p1[0], p1[1], p2[0], p2[1], None, None, pr, z1=p1[2], z2=p2[2])
    g, u = _w(kind, K, NI, 76), _w(kind, K, NI, 77)
    hq, hs = _codes(M, NI)
    G.mlp_gate_up_quant(a, as_, g[0], g[1], u[0], u[1], hq, hs, zg=g[2], zu=u[2])
    for m in range(M):
        o1 = res[m:m + 1].clone()
        G.gemm_i8(a[m:m + 1], as_[m:m + 1], o[0], o[1], o1, residual=o1, b_z=o[2])
        pr1 = torch.zeros((1, 5120), dtype=torch.bfloat16, device="cuda")
        G.proj3(a[m:m + 1], as_[m:m + 1], p1[0], p1[1], p2[0], p2[1], None, None, pr1, z1=p1[2], z2=p2[2])
        hq1, hs1 = _codes(1, NI)
        G.mlp_gate_up_quant(a[m:m + 1], as_[m:m + 1], g[0], g[1], u[0], u[1], hq1, hs1, zg=g[2], zu=u[2])
        torch.cuda.synchronize()
        assert _eq16(o1[0], out[m]), f"gemm row {m}"
        assert _eq16(pr1[0], pr[m]), f"proj3 row {m}"
        assert torch.equal(hq1[0], hq[m]) and _eq32(hs1[0], hs[m]), f"gate/up row {m}"


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("M", [5, 8])
def test_decode_rows_5_to_8_against_oracle(kind, M):
    """Calls of 5-8 rows (decode plans) against the oracle: gemm with an in-place
    residual, and the bf16 gate/up epilogue (mlp_gate_up, kernels/gemm.py:140-151)."""
    _, _, G, _, _ = _k()
    a, as_ = H.engine_act(M, 6144, seed=81 + M)
    d = _w(kind, 6144, 2048, 82)
    res = _act((M, 2048), 83)
    out = res.cuda()
    G.gemm_i8(a.cuda(), as_.cuda(), d[0], d[1], out, residual=out, b_z=d[2])
    n = lambda t: None if t is None else t.cpu().numpy()
    if kind == "w8":
        ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), n(d[0]), n(d[1]), residual=H.np_(res))
    else:
        ref = R.gemm_w4_ref(a.numpy(), as_.numpy(), n(d[0]), H.np_(d[1].cpu()), n(d[2]), residual=H.np_(res))
    H.assert_out_close(out.cpu(), ref)
    a2, as2 = H.engine_act(M, K, seed=84 + M)
    g, u = _w(kind, K, 1024, 85), _w(kind, K, 1024, 86)
    h = torch.empty((M, 1024), dtype=torch.bfloat16, device="cuda")
    if kind == "w8":
        G.mlp_gate_up(a2.cuda(), as2.cuda(), g[0], g[1], u[0], u[1], h)
    else:
        _w4mod().mlp_gate_up_w4(a2.cuda(), as2.cuda(), g[0], g[1], u[0], u[1], h, zg=g[2], zu=u[2])
    if kind == "w8":
        ref = R.mlp_gate_up_ref(a2.numpy(), as2.numpy(), n(g[0]), n(g[1]), n(u[0]), n(u[1]))
    else:
        ref = R.mlp_gate_up_ref(a2.numpy(), as2.numpy(), n(g[0]), H.np_(g[1].cpu()), n(u[0]), H.np_(u[1].cpu()),
                                n(g[2]), n(u[2]))
    H.assert_out_close(h.cpu(), ref)


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_head_job_long_units_equals_call(kind):
    """A wide head (K 2048, N 131072: units of the whole K, no split) with the final
    norm as its producer, as a chain job after a down projection, equals the two calls."""
    EC, FU, G, N_, _ = _k()
    M, N = 2, 131072
    a, as_ = H.engine_act(M, NI, seed=91)
    a, as_ = a.cuda(), as_.cuda()
    d = _w(kind, NI, K, 92)
    hw = _w(kind, K, N, 93)
    fin = (torch.randn(K, generator=H.gen(94)) * 0.1).to(torch.bfloat16).cuda()
    hid0 = _act((M, K), 95).cuda()
    h1 = hid0.clone()
    G.gemm_i8(a, as_, d[0], d[1], h1, residual=h1, b_z=d[2])
    q, s = _codes(M, K)
    N_.rmsnorm_quant(h1, fin, q, s, EPS)
    logits_r = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    G.gemm_i8(q, s, hw[0], hw[1], logits_r, b_z=hw[2], block_n=512)
    h2 = hid0.clone()
    logits = torch.empty_like(logits_r)
    ch = EC.EngineChain(M)
    ch.gemm_i8(a, as_, d[0], d[1], h2, residual=h2, b_z=d[2])
    ch.gemm_i8(None, None, hw[0], hw[1], logits, b_z=hw[2], pro=FU.Producer.rmsnorm(h2, fin, EPS), level=1)
    ch.build().run()
    torch.cuda.synchronize()
    assert ch.wait_error() == 0
    assert _eq16(h2, h1) and _eq16(logits, logits_r)


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("M", [1, 4])
def test_engine_calls_graph_capture(kind, M):
    """One layer's engine calls (producers + the four linears) captured in a HIP graph
    with kernels.qlin.capture on a non-default stream: three replays, with eager work
    and synchronizations between them, equal the eager calls bit for bit."""
    _, _, _, _, C = _k()
    L = Layer(kind, M, "attn", seed=700 + M)
    h_ref = L.hidden.clone()
    xq_r, xs_r = _codes(M, K)
    hq_r, hs_r, proj_r = run_calls(L, h_ref, xq_r, xs_r)
    h = L.hidden.clone()
    xq, xs = _codes(M, K)
    out = {}
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with C.capture(g, stream=s):
        out["r"] = run_calls(L, h, xq, xs)
    torch.cuda.synchronize()
    for rep in range(3):
        h.copy_(L.hidden)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        hq, hs, proj = out["r"]
        assert _eq16(h, h_ref) and torch.equal(hq, hq_r) and _eq32(hs, hs_r) and _eq16(proj, proj_r), \
            f"replay {rep} differs"
        assert torch.equal(xq, xq_r) and _eq32(xs, xs_r)
        torch.empty(1 << 20, device="cuda").normal_()


def test_capture_without_workspace_raises():
    """A call under capture on a stream with no workspace raises instead of sharing
    another stream's workspace."""
    _, _, G, _, _ = _k()
    a, as_ = H.engine_act(1, K, seed=5)
    a, as_ = a.cuda(), as_.cuda()
    b, bs, _ = _w("w8", K, 2048, 6)
    out = torch.empty((1, 2048), dtype=torch.bfloat16, device="cuda")
    G.gemm_i8(a, as_, b, bs, out)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="without a workspace"):
        with torch.cuda.graph(g, stream=s):
            G.gemm_i8(a, as_, b, bs, out)
    torch.cuda.synchronize()
