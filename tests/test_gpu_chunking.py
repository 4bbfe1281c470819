"""Chunk invariance of the engine-signature calls (prefill chunks), under the library's
default dispatch: no plan overrides.

The reference verifies chunked prefill bit-identical to a single-chunk prefill
(ENGINEERING.md:453-455), and its system-prefix reuse relies on it (engine.py:553-570):
a 700-token prompt runs as chunks of 512 + 188 (prefill_chunk = 512,
engine.py:540-545), and a cached prefix ends on a multiple of 32 tokens
(engine.py:567-570).  Every row of a call with at least 5 rows must therefore not
depend on M, on the chunking, or on which kernel family the library picks for that
M.  Calls with 1-8 rows are decode (one sequence, or up to eight best-of rows,
engine.py:392) and run the decode work units, whose rows equal single-row calls
instead (tests/test_gpu_echain.py): a chunk remainder of 1-8 rows agrees with the
unchunked prefill within the GEMM tolerance, not bit for bit (tested below).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

pytestmark = pytest.mark.gpu


def _g():
    from qwen35_amd.kernels import gemm
    return gemm


def _w4(K, N, seed):
    """Engine W4-g128 with explicit zeros: packed nibbles, bf16 scales, uint8 zeros."""
    packed, s, z = H.w4(K, N, seed, group=128, zeros="random")
    return packed, s.to(torch.bfloat16), z


def _weights(kind, K, N, seed):
    if kind == "w8":
        b, s = H.engine_w8(K, N, seed)
        return b, s, None
    return _w4(K, N, seed)


def _cu(t):
    return None if t is None else t.cuda()


# (total rows, chunks): a 700-token prompt in chunks of 512, a 521-token one (its
# remainder of 9 rows the smallest above the decode sizes), and a cached 160-token
# prefix (a multiple of 32) followed by the rest of the prompt
CASES = [(700, ((0, 512), (512, 700))), (521, ((0, 512), (512, 521))), (700, ((0, 160), (160, 700)))]
CASE_IDS = ["512+188", "512+9", "160+540"]


def _run_gemm(a, as_, b, bs, bz, hid, m0, m1):
    gemm = _g()
    h = hid[m0:m1].clone().cuda()
    gemm.gemm_i8(a[m0:m1].contiguous().cuda(), as_[m0:m1].contiguous().cuda(), b.cuda(), bs.cuda(), h,
                 residual=h, b_z=_cu(bz))           # in place, as engine.py:238-240
    return h


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("K,N", [(2048, 2048), (6144, 2048)])
@pytest.mark.parametrize("total,case", CASES, ids=CASE_IDS)
def test_gemm_residual_chunked_equals_whole(kind, K, N, total, case):
    """gemm_i8 / gemm_w4 with the residual in place: the o-projection (2048 -> 2048)
    and the down projection (6144 -> 2048)."""
    a, as_ = H.engine_act(total, K, seed=600 + K)
    b, bs, bz = _weights(kind, K, N, seed=601)
    hid = torch.randn((total, N), generator=H.gen(602)).to(torch.bfloat16)
    whole = _run_gemm(a, as_, b, bs, bz, hid, 0, total)
    parts = torch.cat([_run_gemm(a, as_, b, bs, bz, hid, m0, m1) for m0, m1 in case])
    assert torch.equal(whole, parts)
    # and the whole call is right
    cols = H.sample_cols(N, 256, seed=603)
    hb = H.np_(hid)[:, cols]
    if kind == "w8":
        ref = R.gemm_i8_ref(a.numpy(), as_.numpy(), b.numpy()[:, cols], bs.numpy()[cols], residual=hb)
    else:
        ref = R.gemm_w4_ref(a.numpy(), as_.numpy(), b.numpy()[:, cols], H.np_(bs)[:, cols],
                            bz.numpy()[:, cols], residual=hb)
    H.assert_out_close(whole.cpu()[:, cols], ref)


def _run_proj3(a, as_, ws, m0, m1):
    gemm = _g()
    nt = sum(w[0].shape[1] for w in ws)
    out = torch.empty((m1 - m0, nt), dtype=torch.bfloat16, device="cuda")
    (w1, s1, z1), (w2, s2, z2) = ws
    gemm.proj3(a[m0:m1].contiguous().cuda(), as_[m0:m1].contiguous().cuda(), w1.cuda(), s1.cuda(), w2.cuda(),
               s2.cuda(), None, None, out, z1=_cu(z1), z2=_cu(z2))
    return out


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("total,case", CASES, ids=CASE_IDS)
def test_proj3_chunked_equals_whole(kind, total, case):
    """proj3 as the linear-attention layers call it: lin_qkv (2048 -> 6144) and lin_z
    (2048 -> 2048) into one 8192-column buffer (engine.py:221-226)."""
    K = 2048
    a, as_ = H.engine_act(total, K, seed=610)
    ws = [_weights(kind, K, 6144, seed=611), _weights(kind, K, 2048, seed=612)]
    whole = _run_proj3(a, as_, ws, 0, total)
    parts = torch.cat([_run_proj3(a, as_, ws, m0, m1) for m0, m1 in case])
    assert torch.equal(whole, parts)


def _run_gate_up_quant(a, as_, wg, wu, m0, m1):
    gemm = _g()
    M, N = m1 - m0, wg[0].shape[1]
    q = torch.empty((M, N), dtype=torch.int8, device="cuda")
    s = torch.empty((M, N // 64), dtype=torch.float32, device="cuda")
    gemm.mlp_gate_up_quant(a[m0:m1].contiguous().cuda(), as_[m0:m1].contiguous().cuda(), wg[0].cuda(),
                           wg[1].cuda(), wu[0].cuda(), wu[1].cuda(), q, s, zg=_cu(wg[2]), zu=_cu(wu[2]))
    return q, s


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("total,case", CASES, ids=CASE_IDS)
def test_gate_up_quant_chunked_equals_whole(kind, total, case):
    """mlp_gate_up_quant (2048 -> 6144, engine.py:273-276): int8 codes and scales."""
    K, N = 2048, 6144
    a, as_ = H.engine_act(total, K, seed=620)
    wg, wu = _weights(kind, K, N, seed=621), _weights(kind, K, N, seed=622)
    q, s = _run_gate_up_quant(a, as_, wg, wu, 0, total)
    parts = [_run_gate_up_quant(a, as_, wg, wu, m0, m1) for m0, m1 in case]
    assert torch.equal(q, torch.cat([p[0] for p in parts]))
    assert torch.equal(s, torch.cat([p[1] for p in parts]))


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("K,N", [(2048, 2048), (6144, 2048), (2048, 6144)])
def test_every_row_count_from_9_agrees(kind, K, N):
    """Rows 0-8 of calls with M = 9, 16, 17, 64, 130, 300 and 512 rows are the same
    bits: the 16-row tiles (M <= 16 always, larger M where the time model prefers
    them) and the tiled int8 kernel fold K in one order."""
    gemm = _g()
    Mmax = 512
    a, as_ = H.engine_act(Mmax, K, seed=630 + K + N)
    b, bs, bz = _weights(kind, K, N, seed=631)
    ref = None
    for M in (9, 16, 17, 64, 130, 300, 512):
        out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        gemm.gemm_i8(a[:M].cuda(), as_[:M].cuda(), b.cuda(), bs.cuda(), out, b_z=_cu(bz))
        if ref is None:
            ref = out[:9].clone()
        assert torch.equal(out[:9], ref), f"M={M}"


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("rem", [1, 4, 8])
def test_decode_sized_remainder_within_tolerance(kind, rem):
    """A chunk remainder of 1-8 rows runs the decode work units (so that best-of rows
    equal single rows): its rows agree with the unchunked call within the GEMM
    tolerance, and both agree with the oracle."""
    gemm = _g()
    K, N, total = 2048, 2048, 512 + rem
    a, as_ = H.engine_act(total, K, seed=640 + rem)
    b, bs, bz = _weights(kind, K, N, seed=641)
    whole = torch.empty((total, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), whole, b_z=_cu(bz))
    tail = torch.empty((rem, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a[512:].contiguous().cuda(), as_[512:].contiguous().cuda(), b.cuda(), bs.cuda(), tail,
                 b_z=_cu(bz))
    if kind == "w8":
        ref = R.gemm_i8_ref(a[512:].numpy(), as_[512:].numpy(), b.numpy(), bs.numpy())
    else:
        ref = R.gemm_w4_ref(a[512:].numpy(), as_[512:].numpy(), b.numpy(), H.np_(bs), bz.numpy())
    H.assert_out_close(tail.cpu(), ref)
    H.assert_out_close(whole[512:].cpu(), ref)


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("epi", ["store", "gate_up_quant"])
@pytest.mark.parametrize("M", [17, 200])
def test_families_give_the_same_bits(kind, epi, M, monkeypatch):
    """The tiled int8 kernel and the 16-row tiles, each forced, give identical outputs
    (and the default dispatch picks one of them)."""
    gemm = _g()
    K, N = 2048, 2048
    a, as_ = H.engine_act(M, K, seed=640 + M)
    wg, wu = _weights(kind, K, N, seed=641), _weights(kind, K, N, seed=642)
    hid = torch.randn((M, N), generator=H.gen(643)).to(torch.bfloat16)
    outs = []
    for fam in ("tiled", "skinny", None):
        if fam is None:
            monkeypatch.delenv("QLIN_ENGINE_PREFILL", raising=False)
        else:
            monkeypatch.setenv("QLIN_ENGINE_PREFILL", fam)
        if epi == "store":
            h = hid.clone().cuda()
            gemm.gemm_i8(a.cuda(), as_.cuda(), wg[0].cuda(), wg[1].cuda(), h, residual=h, b_z=_cu(wg[2]))
            outs.append((h,))
        else:
            outs.append(_run_gate_up_quant(a, as_, wg, wu, 0, M))
    for o in outs[1:]:
        for x, y in zip(outs[0], o):
            assert torch.equal(x, y)


def test_down_split_k_rows_beyond_one_workspace_block():
    """A call whose split-K partials would not fit the workspace in one launch (the
    down projection, 4 K splits, 8448 rows: about 264 MB of partial tiles) runs in
    blocks of rows; rows on both sides of a block boundary equal those of a small call
    (rows are independent)."""
    gemm = _g()
    K, N, M = 6144, 2048, 8448
    a, as_ = H.engine_act(M, K, seed=650)
    b, bs = H.engine_w8(K, N, seed=651)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), y)
    for m0 in (0, 8000, 8352):
        yc = torch.empty((96, N), dtype=torch.bfloat16, device="cuda")
        gemm.gemm_i8(a[m0:m0 + 96].contiguous().cuda(), as_[m0:m0 + 96].contiguous().cuda(), b.cuda(), bs.cuda(), yc)
        assert torch.equal(y[m0:m0 + 96], yc)
    cols = H.sample_cols(N, 128, seed=652)
    ref = R.gemm_i8_ref(a.numpy()[::256], as_.numpy()[::256], b.numpy()[:, cols], bs.numpy()[cols])
    H.assert_out_close(y.cpu()[::256][:, cols], ref)
