"""Replay of the engine's quantized-linear call sites into a Workspace-shaped buffer set.

The reference's engine calls the three imported functions from its layer bodies
(engine.py:218-279): per linear-attention layer `proj3(lin_qkv, lin_z)` into the wide
`ws.proj` buffer and `gemm_i8(lin_out)` added in place into `ws.hidden`; per
attention layer `proj3(q, k, v)` and `gemm_i8(o)` in place; per layer the MLP
`mlp_gate_up_quant` into `ws.hq / ws.hs` followed by `gemm_i8(down)` in place; then
the vocabulary head `gemm_i8(..., block_n=512, block_k=64)` of `_final_logits` on the
single-row buffers `xq1 / xs1 / logits` (engine.py:465-471) and of `forward_batch` on
the row buffers with a fresh `[B, V]` output (engine.py:371-374).

Buffers follow the reference Workspace (engine.py:28-66) for the 2B-class config
(hidden 2048, intermediate 6144, 16 linear-attention value heads of 128, 8 query heads
of 256, 2 KV heads): `ws.proj` is `[cap, 8192]` so the attention proj3 (5120 columns)
writes a prefix of a wider row.  Weights are stacked per layer kind as weights.py
stores them (weights.py:297-309): W8 `[n, K, N]` int8 with fp32 `[n, N]` scales; W4
`[n, K/2, N]` with bf16 `[n, K/G, N]` scales and uint8 zeros; the W4 vocab head is
group 64 with no zeros (weights.py:437-460).  The activations the norm kernels would
produce (outside this path) are the oracle's per-64 quantization of seeded rows.
Every call is checked against the oracle on the GPU's own inputs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

pytestmark = pytest.mark.gpu

HID, INTER, V = 2048, 6144, 248320
CONV, VD = 6144, 2048          # 2 * 16 * 128 + 16 * 128, 16 * 128
NQHD, KVD = 2048, 512          # 8 * 256, 2 * 256
PROJ_W = max(CONV + VD, NQHD * 2 + 2 * KVD)


def _g():
    from qwen35_amd.kernels import gemm
    return gemm


class Workspace:
    """The buffers of the reference Workspace that the linear calls touch."""

    def __init__(self, cap):
        d = dict(device="cuda")
        self.hidden = torch.empty((cap, HID), dtype=torch.bfloat16, **d)
        self.xq = torch.empty((cap, HID), dtype=torch.int8, **d)
        self.xs = torch.empty((cap, HID // 64), dtype=torch.float32, **d)
        self.proj = torch.full((cap, PROJ_W), 3.0, dtype=torch.bfloat16, **d)
        self.aq_o = torch.empty((cap, NQHD), dtype=torch.int8, **d)
        self.as_o = torch.empty((cap, NQHD // 64), dtype=torch.float32, **d)
        self.hq = torch.empty((cap, INTER), dtype=torch.int8, **d)
        self.hs = torch.empty((cap, INTER // 64), dtype=torch.float32, **d)
        self.logits = torch.empty((1, V), dtype=torch.bfloat16, **d)
        self.xq1 = torch.empty((1, HID), dtype=torch.int8, **d)
        self.xs1 = torch.empty((1, HID // 64), dtype=torch.float32, **d)

    def view(self, T):
        v = Workspace.__new__(Workspace)
        for k, t in vars(self).items():
            v.__dict__[k] = t if k in ("logits", "xq1", "xs1") else t[:T]
        return v


def _stack(kind, n, K, N, seed, group=128, zeros=True):
    """Stacked per-layer weights in weights.py's layout; returns (w, s, z) tensors on
    the GPU (z None for W8)."""
    g = H.gen(seed)
    if kind == "w8":
        w = torch.randint(-127, 128, (n, K, N), generator=g, dtype=torch.int8)
        s = torch.rand((n, N), generator=g) * 0.002
        return w.cuda(), s.cuda(), None
    w = torch.randint(0, 256, (n, K // 2, N), generator=g, dtype=torch.uint8)
    s = ((torch.rand((n, K // group, N), generator=g) + 0.1) * 0.003).to(torch.bfloat16)
    z = torch.randint(0, 16, (n, K // group, N), generator=g, dtype=torch.uint8) if zeros else None
    return w.cuda(), s.cuda(), (None if z is None else z.cuda())


def _np(t):
    return None if t is None else H.np_(t.cpu())


def _fill_act(q_buf, s_buf, T, seed):
    """What an activation producer writes: per-64 int8 quantization of seeded rows."""
    h = torch.randn((T, q_buf.shape[1]), generator=H.gen(seed)).numpy() * 0.7
    q, s = R.quant_groups(h)
    q_buf[:T].copy_(torch.from_numpy(q))
    s_buf[:T].copy_(torch.from_numpy(s))


def _check_gemm(kind, out, a_q, a_s, w, s, z, residual=None, cols=None):
    a_q, a_s = _np(a_q), _np(a_s)
    w, s, z = _np(w), _np(s), _np(z)
    if cols is not None:
        w, s = w[:, cols], (s[cols] if s.ndim == 1 else s[:, cols])
        z = None if z is None else z[:, cols]
        residual = None if residual is None else residual[:, cols]
    ref = (R.gemm_i8_ref(a_q, a_s, w, s, residual=residual) if kind == "w8"
           else R.gemm_w4_ref(a_q, a_s, w, s, z, residual=residual))
    y = out.cpu() if cols is None else out.cpu()[:, cols]
    H.assert_out_close(y, ref)


def _layer_weights(kind):
    return {
        "lin_qkv": _stack(kind, 2, HID, CONV, 1), "lin_z": _stack(kind, 2, HID, VD, 2),
        "lin_out": _stack(kind, 2, VD, HID, 3),
        "attn_q": _stack(kind, 2, HID, NQHD * 2, 4), "attn_k": _stack(kind, 2, HID, KVD, 5),
        "attn_v": _stack(kind, 2, HID, KVD, 6), "attn_o": _stack(kind, 2, NQHD, HID, 7),
        "mlp_gate": _stack(kind, 2, HID, INTER, 8), "mlp_up": _stack(kind, 2, HID, INTER, 9),
        "mlp_down": _stack(kind, 2, INTER, HID, 10),
    }


def _w(Wd, role, i):
    w, s, z = Wd[role]
    return w[i], s[i], (None if z is None else z[i])


@pytest.mark.parametrize("kind", ["w8", "w4"])
@pytest.mark.parametrize("T", [1, 4, 64])
def test_layer_call_sites(kind, T):
    """A linear-attention layer and an attention layer, each followed by the MLP, at
    decode rows (T = 1, best-of T = 4) and a prefill chunk of 64 rows; layer index 1
    of each stacked weight (a view at an offset), residuals in place."""
    gemm = _g()
    Wd = _layer_weights(kind)
    has_z = kind == "w4"
    ws0 = Workspace(64)
    ws = ws0.view(T)
    hid0 = torch.randn((T, HID), generator=H.gen(20)).to(torch.bfloat16)
    ws.hidden.copy_(hid0)
    li = fi = 1

    # _linear_layer (engine.py:218-242): proj3 into the wide proj buffer
    _fill_act(ws.xq, ws.xs, T, 21)
    (w1, s1, z1), (w2, s2, z2) = _w(Wd, "lin_qkv", li), _w(Wd, "lin_z", li)
    gemm.proj3(ws.xq, ws.xs, w1, s1, w2, s2, None, None, ws.proj, block_k=64,
               z1=z1 if has_z else None, z2=z2 if has_z else None)
    ref = R.proj3_ref(_np(ws.xq), _np(ws.xs), _np(w1), _np(s1), _np(w2), _np(s2), None, None, _np(z1), _np(z2))
    H.assert_out_close(ws.proj.cpu()[:, :CONV + VD], ref)
    # gemm_i8(lin_out) added in place into hidden
    _fill_act(ws.aq_o, ws.as_o, T, 22)
    w, s, z = _w(Wd, "lin_out", li)
    before = _np(ws.hidden)
    gemm.gemm_i8(ws.aq_o, ws.as_o, w, s, ws.hidden, residual=ws.hidden, b_z=z if has_z else None)
    _check_gemm(kind, ws.hidden, ws.aq_o, ws.as_o, w, s, z, residual=before)

    # _mlp (engine.py:266-279): gate/up + requant, then down in place (down reads the
    # GPU's own int8 codes)
    def mlp(i, seed):
        _fill_act(ws.xq, ws.xs, T, seed)
        (wg, sg, zg), (wu, su, zu) = _w(Wd, "mlp_gate", i), _w(Wd, "mlp_up", i)
        gemm.mlp_gate_up_quant(ws.xq, ws.xs, wg, sg, wu, su, ws.hq, ws.hs, zg=zg if has_z else None,
                               zu=zu if has_z else None)
        qr, sr = R.mlp_gate_up_quant_ref(_np(ws.xq), _np(ws.xs), _np(wg), _np(sg), _np(wu), _np(su), _np(zg),
                                         _np(zu))
        deq = ws.hq.cpu().numpy().astype(np.float32) * np.repeat(ws.hs.cpu().numpy(), 64, 1)
        assert R.max_rel_err(deq, qr.astype(np.float32) * np.repeat(sr, 64, 1)) <= 1e-2
        w, s, z = _w(Wd, "mlp_down", i)
        before = _np(ws.hidden)
        gemm.gemm_i8(ws.hq, ws.hs, w, s, ws.hidden, residual=ws.hidden, b_z=z if has_z else None)
        _check_gemm(kind, ws.hidden, ws.hq, ws.hs, w, s, z, residual=before)

    mlp(0, 23)

    # _attn_layer (engine.py:244-268): q (with gate) / k / v into the prefix of proj
    _fill_act(ws.xq, ws.xs, T, 24)
    (q, sq, zq), (k, sk, zk), (v, sv, zv) = (_w(Wd, "attn_q", fi), _w(Wd, "attn_k", fi), _w(Wd, "attn_v", fi))
    ws.proj.fill_(3.0)
    gemm.proj3(ws.xq, ws.xs, q, sq, k, sk, v, sv, ws.proj, block_k=64, z1=zq if has_z else None,
               z2=zk if has_z else None, z3=zv if has_z else None)
    ref = R.proj3_ref(_np(ws.xq), _np(ws.xs), _np(q), _np(sq), _np(k), _np(sk), _np(v), _np(sv), _np(zq),
                      _np(zk), _np(zv))
    nt = NQHD * 2 + 2 * KVD
    H.assert_out_close(ws.proj.cpu()[:, :nt], ref)
    assert bool((ws.proj.cpu()[:, nt:] == 3.0).all())     # the rest of the row untouched
    _fill_act(ws.aq_o, ws.as_o, T, 25)
    w, s, z = _w(Wd, "attn_o", fi)
    before = _np(ws.hidden)
    gemm.gemm_i8(ws.aq_o, ws.as_o, w, s, ws.hidden, residual=ws.hidden, b_z=z if has_z else None)
    _check_gemm(kind, ws.hidden, ws.aq_o, ws.as_o, w, s, z, residual=before)
    mlp(1, 26)


def _head(kind):
    """weights.py:437-477: W8 int8 [H, V] + fp32 [V]; W4 nibbles [H/2, V] + bf16
    group-64 scales [H/64, V], no zeros."""
    if kind == "w8":
        w, s, _ = _stack("w8", 1, HID, V, 30)
        return w[0], s[0]
    w, s, _ = _stack("w4", 1, HID, V, 30, group=64, zeros=False)
    return w[0], s[0]


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_final_logits_and_batch_head(kind):
    """_final_logits (last row through xq1 / xs1 into ws.logits [1, V]) and
    forward_batch's head (B = 4 rows into a fresh [B, V]), with the call's tile
    keywords; sampled vocabulary columns and the last 512 against the oracle."""
    gemm = _g()
    head_w, head_s = _head(kind)
    ws = Workspace(64).view(4)
    cols = np.concatenate([H.sample_cols(V - 512, 4096, seed=31), np.arange(V - 512, V)])
    # _final_logits
    _fill_act(ws.xq1, ws.xs1, 1, 32)
    gemm.gemm_i8(ws.xq1, ws.xs1, head_w, head_s, ws.logits, block_n=512, block_k=64)
    _check_gemm(kind, ws.logits, ws.xq1, ws.xs1, head_w, head_s, None, cols=cols)
    # forward_batch: B rows
    B = 4
    _fill_act(ws.xq, ws.xs, B, 33)
    out = torch.empty((B, V), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(ws.xq, ws.xs, head_w, head_s, out, block_n=512, block_k=64)
    _check_gemm(kind, out, ws.xq, ws.xs, head_w, head_s, None, cols=cols)
    # row 0 of the batch equals a single-row call on the same codes (I1)
    one = torch.empty((1, V), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(ws.xq[:1], ws.xs[:1], head_w, head_s, one, block_n=512, block_k=64)
    assert torch.equal(one[0], out[0])
