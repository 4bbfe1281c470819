"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture (integers exactly, floats to fp32 BLAS
reassociation noise).  GPU: the kernels match every fixture to the parity bar."""
from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch

import helpers as H
from oracle import ref_cpu as R

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def close(a, b, rtol=1e-6):
    return R.max_rel_err(a, b) <= rtol


# ---------------------------------------------------------------- oracle vs fixtures (CPU)

def test_oracle_reproduces_unpack():
    g = load("w4_unpack_all_bytes")
    assert np.array_equal(R.unpack_w4(g["packed"]), g["nib"])


def test_oracle_reproduces_a16():
    g = load("a16_w8")
    assert close(R.linear_w8_ref(g["x"], g["w"], g["s"]), g["y"])
    g = load("a16_w4_g128_zeros")
    assert np.array_equal(R.dequant_w4_f32(g["w"], g["s"], g["z"]), g["dq"])
    assert close(R.linear_w4_ref(g["x"], g["w"], g["s"], g["z"]), g["y"])


def test_oracle_reproduces_engine():
    g = load("engine_gemm_i8_res")
    assert close(R.gemm_i8_ref(g["a_q"], g["a_s"], g["b"], g["b_s"], residual=g["res"]), g["y"])
    g = load("engine_gemm_w4_g64_zeros")
    assert close(R.gemm_w4_ref(g["a_q"], g["a_s"], g["b"], g["b_s"], b_z=g["b_z"]), g["y"])
    g = load("engine_proj3_i8")
    y = R.proj3_ref(g["a_q"], g["a_s"], g["w1"], g["s1"], g["w2"], g["s2"], g["w3"], g["s3"])
    assert close(y, g["y"])
    g = load("engine_gate_up_quant_i8")
    assert close(R.mlp_gate_up_ref(g["a_q"], g["a_s"], g["wg"], g["sg"], g["wu"], g["su"]), g["h"])
    q, qs = R.quant_groups(R.round_bf16(g["h"]))
    assert np.array_equal(q, g["q"]) and np.array_equal(qs, g["qs"])


# ---------------------------------------------------------------- kernels vs fixtures (GPU)

def _t(a, bf16=False):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if bf16:
        t = t.view(torch.int16).view(torch.bfloat16)
    return t.cuda()


@pytest.mark.gpu
def test_kernels_match_a16_fixtures():
    from qwen35_amd.kernels import layout, linear
    g = load("w4_unpack_all_bytes")
    assert np.array_equal(layout.w4_unpack(_t(g["packed"])).cpu().numpy(), g["nib"])
    g = load("a16_w8")
    y = torch.empty((3, 64), dtype=torch.float16, device="cuda")
    linear.linear_w8(_t(g["x"]), _t(g["w"]), _t(g["s"]), y)
    H.assert_out_close(y, g["y"])
    g = load("a16_w4_g128_zeros")
    assert np.array_equal(layout.w4_dequant_f32(_t(g["w"]), _t(g["s"]), _t(g["z"])).cpu().numpy(), g["dq"])
    linear.linear_w4(_t(g["x"]), _t(g["w"]), _t(g["s"]), y, w_zero=_t(g["z"]))
    H.assert_out_close(y, g["y"])


@pytest.mark.gpu
def test_kernels_match_engine_fixtures():
    from qwen35_amd.kernels import gemm
    g = load("engine_gemm_i8_res")
    out = _t(g["res"], bf16=True).clone()
    gemm.gemm_i8(_t(g["a_q"]), _t(g["a_s"]), _t(g["b"]), _t(g["b_s"]), out, residual=out)
    H.assert_out_close(out, g["y"])
    g = load("engine_gemm_w4_g64_zeros")
    out = torch.empty((4, 64), dtype=torch.bfloat16, device="cuda")
    gemm.gemm_i8(_t(g["a_q"]), _t(g["a_s"]), _t(g["b"]), _t(g["b_s"], bf16=True), out, b_z=_t(g["b_z"]))
    H.assert_out_close(out, g["y"])
    g = load("engine_proj3_i8")
    out = torch.empty((3, 128), dtype=torch.bfloat16, device="cuda")
    gemm.proj3(_t(g["a_q"]), _t(g["a_s"]), _t(g["w1"]), _t(g["s1"]), _t(g["w2"]), _t(g["s2"]),
               _t(g["w3"]), _t(g["s3"]), out)
    H.assert_out_close(out, g["y"])
    g = load("engine_gate_up_quant_i8")
    q = torch.empty((3, 128), dtype=torch.int8, device="cuda")
    qs = torch.empty((3, 2), dtype=torch.float32, device="cuda")
    gemm.mlp_gate_up_quant(_t(g["a_q"]), _t(g["a_s"]), _t(g["wg"]), _t(g["sg"]), _t(g["wu"]), _t(g["su"]),
                           q, qs)
    deq = q.cpu().numpy().astype(np.float32) * np.repeat(qs.cpu().numpy(), 64, 1)
    assert R.max_rel_err(deq, g["h"]) <= 1e-2
    assert (q.cpu().numpy() == g["q"]).mean() > 0.99
