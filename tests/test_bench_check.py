"""The bench's own output check (bench.check_sweep), on the CPU: it accepts outputs that
equal dequantize + fp32 matmul rounded to fp16, and it rejects a planted error in one
column, in the full check of the last layer copy and in the sampled columns of the
other copies and of the head."""
from __future__ import annotations

import importlib.util
import pathlib
import types

import pytest
import torch

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _case(bench, kind, layers=2, M=2):
    gen = torch.Generator().manual_seed(5)
    shapes = [("a", 256, 64), ("b", 128, 128)]
    head = ("h", 256, 512)

    def weights(K, N):
        if kind == "w8":
            w = torch.randint(-127, 128, (K, N), generator=gen, dtype=torch.int8)
            s = ((torch.randn(N, generator=gen) * 0.02).abs() / 127).to(torch.float16)
        else:
            w = torch.randint(0, 256, (K // 2, N), generator=gen, dtype=torch.uint8)
            s = ((torch.randn((K // 128, N), generator=gen) * 0.02).abs() / 7).to(torch.float16)
        return types.SimpleNamespace(w=w, s=s, K=K, N=N)

    lw = [[weights(K, N) for (_, K, N) in shapes] for _ in range(layers)]
    hw = weights(head[1], head[2])
    xs = {M: torch.randn((M, 256), generator=gen).to(torch.float16)}

    def run(w):
        return (xs[M][:, :w.K].float() @ bench.torch_dequant(kind, w.w, w.s)).to(torch.float16)

    outs = {M: [[run(w) for w in layer] for layer in lw]}
    hout = {M: run(hw)}
    return (lw, hw, xs, outs, hout), shapes, head, [M], layers


@pytest.mark.parametrize("kind", ["w8", "w4"])
def test_check_sweep_accepts_correct_outputs(kind):
    bench = _bench()
    ctx, shapes, head, ms, layers = _case(bench, kind)
    r = bench.check_sweep(ctx, kind, shapes, head, ms, layers, max_cols=128, every_layer_cols=32)
    assert r["ok"] and r["max_rel_err"] <= 2.0 ** -11 + 1e-6
    assert r["jobs"] == len(shapes) * layers + 1


@pytest.mark.parametrize("where", ["last_layer", "other_layer", "head"])
def test_check_sweep_rejects_a_planted_error(where):
    bench = _bench()
    ctx, shapes, head, ms, layers = _case(bench, "w4")
    lw, hw, xs, outs, hout = ctx
    M = ms[0]
    if where == "last_layer":
        outs[M][layers - 1][1][0, 7] += 0.5
    elif where == "other_layer":
        outs[M][0][0][:, :] += 0.5       # every column, so any sample sees it
    else:
        hout[M][:, :] *= 1.01
    r = bench.check_sweep(ctx, "w4", shapes, head, ms, layers, max_cols=128, every_layer_cols=32)
    assert not r["ok"]
