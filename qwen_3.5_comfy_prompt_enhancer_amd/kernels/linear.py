"""A16 weight-only quantized linears: fp16 activations, engine-layout weights.

The reference computes this form on its CPU path -- dequantize through the layouts
of quant_formats.py (quant_formats.py:6-9), then an fp32 matmul.  These functions
are the gfx950 counterpart and read the same packed layouts as the engine kernels:

* `linear_w8`: `out = x @ (w * scale[None, :])`, `w` int8 [K, N], `scale` [N];
* `linear_w4`: `out = x @ ((nibble - z) * scale[k // group, n])`, `w` uint8
  [K//2, N] (even k in the low nibble), `scale` [K//group, N], `zero` uint8
  [K//group, N] or None (z = 8).

`x` is fp16 [M, K] (row stride may exceed K); `out` / `residual` are fp16 or bf16
[M, N] row-major.  Weights are converted to fp16 exactly in registers and
multiplied on MFMA with fp32 accumulation.  W8 column scales multiply the fp32
result.  W4 group scales are applied in fp32 per group for M <= 16; for M > 16 (the
tiled prefill kernel) each group scale, times 2^8, is folded into the fp16 weight
values (one fp16 rounding; exact range for scales in [2^-22, 17]) and the result is
multiplied by 2^-8 in fp32.
"""
from __future__ import annotations

import torch

from . import qlin as C

__all__ = ["linear_w8", "linear_w4", "linear"]


def _check_x(x):
    if x.dtype != torch.float16 or x.dim() != 2:
        raise ValueError("x must be float16 [M, K]")
    C.require_rowmajor("x", x)
    return x.shape


def _check_out(name, t, M, N):
    if t.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"{name} must be float16 or bfloat16")
    C.require_rowmajor(name, t)
    if t.shape[0] < M or t.shape[1] < N:
        raise ValueError(f"{name} is {tuple(t.shape)}, need at least [{M}, {N}]")


def linear_w8(x, w, w_scale, out, residual=None):
    """out[M,N] = x @ (w * w_scale) (+ residual)."""
    M, K = _check_x(x)
    if w.dtype != torch.int8 or w.dim() != 2 or w.shape[0] != K:
        raise ValueError(f"w must be int8 [K={K}, N]")
    N = w.shape[1]
    if w_scale.dim() != 1 or w_scale.shape[0] != N:
        raise ValueError(f"w_scale must be [N={N}]")
    C.require_contig("w", w)
    C.require_contig("w_scale", w_scale)
    _check_out("out", out, M, N)
    if residual is not None:
        _check_out("residual", residual, M, N)
        if residual.dtype != out.dtype:
            raise ValueError("residual must have the dtype of out")
    C.require_cuda(x, w, w_scale, out, residual)
    ws = C.workspace(out.device)
    C.call("qlin_linear_w8", C.ptr(x), C.QLIN_F16, M, K, x.stride(0), C.ptr(w), C.ptr(w_scale),
           C.dtype_code(w_scale), N, C.ptr(out), C.dtype_code(out), out.stride(0), C.ptr(residual),
           residual.stride(0) if residual is not None else 0, C.ptr(ws), ws.numel(),
           C.stream_of(out))
    return out


def linear_w4(x, w_packed, w_scale, out, w_zero=None, group=None, residual=None):
    """out[M,N] = x @ ((nibble - z) * w_scale[k // group]) (+ residual)."""
    M, K = _check_x(x)
    if w_packed.dtype != torch.uint8 or w_packed.dim() != 2 or w_packed.shape[0] * 2 != K:
        raise ValueError(f"w_packed must be uint8 [K/2={K // 2}, N]")
    N = w_packed.shape[1]
    if w_scale.dim() != 2 or w_scale.shape[1] != N or w_scale.shape[0] == 0:
        raise ValueError(f"w_scale must be [K/group, N={N}]")
    g = K // w_scale.shape[0]
    if g * w_scale.shape[0] != K or (group is not None and group != g):
        raise ValueError(f"w_scale rows {w_scale.shape[0]} do not match K={K} / group={group}")
    if w_zero is not None:
        if w_zero.dtype != torch.uint8 or tuple(w_zero.shape) != tuple(w_scale.shape):
            raise ValueError(f"w_zero must be uint8 {tuple(w_scale.shape)}")
        C.require_contig("w_zero", w_zero)
    C.require_contig("w_packed", w_packed)
    C.require_contig("w_scale", w_scale)
    _check_out("out", out, M, N)
    if residual is not None:
        _check_out("residual", residual, M, N)
        if residual.dtype != out.dtype:
            raise ValueError("residual must have the dtype of out")
    C.require_cuda(x, w_packed, w_scale, w_zero, out, residual)
    ws = C.workspace(out.device)
    C.call("qlin_linear_w4", C.ptr(x), C.QLIN_F16, M, K, x.stride(0), C.ptr(w_packed),
           C.ptr(w_scale), C.dtype_code(w_scale), C.ptr(w_zero), g, N, C.ptr(out),
           C.dtype_code(out), out.stride(0), C.ptr(residual),
           residual.stride(0) if residual is not None else 0, C.ptr(ws), ws.numel(),
           C.stream_of(out))
    return out


def linear(x, w, w_scale, out, w_zero=None, residual=None):
    """Dispatch on the weight dtype: uint8 packed nibbles -> `linear_w4`, int8 ->
    `linear_w8` (the engine's rule, kernels/gemm.py:15-17)."""
    if w.dtype == torch.uint8:
        return linear_w4(x, w, w_scale, out, w_zero=w_zero, residual=residual)
    return linear_w8(x, w, w_scale, out, residual=residual)
