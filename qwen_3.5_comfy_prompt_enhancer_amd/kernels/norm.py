"""Activation producers of the engine path with the reference's call signatures
(drop-in for rmsnorm_quant / gate_mul_quant / norm_gated_quant of the reference's
kernels/norm.py).

Each turns 16-bit activations into what every engine-signature linear consumes: int8
codes `q [M, K]` and one fp32 scale per 64 columns `s [M, K/64]`, with
`s = max(amax / 127, 1e-8)` and `q = round_half_away(y / s)` (kernels/norm.py:15-25).
The gfx950 kernels fix the arithmetic operation by operation (fp32 without fused
multiply-add, sums of squares in a fixed lane order, rsqrt as 1/sqrt, exp by
Cody-Waite reduction and a degree-7 Taylor polynomial), so the codes of a row are
the same whichever launch makes them -- these standalone calls, or the prologue of
the fused linears in `kernels/fused.py`.
"""
from __future__ import annotations

import torch

from . import qlin as C
from .common import GROUP

__all__ = ["rmsnorm_quant", "gate_mul_quant", "norm_gated_quant", "QLIN_PRO_RMSNORM",
           "QLIN_PRO_GATE_MUL", "QLIN_PRO_NORM_GATED"]

QLIN_PRO_RMSNORM = 1
QLIN_PRO_GATE_MUL = 2
QLIN_PRO_NORM_GATED = 3

_ACT_DT = (torch.bfloat16, torch.float16)


def check_codes(q, s, M, K):
    """q int8 [M, K] and s float32 [M, K/64], both contiguous."""
    if K % GROUP != 0:
        raise ValueError(f"K={K} must be a multiple of {GROUP}")
    if q.dtype != torch.int8 or tuple(q.shape) != (M, K):
        raise ValueError(f"q must be int8 [{M}, {K}]")
    if s.dtype != torch.float32 or tuple(s.shape) != (M, K // GROUP):
        raise ValueError(f"s must be float32 [{M}, {K // GROUP}]")
    C.require_contig("q", q)
    C.require_contig("s", s)


def check_act16(name, t):
    if t.dtype not in _ACT_DT:
        raise ValueError(f"{name} must be bfloat16 or float16")
    C.require_rowmajor(name, t)


def rmsnorm_quant(x, w, q, s, eps=1e-6, one_plus=True):
    """`y = x * rsqrt(mean(x^2) + eps) * (w + 1 if one_plus else w)`, quantized per 64
    columns into q / s (kernels/norm.py:48-57).  x: bf16/fp16 [M, K] (the row stride
    may differ), w: [K], q: int8 [M, K], s: fp32 [M, K/64].  Returns (q, s)."""
    M, K = q.shape
    check_codes(q, s, M, K)
    check_act16("x", x)
    if x.shape[0] < M or x.shape[1] < K:
        raise ValueError(f"x is {tuple(x.shape)}, need [{M}, {K}]")
    if w.dim() != 1 or w.shape[0] != K:
        raise ValueError(f"w must be [{K}]")
    C.require_contig("w", w)
    C.require_cuda(x, w, q, s)
    C.call("qlin_rmsnorm_quant", C.ptr(x), x.stride(0), C.dtype_code(x), C.ptr(w), C.dtype_code(w), M, K,
           float(eps), 1 if one_plus else 0, C.ptr(q), C.ptr(s), C.stream_of(q))
    return q, s


def gate_mul_quant(a, g, q, s, hd=256):
    """`y = a * sigmoid(g[gate])` with g laid out as [M, heads, 2 * hd] (each head's
    gates in its second half), quantized per 64 columns (kernels/norm.py:182-188).
    a: [M, N] contiguous, g: [M, >= 2 N] with its own row stride.  Returns (q, s)."""
    M, N = a.shape
    check_codes(q, s, M, N)
    check_act16("a", a)
    C.require_contig("a", a)
    check_act16("g", g)
    if g.dtype != a.dtype:
        raise ValueError("a and g must share a dtype")
    if g.shape[0] < M or g.shape[1] < 2 * N:
        raise ValueError(f"g is {tuple(g.shape)}, need [{M}, {2 * N}]")
    C.require_cuda(a, g, q, s)
    C.call("qlin_gate_mul_quant", C.ptr(a), a.stride(0), C.ptr(g), g.stride(0), C.dtype_code(a), M, N,
           int(hd), C.ptr(q), C.ptr(s), C.stream_of(q))
    return q, s


def norm_gated_quant(v, z, w, q, s, eps=1e-6):
    """Per (row, head) gated RMSNorm `bf16(v * rsqrt(mean_head(v^2) + eps) * w *
    silu(z))`, quantized per 64 columns (kernels/norm.py:127-137).  v: [T, NV*HD]
    contiguous, z: [T, NV*HD] gate columns (its own row stride), w: [HD].
    Returns (q, s)."""
    T, N = v.shape
    check_codes(q, s, T, N)
    check_act16("v", v)
    C.require_contig("v", v)
    check_act16("z", z)
    if z.dtype != v.dtype:
        raise ValueError("v and z must share a dtype")
    if z.shape[0] < T or z.shape[1] < N:
        raise ValueError(f"z is {tuple(z.shape)}, need [{T}, {N}]")
    if w.dim() != 1:
        raise ValueError("w must be 1-D [HD]")
    C.require_contig("w", w)
    C.require_cuda(v, z, w, q, s)
    C.call("qlin_norm_gated_quant", C.ptr(v), C.ptr(z), z.stride(0), C.dtype_code(v), C.ptr(w),
           C.dtype_code(w), T, N, w.shape[0], float(eps), C.ptr(q), C.ptr(s), C.stream_of(q))
    return q, s
