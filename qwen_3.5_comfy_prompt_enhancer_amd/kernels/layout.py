"""GPU unpack / dequant of the engine weight layouts (bit-exactness checks).

These expose the exact values the GEMM kernels consume:

* `w4_unpack(packed)` -> uint8 nibbles [K, N] in natural K order (kernels/w4.py:51-61);
* `w4_dequant_f32(packed, scale, zero=None)` -> fp32 `(nibble - z) * scale[k // G, n]`
  (quant_formats.py:6-8, kernels/w4.py:103-104);
* `w8_dequant_f32(w, scale)` -> fp32 `w * scale[None, :]` (quant_formats.py:9).

and, on the GPU, the load-time producers of those layouts with the reference's
arithmetic and return types:

* `requant_w4_sym(w, group=32)` -> (packed uint8 [K//2, N], bf16 scale [K//group, N])
  (quant_formats.py:253-267);
* `requant_w8_row(w)` -> (int8 [K, N], fp32 scale [N]) (quant_formats.py:270-275);

and the external int4 formats' nibble decode into the engine layout:

* `gptq_w4_to_engine(qweight)`: int32 [K/8, N] -> packed [K/2, N] (quant_formats.py:
  369-372, 411-412);
* `awq_w4_to_engine(qweight)`: int32 [K, N/8] in AWQ order -> packed [K/2, N]
  (quant_formats.py:442-444, 466);
* `gptq_zeros(qzeros, plus_one=True)` / `awq_zeros(qzeros)`: int32 [G, N/8] -> uint8
  [G, N] (quant_formats.py:396-400, 445-446);
* `ct_w4_to_engine(weight_packed, K=None, weight_scale=None)`: compressed-tensors
  symmetric int4, int32 [N, W] -> packed [K/2, N], and its group scales [N, K/G] ->
  [K/G, N] (quant_formats.py:282-354, the native-group branch at 348-350).
"""
from __future__ import annotations

import torch

from . import qlin as C

__all__ = ["w4_unpack", "w4_dequant_f32", "w8_dequant_f32", "requant_w4_sym", "requant_w8_row",
           "gptq_w4_to_engine", "awq_w4_to_engine", "gptq_zeros", "awq_zeros", "ct_w4_to_engine"]


def w4_unpack(packed: torch.Tensor) -> torch.Tensor:
    if packed.dtype != torch.uint8 or packed.dim() != 2:
        raise ValueError("packed must be uint8 [K/2, N]")
    C.require_contig("packed", packed)
    C.require_cuda(packed)
    K, N = packed.shape[0] * 2, packed.shape[1]
    out = torch.empty((K, N), dtype=torch.uint8, device=packed.device)
    C.call("qlin_w4_unpack", C.ptr(packed), K, N, C.ptr(out), C.stream_of(packed))
    return out


def w4_dequant_f32(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor | None = None):
    if packed.dtype != torch.uint8 or packed.dim() != 2:
        raise ValueError("packed must be uint8 [K/2, N]")
    K, N = packed.shape[0] * 2, packed.shape[1]
    if scale.dim() != 2 or scale.shape[1] != N or K % scale.shape[0] != 0:
        raise ValueError("scale must be [K/group, N]")
    group = K // scale.shape[0]
    if zero is not None and (zero.dtype != torch.uint8 or zero.shape != scale.shape):
        raise ValueError("zero must be uint8 shaped like scale")
    for name, t in (("packed", packed), ("scale", scale), ("zero", zero)):
        C.require_contig(name, t)
    C.require_cuda(packed, scale, zero)
    out = torch.empty((K, N), dtype=torch.float32, device=packed.device)
    C.call("qlin_w4_dequant_f32", C.ptr(packed), C.ptr(scale), C.dtype_code(scale), C.ptr(zero),
           group, K, N, C.ptr(out), C.stream_of(packed))
    return out


def w8_dequant_f32(w: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    if w.dtype != torch.int8 or w.dim() != 2 or scale.dim() != 1 or scale.shape[0] != w.shape[1]:
        raise ValueError("w must be int8 [K, N] and scale [N]")
    C.require_contig("w", w)
    C.require_contig("scale", scale)
    C.require_cuda(w, scale)
    K, N = w.shape
    out = torch.empty((K, N), dtype=torch.float32, device=w.device)
    C.call("qlin_w8_dequant_f32", C.ptr(w), C.ptr(scale), C.dtype_code(scale), K, N, C.ptr(out),
           C.stream_of(w))
    return out


def _f32_weights(w: torch.Tensor) -> torch.Tensor:
    if w.dim() != 2 or not w.is_floating_point():
        raise ValueError("w must be a float [K, N] tensor")
    C.require_cuda(w)
    return w.to(torch.float32).contiguous()


def requant_w4_sym(w: torch.Tensor, group: int = 32):
    """float [K, N] -> (packed [K//2, N] uint8, scales [K//group, N] bf16): symmetric
    int4 per (group, column) on the grid [-8, 7] + 8 (quant_formats.py:253-267)."""
    K, N = w.shape
    assert group in (32, 64) and K % group == 0, (K, group)
    w = _f32_weights(w)
    packed = torch.empty((K // 2, N), dtype=torch.uint8, device=w.device)
    scale = torch.empty((K // group, N), dtype=torch.bfloat16, device=w.device)
    C.call("qlin_requant_w4_sym", C.ptr(w), K, N, group, C.ptr(packed), C.ptr(scale), C.stream_of(w))
    return packed, scale


def requant_w8_row(w: torch.Tensor):
    """float [K, N] -> (int8 [K, N], fp32 scale [N]) per-column symmetric
    (quant_formats.py:270-275)."""
    w = _f32_weights(w)
    K, N = w.shape
    q = torch.empty((K, N), dtype=torch.int8, device=w.device)
    scale = torch.empty((N,), dtype=torch.float32, device=w.device)
    C.call("qlin_requant_w8_row", C.ptr(w), K, N, C.ptr(q), C.ptr(scale), C.stream_of(w))
    return q, scale


def _i32_words(name: str, t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.int32 or t.dim() != 2:
        raise ValueError(f"{name} must be an int32 [rows, words] tensor")
    C.require_contig(name, t)
    C.require_cuda(t)
    return t


def gptq_w4_to_engine(qweight: torch.Tensor) -> torch.Tensor:
    """GPTQ int4 qweight int32 [K/8, N] -> engine packed uint8 [K/2, N]."""
    qweight = _i32_words("qweight", qweight)
    K, N = qweight.shape[0] * 8, qweight.shape[1]
    packed = torch.empty((K // 2, N), dtype=torch.uint8, device=qweight.device)
    C.call("qlin_w4_repack_gptq", C.ptr(qweight), K, N, C.ptr(packed), C.stream_of(qweight))
    return packed


def awq_w4_to_engine(qweight: torch.Tensor) -> torch.Tensor:
    """AWQ int4 qweight int32 [K, N/8] (AWQ nibble order) -> engine packed uint8 [K/2, N]."""
    qweight = _i32_words("qweight", qweight)
    K, N = qweight.shape[0], qweight.shape[1] * 8
    packed = torch.empty((K // 2, N), dtype=torch.uint8, device=qweight.device)
    C.call("qlin_w4_repack_awq", C.ptr(qweight), K, N, C.ptr(packed), C.stream_of(qweight))
    return packed


def _zeros(qzeros: torch.Tensor, awq: int, add: int) -> torch.Tensor:
    qzeros = _i32_words("qzeros", qzeros)
    G, N = qzeros.shape[0], qzeros.shape[1] * 8
    z = torch.empty((G, N), dtype=torch.uint8, device=qzeros.device)
    C.call("qlin_w4_zeros_unpack", C.ptr(qzeros), G, N, awq, add, C.ptr(z), C.stream_of(qzeros))
    return z


def gptq_zeros(qzeros: torch.Tensor, plus_one: bool = True) -> torch.Tensor:
    """GPTQ qzeros int32 [G, N/8] -> uint8 zeros [G, N] (+1: the effective zero)."""
    return _zeros(qzeros, 0, 1 if plus_one else 0)


def awq_zeros(qzeros: torch.Tensor) -> torch.Tensor:
    """AWQ qzeros int32 [G, N/8] (AWQ nibble order) -> uint8 zeros [G, N]."""
    return _zeros(qzeros, 1, 0)


def ct_w4_to_engine(weight_packed: torch.Tensor, K: int | None = None, weight_scale: torch.Tensor | None = None):
    """compressed-tensors pack-quantized symmetric int4 -> the engine W4 layout.

    `weight_packed` int32 [N, W] (8 K-nibbles per word, straight order; one output
    feature per row), `K` the input features (default 8 W; `weight_shape` of the
    checkpoint).  Returns packed uint8 [K/2, N] (the value of a nibble is nibble - 8:
    zero point 8, the engine's default), and, if `weight_scale` [N, K/G] is given, the
    scales transposed to [K/G, N] as `decode_ct` returns them (quant_formats.py:350)."""
    weight_packed = _i32_words("weight_packed", weight_packed)
    N, W = weight_packed.shape
    K = 8 * W if K is None else int(K)
    packed = torch.empty((K // 2, N), dtype=torch.uint8, device=weight_packed.device)
    C.call("qlin_w4_repack_ct", C.ptr(weight_packed), N, W, K, C.ptr(packed), C.stream_of(weight_packed))
    if weight_scale is None:
        return packed
    if weight_scale.dim() != 2 or weight_scale.shape[0] != N:
        raise ValueError(f"weight_scale must be [N={N}, K/G]")
    return packed, weight_scale.t().contiguous()
