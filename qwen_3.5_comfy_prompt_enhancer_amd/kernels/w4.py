"""W4 (packed int4, group-scaled) GEMMs with the engine's call signatures (drop-in for
the reference's kernels/w4.py).

Layout (kernels/w4.py:3-11, quant_formats.py:6-8):

* `W`  -- uint8 [K//2, N]; byte (j, n) holds k = 2j in the low nibble and k = 2j+1 in
  the high nibble;
* `WS` -- bf16 / fp16 / fp32 [K//WGRP, N], one scale per WGRP-element group along K;
* `Z`  -- optional uint8 [K//WGRP, N], one real zero per group; a stored element
  decodes to `nibble - z`, and the symmetric grid is z = 8.

WGRP = K // WS.shape[0] (kernels/w4.py:155) may be 32, 64 or any multiple of 64.  The
gfx950 kernels turn the nibbles into int8 `16 * (nibble - 8)` in registers and run
exact int8 MFMA dot products per sub-block of min(WGRP, 64) K values; explicit zeros
add the exact integer correction `(8 - z) * sum(a_q)`.  The per-sub-block fp32
epilogue is the reference's `acc * (a_s * w_s)` (kernels/w4.py:103-104).
"""
from __future__ import annotations

import torch

from . import qlin as C
from .common import GROUP

__all__ = ["gemm_w4", "proj3_w4", "mlp_gate_up_quant_w4", "mlp_gate_up_w4"]


def _check_act(a_q, a_s):
    if a_q.dtype != torch.int8 or a_q.dim() != 2:
        raise ValueError("a_q must be int8 [M, K]")
    M, K = a_q.shape
    if K % GROUP != 0:
        raise ValueError(f"K={K} must be a multiple of {GROUP}")
    if a_s.dtype != torch.float32 or tuple(a_s.shape) != (M, K // GROUP):
        raise ValueError(f"a_s must be float32 [M, K/{GROUP}] = [{M}, {K // GROUP}]")
    C.require_contig("a_q", a_q)
    C.require_contig("a_s", a_s)
    return M, K


def _check_w4(name, w, s, z, K, group=None):
    """Validates one packed weight; returns (N, group)."""
    if w.dtype != torch.uint8 or w.dim() != 2 or w.shape[0] * 2 != K:
        raise ValueError(f"{name} must be uint8 [K/2={K // 2}, N]")
    N = w.shape[1]
    if s is None or s.dim() != 2 or s.shape[1] != N or s.shape[0] == 0:
        raise ValueError(f"scale of {name} must be [K/group, N={N}]")
    g = K // s.shape[0]
    if g * s.shape[0] != K:
        raise ValueError(f"scale rows of {name} do not divide K={K}")
    if group is not None and g != group:
        raise ValueError("all weights of one call must share the weight group")
    if z is not None:
        if z.dtype != torch.uint8 or tuple(z.shape) != tuple(s.shape):
            raise ValueError(f"zeros of {name} must be uint8 {tuple(s.shape)}")
        C.require_contig(f"zeros of {name}", z)
    C.require_contig(name, w)
    C.require_contig(f"scale of {name}", s)
    return N, g


def fill_zeros(zs, scales, fill):
    """The zero tensors a multi-weight call passes on when its weights give zeros only
    in part: the reference then runs its kernel with zeros for every weight, and a
    weight without its own reads the memory of `fill` (the first given zero tensor)
    with its own [K/group, N] strides (kernels/w4.py:235-241 and 309-314 pass `fill`
    in place of each missing one; _w4_acc indexes it by the weight's row stride,
    kernels/w4.py:82-83).  `scales[i]` is weight i's scale tensor (its shape is the
    zero shape), None for an absent weight.  All given or all None: returned as is.
    A weight whose zero grid needs more elements than `fill` holds is refused (the
    reference would read past the end of `fill`)."""
    if fill is None or all(z is not None for z, s in zip(zs, scales) if s is not None):
        return list(zs)
    if fill.dtype != torch.uint8:
        raise ValueError("zeros must be uint8")
    C.require_contig("zeros", fill)
    flat = fill.reshape(-1)
    out = []
    for z, s in zip(zs, scales):
        if z is None and s is not None:
            rows, n = s.shape
            if flat.numel() < rows * n:
                raise ValueError(f"the given zeros ({flat.numel()} elements) cannot stand in for a "
                                 f"missing [{rows}, {n}] zero grid")
            z = flat[: rows * n].view(rows, n)
        out.append(z)
    return out


def _check_out(name, t, M, N, dtype=torch.bfloat16):
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}")
    C.require_rowmajor(name, t)
    if t.shape[0] < M or t.shape[1] < N:
        raise ValueError(f"{name} is {tuple(t.shape)}, need at least [{M}, {N}]")


def gemm_w4(a_q, a_s, b, b_s, out, residual=None, b_z=None, block_m=None, block_n=None,
            block_k=64, group_m=8, num_warps=None, num_stages=3):
    """out[M,N] (bf16) = (a_q * a_s) @ ((unpack(b) - z) * b_s), optional residual add
    (kernels/w4.py:139-166)."""
    M, K = _check_act(a_q, a_s)
    N, group = _check_w4("b", b, b_s, b_z, K)
    _check_out("out", out, M, N)
    if residual is not None:
        _check_out("residual", residual, M, N)
    C.require_cuda(a_q, a_s, b, b_s, b_z, out, residual)
    ws = C.workspace(out.device)
    C.call("qlin_gemm_w4", C.ptr(a_q), C.ptr(a_s), M, K, C.ptr(b), C.ptr(b_s), C.dtype_code(b_s),
           C.ptr(b_z), group, N, C.ptr(out), out.stride(0), C.ptr(residual),
           residual.stride(0) if residual is not None else 0, C.ptr(ws), ws.numel(),
           C.stream_of(out))
    return out


def proj3_w4(a_q, a_s, w1, s1, w2, s2, w3, s3, out, z1=None, z2=None, z3=None, block_k=64):
    """Three W4 projections sharing one activation tile; per-projection group zeros
    (kernels/w4.py:220-251).  Zeros given for only some projections follow the
    reference's fill rule (fill_zeros)."""
    M, K = _check_act(a_q, a_s)
    z1, z2, z3 = fill_zeros((z1, z2, z3), (s1, s2 if w2 is not None else None, s3 if w3 is not None else None),
                            next((z for z in (z1, z2, z3) if z is not None), None))
    ns = []
    group = None
    for name, w, s, z in (("w1", w1, s1, z1), ("w2", w2, s2, z2), ("w3", w3, s3, z3)):
        if w is None:
            ns.append(0)
            continue
        n, group = _check_w4(name, w, s, z, K, group)
        if s.dtype != s1.dtype:
            raise ValueError("all projection scales must share a dtype")
        ns.append(n)
    n1, n2, n3 = ns
    _check_out("out", out, M, n1 + n2 + n3)
    C.require_cuda(a_q, a_s, w1, s1, z1, w2, s2, z2, w3, s3, z3, out)
    ws = C.workspace(out.device)
    C.call("qlin_proj3_w4", C.ptr(a_q), C.ptr(a_s), M, K,
           C.ptr(w1), C.ptr(s1), C.ptr(z1), n1,
           C.ptr(w2), C.ptr(s2), C.ptr(z2), n2,
           C.ptr(w3), C.ptr(s3), C.ptr(z3), n3,
           C.dtype_code(s1), group, C.ptr(out), out.stride(0), C.ptr(ws), ws.numel(),
           C.stream_of(out))
    return out


def _gate_up_common(a_q, a_s, wg, sg, wu, su, zg, zu):
    M, K = _check_act(a_q, a_s)
    N, group = _check_w4("wg", wg, sg, zg, K)
    Nu, _ = _check_w4("wu", wu, su, zu, K, group)
    if Nu != N:
        raise ValueError("gate and up must have the same N")
    if sg.dtype != su.dtype:
        raise ValueError("gate and up scales must share a dtype")
    return M, K, N, group


def mlp_gate_up_quant_w4(a_q, a_s, wg, sg, wu, su, out_q, out_s, zg=None, zu=None, block_k=64):
    """W4 gate/up fusion + per-64 int8 quantization; `zg`/`zu` optional per-group
    zeros ([K//WGRP, N]) (kernels/w4.py:300-323); one of them alone stands in for
    the other (fill_zeros).  Returns (out_q, out_s)."""
    zg, zu = fill_zeros((zg, zu), (sg, su), zg if zg is not None else zu)
    M, K, N, group = _gate_up_common(a_q, a_s, wg, sg, wu, su, zg, zu)
    if N % GROUP != 0:
        raise ValueError(f"N={N} must be a multiple of {GROUP}")
    if out_q.dtype != torch.int8 or tuple(out_q.shape) != (M, N):
        raise ValueError(f"out_q must be int8 [{M}, {N}]")
    if out_s.dtype != torch.float32 or tuple(out_s.shape) != (M, N // GROUP):
        raise ValueError(f"out_s must be float32 [{M}, {N // GROUP}]")
    C.require_contig("out_q", out_q)
    C.require_contig("out_s", out_s)
    C.require_cuda(a_q, a_s, wg, sg, zg, wu, su, zu, out_q, out_s)
    ws = C.workspace(out_q.device)
    C.call("qlin_mlp_gate_up_quant_w4", C.ptr(a_q), C.ptr(a_s), M, K, C.ptr(wg), C.ptr(sg),
           C.ptr(zg), C.ptr(wu), C.ptr(su), C.ptr(zu), C.dtype_code(sg), group, N, C.ptr(out_q),
           C.ptr(out_s), C.ptr(ws), ws.numel(), C.stream_of(out_q))
    return out_q, out_s


def mlp_gate_up_w4(a_q, a_s, wg, sg, wu, su, out, zg=None, zu=None):
    """bf16 silu(gate) * up with W4 weights.  The reference's `mlp_gate_up`
    (kernels/gemm.py:140-151) is W8 only; this W4 form lets the fused quant epilogue
    be checked against the unfused composition (.dev/test_fused.py:22-46).  Zeros
    as mlp_gate_up_quant_w4."""
    zg, zu = fill_zeros((zg, zu), (sg, su), zg if zg is not None else zu)
    M, K, N, group = _gate_up_common(a_q, a_s, wg, sg, wu, su, zg, zu)
    if out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N):
        raise ValueError(f"out must be bf16 [{M}, {N}]")
    C.require_contig("out", out)
    C.require_cuda(a_q, a_s, wg, sg, zg, wu, su, zu, out)
    ws = C.workspace(out.device)
    C.call("qlin_mlp_gate_up_w4", C.ptr(a_q), C.ptr(a_s), M, K, C.ptr(wg), C.ptr(sg), C.ptr(zg),
           C.ptr(wu), C.ptr(su), C.ptr(zu), C.dtype_code(sg), group, N, C.ptr(out), C.ptr(ws),
           ws.numel(), C.stream_of(out))
    return out
