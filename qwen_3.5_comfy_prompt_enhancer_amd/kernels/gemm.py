"""INT8-activation quantized GEMMs with the engine's call signatures (drop-in for the
reference's kernels/gemm.py).

Every function keeps the reference signature, dispatches on the weight dtype
(`uint8` packed nibbles -> the W4 path, kernels/gemm.py:15-17), validates shapes,
dtypes, contiguity and device, and launches the hand-written gfx950 kernels of
libqlin.so on the current HIP stream.  The Triton tile keywords (`block_m`,
`block_n`, `block_k`, `group_m`) are accepted and ignored: tiling is chosen by the
library from K and N.  Outputs are written in place and returned, as in the
reference.
"""
from __future__ import annotations

import torch

from . import qlin as C
from .common import GROUP
from .w4 import gemm_w4, mlp_gate_up_quant_w4, mlp_gate_up_w4, proj3_w4

__all__ = ["GROUP", "gemm_i8", "mlp_gate_up", "mlp_gate_up_quant", "proj3"]


def _is_w4(b) -> bool:
    """W4 checkpoints store uint8 packed nibbles; W8 stores int8 + 1-D scales
    (kernels/gemm.py:15-17)."""
    return b.dtype == torch.uint8


def _check_act(a_q, a_s) -> tuple[int, int]:
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


def _check_w8(name, w, s, K):
    if w.dtype != torch.int8 or w.dim() != 2 or w.shape[0] != K:
        raise ValueError(f"{name} must be int8 [K={K}, N]")
    N = w.shape[1]
    if s is None or s.dim() != 1 or s.shape[0] != N:
        raise ValueError(f"scale of {name} must be [N={N}]")
    C.require_contig(name, w)
    C.require_contig(f"scale of {name}", s)
    return N


def _check_out(name, t, M, N, dtype=torch.bfloat16):
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}")
    C.require_rowmajor(name, t)
    if t.shape[0] < M or t.shape[1] < N:
        raise ValueError(f"{name} is {tuple(t.shape)}, need at least [{M}, {N}]")


def gemm_i8(a_q, a_s, b, b_s, out, residual=None, block_m=None, block_n=None, block_k=64,
            group_m=8, b_z=None):
    """out[M,N] (bf16) = (a_q * a_s) @ (b * b_s), optional residual add
    (kernels/gemm.py:60-92).

    `b` is int8 [K,N] with one scale per output column, or uint8 [K//2,N] packed
    int4 with per-group scales (then `b_z` may hold per-group zeros).  `a_s` holds
    one scale per GROUP of K ([M, K//GROUP]).  `residual` may be `out` itself."""
    if _is_w4(b):
        return gemm_w4(a_q, a_s, b, b_s, out, residual=residual, b_z=b_z, block_m=block_m,
                       block_n=block_n, block_k=block_k, group_m=group_m)
    M, K = _check_act(a_q, a_s)
    N = _check_w8("b", b, b_s, K)
    _check_out("out", out, M, N)
    if residual is not None:
        _check_out("residual", residual, M, N)
    C.require_cuda(a_q, a_s, b, b_s, out, residual)
    ws = C.workspace(out.device)
    C.call("qlin_gemm_i8", C.ptr(a_q), C.ptr(a_s), M, K, C.ptr(b), C.ptr(b_s), C.dtype_code(b_s), N,
           C.ptr(out), out.stride(0), C.ptr(residual),
           residual.stride(0) if residual is not None else 0,
           C.ptr(ws), ws.numel(), C.stream_of(out))
    return out


def mlp_gate_up(a_q, a_s, wg, wsg, wu, wsu, out, block_k=64):
    """out[M,N] (bf16) = silu(gate(x)) * up(x) (kernels/gemm.py:140-151)."""
    if _is_w4(wg):
        return mlp_gate_up_w4(a_q, a_s, wg, wsg, wu, wsu, out)
    M, K = _check_act(a_q, a_s)
    N = _check_w8("wg", wg, wsg, K)
    if _check_w8("wu", wu, wsu, K) != N:
        raise ValueError("gate and up must have the same N")
    if wsg.dtype != wsu.dtype:
        raise ValueError("gate and up scales must share a dtype")
    _check_out("out", out, M, N)
    C.require_contig("out", out)
    C.require_cuda(a_q, a_s, wg, wsg, wu, wsu, out)
    ws = C.workspace(out.device)
    C.call("qlin_mlp_gate_up_i8", C.ptr(a_q), C.ptr(a_s), M, K, C.ptr(wg), C.ptr(wsg), C.ptr(wu),
           C.ptr(wsu), C.dtype_code(wsg), N, C.ptr(out), C.ptr(ws), ws.numel(), C.stream_of(out))
    return out


def mlp_gate_up_quant(a_q, a_s, wg, wsg, wu, wsu, out_q, out_s, block_k=64, zg=None, zu=None):
    """Fused gate/up MLP + per-64 int8 quantization of the activation that feeds
    down_proj (kernels/gemm.py:214-231).  Returns (out_q, out_s)."""
    if _is_w4(wg):
        return mlp_gate_up_quant_w4(a_q, a_s, wg, wsg, wu, wsu, out_q, out_s, zg=zg, zu=zu,
                                    block_k=block_k)
    M, K = _check_act(a_q, a_s)
    N = _check_w8("wg", wg, wsg, K)
    if _check_w8("wu", wu, wsu, K) != N:
        raise ValueError("gate and up must have the same N")
    if wsg.dtype != wsu.dtype:
        raise ValueError("gate and up scales must share a dtype")
    _check_quant_out(out_q, out_s, M, N)
    C.require_cuda(a_q, a_s, wg, wsg, wu, wsu, out_q, out_s)
    ws = C.workspace(out_q.device)
    C.call("qlin_mlp_gate_up_quant_i8", C.ptr(a_q), C.ptr(a_s), M, K, C.ptr(wg), C.ptr(wsg),
           C.ptr(wu), C.ptr(wsu), C.dtype_code(wsg), N, C.ptr(out_q), C.ptr(out_s), C.ptr(ws),
           ws.numel(), C.stream_of(out_q))
    return out_q, out_s


def _check_quant_out(out_q, out_s, M, N):
    if N % GROUP != 0:
        raise ValueError(f"N={N} must be a multiple of {GROUP}")
    if out_q.dtype != torch.int8 or tuple(out_q.shape) != (M, N):
        raise ValueError(f"out_q must be int8 [{M}, {N}]")
    if out_s.dtype != torch.float32 or tuple(out_s.shape) != (M, N // GROUP):
        raise ValueError(f"out_s must be float32 [{M}, {N // GROUP}]")
    C.require_contig("out_q", out_q)
    C.require_contig("out_s", out_s)


def proj3(a_q, a_s, w1, s1, w2, s2, w3, s3, out, block_k=64, z1=None, z2=None, z3=None):
    """Three projections sharing (a_q, a_s), written side by side into
    out[:, 0:N1], [N1:N1+N2], [N1+N2:N1+N2+N3] (kernels/gemm.py:290-312).
    `w2`/`w3` may be None."""
    if _is_w4(w1):
        return proj3_w4(a_q, a_s, w1, s1, w2, s2, w3, s3, out, block_k=block_k, z1=z1, z2=z2,
                        z3=z3)
    M, K = _check_act(a_q, a_s)
    ns = []
    for name, w, s in (("w1", w1, s1), ("w2", w2, s2), ("w3", w3, s3)):
        ns.append(0 if w is None else _check_w8(name, w, s, K))
        if w is not None and s.dtype != s1.dtype:
            raise ValueError("all projection scales must share a dtype")
    n1, n2, n3 = ns
    _check_out("out", out, M, n1 + n2 + n3)
    C.require_cuda(a_q, a_s, w1, s1, w2, s2, w3, s3, out)
    ws = C.workspace(out.device)
    C.call("qlin_proj3_i8", C.ptr(a_q), C.ptr(a_s), M, K, C.ptr(w1), C.ptr(s1), n1, C.ptr(w2),
           C.ptr(s2), n2, C.ptr(w3), C.ptr(s3), n3, C.dtype_code(s1), C.ptr(out), out.stride(0),
           C.ptr(ws), ws.numel(), C.stream_of(out))
    return out
