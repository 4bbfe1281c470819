"""Engine-signature linears that make their own int8 activations.

The reference's engine runs every linear as two launches: an activation producer
(kernels/norm.py: rmsnorm_quant, gate_mul_quant, norm_gated_quant) writes int8 codes
and per-64 scales, then the linear (kernels/gemm.py / w4.py) reads them back
(engine.py:220-226, 236-240, 265-268, 272-276, 371-374).  Here one call does both:

    pro = Producer.rmsnorm(ws.hidden, w["in_norm"][i], eps, q=ws.xq, s=ws.xs)
    pro_proj3(pro, wq, sq, wk, sk, wv, sv, ws.proj)      # == rmsnorm_quant + proj3

Decode-shaped launches make the codes of their rows and K range in a prologue, while
their first weight loads are in flight; wide launches (the vocab head) and prefill's
tiled kernel run the producer as a launch of its own first.  Either way the result
equals the two-call sequence bit for bit.  `q` / `s` are optional: given, the codes
are written there too (the engine's gate_proj reads ws.xq / ws.xs, engine.py:227);
omitted, they are not kept.  The producer's inputs must not overlap the output.
"""
from __future__ import annotations

import ctypes

import torch

from . import qlin as C
from .gemm import _check_out, _check_quant_out, _check_w8
from .norm import (QLIN_PRO_GATE_MUL, QLIN_PRO_NORM_GATED, QLIN_PRO_RMSNORM, check_act16,
                   check_codes)
from .w4 import _check_w4, fill_zeros

__all__ = ["Producer", "pro_gemm_i8", "pro_proj3", "pro_mlp_gate_up_quant"]


class _CProducer(ctypes.Structure):
    """include/qlin.h qlin_producer."""
    _fields_ = [
        ("kind", ctypes.c_int),
        ("x", ctypes.c_void_p), ("ldx", ctypes.c_int64), ("x_dtype", ctypes.c_int),
        ("g", ctypes.c_void_p), ("ldg", ctypes.c_int64),
        ("w", ctypes.c_void_p), ("w_dtype", ctypes.c_int),
        ("hd", ctypes.c_int), ("one_plus", ctypes.c_int), ("eps", ctypes.c_float),
        ("q", ctypes.c_void_p), ("s", ctypes.c_void_p),
    ]


_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_S = ctypes.c_size_t
_PRO = ctypes.POINTER(_CProducer)

_SIGS = {
    "qlin_pro_gemm_i8": [_PRO, _I, _I, _P, _P, _I, _I, _P, _L, _P, _L, _P, _S, _P],
    "qlin_pro_gemm_w4": [_PRO, _I, _I, _P, _P, _I, _P, _I, _I, _P, _L, _P, _L, _P, _S, _P],
    "qlin_pro_proj3_i8": [_PRO, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P, _I, _I, _P, _L, _P, _S, _P],
    "qlin_pro_proj3_w4": [_PRO, _I, _I, _P, _P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _P, _L,
                          _P, _S, _P],
    "qlin_pro_mlp_gate_up_quant_i8": [_PRO, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P, _P, _S, _P],
    "qlin_pro_mlp_gate_up_quant_w4": [_PRO, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _S,
                                      _P],
}
EXPORTS = tuple(_SIGS)


def _fn(name):
    L = C.lib()
    f = getattr(L, name)
    if getattr(f, "_qlin_bound", False) is False:
        f.restype = ctypes.c_int
        f.argtypes = _SIGS[name]
        f._qlin_bound = True
    return f


class Producer:
    """One activation producer (kernels/norm.py) for the pro_* linears.  Use the
    constructors; `rows` is M and `cols` the K the producer makes."""

    def __init__(self, kind, x, g, w, hd, one_plus, eps, q, s, rows, cols):
        self.kind, self.x, self.g, self.w = kind, x, g, w
        self.hd, self.one_plus, self.eps = hd, one_plus, eps
        self.q, self.s = q, s
        self.rows, self.cols = rows, cols
        if (q is None) != (s is None):
            raise ValueError("give both q and s, or neither")
        if q is not None:
            check_codes(q, s, rows, cols)

    @classmethod
    def rmsnorm(cls, x, w, eps=1e-6, one_plus=True, q=None, s=None):
        """rmsnorm_quant(x, w, q, s, eps, one_plus) (kernels/norm.py:48-57): x [M, K]
        bf16/fp16 (row stride may differ), w [K]."""
        check_act16("x", x)
        if w.dim() != 1 or w.shape[0] > x.shape[1]:
            raise ValueError("w must be [K] with K <= x.shape[1]")
        C.require_contig("w", w)
        return cls(QLIN_PRO_RMSNORM, x, None, w, 0, one_plus, eps, q, s, x.shape[0], w.shape[0])

    @classmethod
    def gate_mul(cls, a, g, hd=256, q=None, s=None):
        """gate_mul_quant(a, g, q, s, hd) (kernels/norm.py:182-188): a [M, N]
        contiguous, g [M, >= 2 N] gate rows."""
        check_act16("a", a)
        C.require_contig("a", a)
        check_act16("g", g)
        if g.dtype != a.dtype or g.shape[0] < a.shape[0] or g.shape[1] < 2 * a.shape[1]:
            raise ValueError(f"g must be {a.dtype} [{a.shape[0]}, >= {2 * a.shape[1]}]")
        return cls(QLIN_PRO_GATE_MUL, a, g, None, hd, False, 0.0, q, s, a.shape[0], a.shape[1])

    @classmethod
    def norm_gated(cls, v, z, w, eps=1e-6, q=None, s=None):
        """norm_gated_quant(v, z, w, q, s, eps) (kernels/norm.py:127-137): v [T, NV*HD]
        contiguous, z [T, NV*HD] (own row stride), w [HD]."""
        check_act16("v", v)
        C.require_contig("v", v)
        check_act16("z", z)
        if z.dtype != v.dtype or z.shape[0] < v.shape[0] or z.shape[1] < v.shape[1]:
            raise ValueError(f"z must be {v.dtype} covering v's shape {tuple(v.shape)}")
        if w.dim() != 1:
            raise ValueError("w must be [HD]")
        C.require_contig("w", w)
        return cls(QLIN_PRO_NORM_GATED, v, z, w, w.shape[0], False, eps, q, s, v.shape[0], v.shape[1])

    def tensors(self):
        return (self.x, self.g, self.w, self.q, self.s)

    def c_struct(self) -> _CProducer:
        p = _CProducer()
        p.kind = self.kind
        p.x = self.x.data_ptr()
        p.ldx = self.x.stride(0)
        p.x_dtype = C.dtype_code(self.x)
        p.g = self.g.data_ptr() if self.g is not None else None
        p.ldg = self.g.stride(0) if self.g is not None else 0
        p.w = self.w.data_ptr() if self.w is not None else None
        p.w_dtype = C.dtype_code(self.w) if self.w is not None else 0
        p.hd = int(self.hd)
        p.one_plus = 1 if self.one_plus else 0
        p.eps = float(self.eps)
        p.q = self.q.data_ptr() if self.q is not None else None
        p.s = self.s.data_ptr() if self.s is not None else None
        return p


def _is_w4(b) -> bool:
    return b.dtype == torch.uint8


def pro_gemm_i8(pro: Producer, b, b_s, out, residual=None, b_z=None):
    """The producer, then gemm_i8(q, s, b, b_s, out, residual, b_z=b_z)
    (kernels/gemm.py:60-92, kernels/w4.py:139-166), in one call."""
    M, K = pro.rows, pro.cols
    if _is_w4(b):
        N, grp = _check_w4("b", b, b_s, b_z, K)
    else:
        if b_z is not None:
            raise ValueError("b_z applies to W4 weights only")
        N = _check_w8("b", b, b_s, K)
    _check_out("out", out, M, N)
    if residual is not None:
        _check_out("residual", residual, M, N)
    C.require_cuda(*pro.tensors(), b, b_s, b_z, out, residual)
    ws = C.workspace(out.device)
    p = pro.c_struct()
    ldr = residual.stride(0) if residual is not None else 0
    if _is_w4(b):
        st = _fn("qlin_pro_gemm_w4")(ctypes.byref(p), M, K, C.ptr(b), C.ptr(b_s), C.dtype_code(b_s), C.ptr(b_z),
                                     grp, N, C.ptr(out), out.stride(0), C.ptr(residual), ldr, C.ptr(ws),
                                     ws.numel(), C.stream_of(out))
        C.check(st, "qlin_pro_gemm_w4")
    else:
        st = _fn("qlin_pro_gemm_i8")(ctypes.byref(p), M, K, C.ptr(b), C.ptr(b_s), C.dtype_code(b_s), N,
                                     C.ptr(out), out.stride(0), C.ptr(residual), ldr, C.ptr(ws), ws.numel(),
                                     C.stream_of(out))
        C.check(st, "qlin_pro_gemm_i8")
    return out


def pro_proj3(pro: Producer, w1, s1, w2, s2, w3, s3, out, z1=None, z2=None, z3=None):
    """The producer, then proj3(q, s, w1, s1, w2, s2, w3, s3, out, z1=.., z2=.., z3=..)
    (kernels/gemm.py:290-312, kernels/w4.py:220-251), in one call."""
    M, K = pro.rows, pro.cols
    p = pro.c_struct()
    if _is_w4(w1):
        z1, z2, z3 = fill_zeros((z1, z2, z3), (s1, s2 if w2 is not None else None, s3 if w3 is not None else None),
                                next((z for z in (z1, z2, z3) if z is not None), None))
        ns, grp = [], None
        for name, w, s, z in (("w1", w1, s1, z1), ("w2", w2, s2, z2), ("w3", w3, s3, z3)):
            if w is None:
                ns.append(0)
                continue
            n, grp = _check_w4(name, w, s, z, K, grp)
            if s.dtype != s1.dtype:
                raise ValueError("all projection scales must share a dtype")
            ns.append(n)
        n1, n2, n3 = ns
        _check_out("out", out, M, n1 + n2 + n3)
        C.require_cuda(*pro.tensors(), w1, s1, w2, s2, w3, s3, z1, z2, z3, out)
        ws = C.workspace(out.device)
        st = _fn("qlin_pro_proj3_w4")(ctypes.byref(p), M, K, C.ptr(w1), C.ptr(s1), C.ptr(z1), n1, C.ptr(w2),
                                      C.ptr(s2), C.ptr(z2), n2, C.ptr(w3), C.ptr(s3), C.ptr(z3), n3,
                                      C.dtype_code(s1), grp, C.ptr(out), out.stride(0), C.ptr(ws), ws.numel(),
                                      C.stream_of(out))
        C.check(st, "qlin_pro_proj3_w4")
        return out
    ns = []
    for name, w, s in (("w1", w1, s1), ("w2", w2, s2), ("w3", w3, s3)):
        ns.append(0 if w is None else _check_w8(name, w, s, K))
        if w is not None and s.dtype != s1.dtype:
            raise ValueError("all projection scales must share a dtype")
    n1, n2, n3 = ns
    _check_out("out", out, M, n1 + n2 + n3)
    C.require_cuda(*pro.tensors(), w1, s1, w2, s2, w3, s3, out)
    ws = C.workspace(out.device)
    st = _fn("qlin_pro_proj3_i8")(ctypes.byref(p), M, K, C.ptr(w1), C.ptr(s1), n1, C.ptr(w2), C.ptr(s2), n2,
                                  C.ptr(w3), C.ptr(s3), n3, C.dtype_code(s1), C.ptr(out), out.stride(0),
                                  C.ptr(ws), ws.numel(), C.stream_of(out))
    C.check(st, "qlin_pro_proj3_i8")
    return out


def pro_mlp_gate_up_quant(pro: Producer, wg, wsg, wu, wsu, out_q, out_s, zg=None, zu=None):
    """The producer, then mlp_gate_up_quant(q, s, wg, wsg, wu, wsu, out_q, out_s, zg=..,
    zu=..) (kernels/gemm.py:214-231, kernels/w4.py:300-323), in one call.  Returns
    (out_q, out_s)."""
    M, K = pro.rows, pro.cols
    p = pro.c_struct()
    if wsg.dtype != wsu.dtype:
        raise ValueError("gate and up scales must share a dtype")
    if _is_w4(wg):
        zg, zu = fill_zeros((zg, zu), (wsg, wsu), zg if zg is not None else zu)
        N, grp = _check_w4("wg", wg, wsg, zg, K)
        if _check_w4("wu", wu, wsu, zu, K, grp)[0] != N:
            raise ValueError("gate and up must have the same N")
        _check_quant_out(out_q, out_s, M, N)
        C.require_cuda(*pro.tensors(), wg, wsg, wu, wsu, zg, zu, out_q, out_s)
        ws = C.workspace(out_q.device)
        st = _fn("qlin_pro_mlp_gate_up_quant_w4")(ctypes.byref(p), M, K, C.ptr(wg), C.ptr(wsg), C.ptr(zg),
                                                  C.ptr(wu), C.ptr(wsu), C.ptr(zu), C.dtype_code(wsg), grp, N,
                                                  C.ptr(out_q), C.ptr(out_s), C.ptr(ws), ws.numel(),
                                                  C.stream_of(out_q))
        C.check(st, "qlin_pro_mlp_gate_up_quant_w4")
        return out_q, out_s
    N = _check_w8("wg", wg, wsg, K)
    if _check_w8("wu", wu, wsu, K) != N:
        raise ValueError("gate and up must have the same N")
    _check_quant_out(out_q, out_s, M, N)
    C.require_cuda(*pro.tensors(), wg, wsg, wu, wsu, out_q, out_s)
    ws = C.workspace(out_q.device)
    st = _fn("qlin_pro_mlp_gate_up_quant_i8")(ctypes.byref(p), M, K, C.ptr(wg), C.ptr(wsg), C.ptr(wu),
                                              C.ptr(wsu), C.dtype_code(wsg), N, C.ptr(out_q), C.ptr(out_s),
                                              C.ptr(ws), ws.numel(), C.stream_of(out_q))
    C.check(st, "qlin_pro_mlp_gate_up_quant_i8")
    return out_q, out_s
