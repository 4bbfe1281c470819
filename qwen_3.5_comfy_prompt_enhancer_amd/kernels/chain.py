"""Decode chains: many A16 linears in one persistent launch.

The reference launches one kernel per linear and names whole-step decode capture as
its next step, since decode is dispatch-bound (ENGINEERING.md:383-399).  A
`DecodeChain` holds a list of linears -- each one what `linear_w8` / `linear_w4`
computes, with fp16 activations -- with dependency levels, and `run()` computes all of
them in one launch of libqlin.so's chain kernel.  Every input of a job must be written
before `run()` or be the output of a job of a lower level; anything that is not a
linear (attention, a norm, an activation function) ends a chain.  For example, the
independent GEMVs of a decode sweep, then a projection of one of their outputs:

    chain = DecodeChain(M=1)
    chain.add(x, wq, sq, q_out)                         # level 0: x written before run()
    chain.add(x, wk, sk, k_out)                         # level 0
    chain.add(q_out, wp, sp, p_out, level=1)            # reads q_out, written by level 0
    chain.build()
    chain.run()                                         # every job, one launch

The engine's own decode step holds int8 activations and producers between its linears:
it runs on `kernels/echain.py` `EngineChain` instead.  Levels start at 0 and rise by at
most 1 along the list.  The tensors are bound when `build()` runs: write new inputs
into the same tensors and call `run()` again (a HIP graph may capture `run()`).  W4
jobs take group-128 scales.
"""
from __future__ import annotations

import ctypes

import torch

from . import qlin as C

__all__ = ["DecodeChain"]


class _Job(ctypes.Structure):
    """include/qlin.h qlin_chain_job."""
    _fields_ = [
        ("x", ctypes.c_void_p), ("ldx", ctypes.c_int64),
        ("w", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("scale_dtype", ctypes.c_int),
        ("zero", ctypes.c_void_p),
        ("K", ctypes.c_int), ("N", ctypes.c_int), ("group", ctypes.c_int),
        ("out", ctypes.c_void_p), ("out_dtype", ctypes.c_int), ("ldo", ctypes.c_int64),
        ("residual", ctypes.c_void_p), ("ldr", ctypes.c_int64),
        ("level", ctypes.c_int),
    ]


def _bind(L):
    if getattr(L, "_chain_bound", False):
        return
    P = ctypes.POINTER(_Job)
    L.qlin_chain_bytes.restype = ctypes.c_size_t
    L.qlin_chain_bytes.argtypes = [P, ctypes.c_int, ctypes.c_int]
    L.qlin_chain_init.restype = ctypes.c_int
    L.qlin_chain_init.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                  ctypes.c_void_p]
    L.qlin_chain_run.restype = ctypes.c_int
    L.qlin_chain_run.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    L._chain_bound = True


class DecodeChain:
    """A list of A16 linears run in one launch (see the module docstring)."""

    def __init__(self, M: int):
        if not 1 <= M <= 16:
            raise ValueError("a chain computes 1-16 rows")
        self.M = M
        self._jobs: list[_Job] = []
        self._keep: list = []        # tensors the plan points to
        self.plan = None
        self.level = 0

    def add(self, x, w, scale, out, zero=None, residual=None, level=None):
        """Append out[M,N] = x @ dequant(w) (+ residual).  `w` int8 [K,N] (W8, scale
        [N]) or uint8 [K/2,N] packed nibbles (W4 group 128, scale [K/128,N], `zero`
        uint8 [K/128,N] or None).  `level` defaults to the previous job's."""
        if self.plan is not None:
            raise RuntimeError("the chain is built; make a new one to add jobs")
        lvl = self.level if level is None else int(level)
        if x.dtype != torch.float16 or x.dim() != 2 or x.shape[0] < self.M:
            raise ValueError(f"x must be float16 [>= {self.M}, K]")
        C.require_rowmajor("x", x)
        K = x.shape[1]
        w4 = w.dtype == torch.uint8
        if w4:
            if w.dim() != 2 or w.shape[0] * 2 != K:
                raise ValueError(f"w must be uint8 [K/2={K // 2}, N]")
            if scale.dim() != 2 or scale.shape[0] * 128 != K or scale.shape[1] != w.shape[1]:
                raise ValueError("W4 chain jobs take group-128 scales [K/128, N]")
            if zero is not None and (zero.dtype != torch.uint8 or tuple(zero.shape) != tuple(scale.shape)):
                raise ValueError(f"zero must be uint8 {tuple(scale.shape)}")
        else:
            if w.dtype != torch.int8 or w.dim() != 2 or w.shape[0] != K:
                raise ValueError(f"w must be int8 [K={K}, N]")
            if scale.dim() != 1 or scale.shape[0] != w.shape[1]:
                raise ValueError("W8 scale must be [N]")
            if zero is not None:
                raise ValueError("zeros are for W4 jobs")
        N = w.shape[1]
        for name, t in (("w", w), ("scale", scale), ("zero", zero)):
            C.require_contig(name, t)
        if out.dtype not in (torch.float16, torch.bfloat16) or out.shape[0] < self.M or out.shape[1] < N:
            raise ValueError(f"out must be float16/bfloat16 [>= {self.M}, >= {N}]")
        C.require_rowmajor("out", out)
        if residual is not None:
            if residual.dtype != out.dtype or residual.shape[0] < self.M or residual.shape[1] < N:
                raise ValueError("residual must match out")
            C.require_rowmajor("residual", residual)
        C.require_cuda(x, w, scale, zero, out, residual)
        j = _Job(x=C.ptr(x), ldx=x.stride(0), w=C.ptr(w), scale=C.ptr(scale),
                 scale_dtype=C.dtype_code(scale), zero=C.ptr(zero), K=K, N=N, group=128 if w4 else 0,
                 out=C.ptr(out), out_dtype=C.dtype_code(out), ldo=out.stride(0), residual=C.ptr(residual),
                 ldr=residual.stride(0) if residual is not None else 0, level=lvl)
        self._jobs.append(j)
        self._keep.extend(t for t in (x, w, scale, zero, out, residual) if t is not None)
        self.level = lvl
        self.device = out.device
        return self

    def build(self):
        """Validate the jobs and write the plan to device memory (once)."""
        if not self._jobs:
            raise ValueError("empty chain")
        L = C.lib()
        _bind(L)
        arr = (_Job * len(self._jobs))(*self._jobs)
        n = L.qlin_chain_bytes(arr, len(self._jobs), self.M)
        if n == 0:
            C.check(C.QLIN_ERR_INVALID, "qlin_chain_bytes")
        plan = torch.empty(n, dtype=torch.uint8, device=self.device)
        C.check(L.qlin_chain_init(arr, len(self._jobs), self.M, C.ptr(plan), n,
                                  C.current_stream(self.device)), "qlin_chain_init")
        self.plan = plan
        return self

    def run(self):
        """Every job, one launch, on the current stream."""
        if self.plan is None:
            self.build()
        L = C.lib()
        C.check(L.qlin_chain_run(C.ptr(self.plan), C.current_stream(self.device)),
                "qlin_chain_run")

    def wait_error(self) -> int:
        """1 if a dependency wait of the last finished launch gave up, else 0 (reads device
        memory; synchronizes with the current stream)."""
        return int(self.plan[20:24].view(torch.int32).item())

    def run_checked(self):
        """run(), then wait for it and raise if a dependency wait gave up."""
        self.run()
        if self.wait_error():
            raise RuntimeError("decode chain: a dependency wait gave up (a job read inputs that no lower level "
                               "wrote in time)")

    @property
    def nbytes(self) -> int:
        return 0 if self.plan is None else self.plan.numel()
