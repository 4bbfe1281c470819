"""Engine decode chains: the engine-signature linears of a decode step, with their
activation producers, in one persistent launch.

Between two mixer kernels (attention / the delta rule) the engine's decode step makes
a dependent run of calls (engine.py:236-279, 265-268, 272-279, 218-226):

    gate_mul_quant | norm_gated_quant -> gemm_i8 (o-projection, hidden += ...)
    -> rmsnorm_quant -> mlp_gate_up_quant -> gemm_i8 (down, hidden += ...)
    -> rmsnorm_quant (next layer) -> proj3

An `EngineChain` holds that run as jobs with the reference call signatures, each with
its activations in memory (a_q, a_s) or made by a `fused.Producer` in the job's own
work units (the producer may read what an earlier level of the same chain wrote), and
`run()` executes all of them in one launch:

    ch = EngineChain(M=1)
    ch.gemm_i8(None, None, wo, so, hidden, residual=hidden,                  # level 0
               pro=Producer.gate_mul(aout, proj, hd=256))
    ch.mlp_gate_up_quant(None, None, wg, sg, wu, su, hq, hs, level=1,
                         pro=Producer.rmsnorm(hidden, post_norm, eps))
    ch.gemm_i8(hq, hs, wd, sd, hidden, residual=hidden, level=2)             # reads level 1
    ch.proj3(None, None, wq, sq, wk, sk, wv, sv, proj, level=3,
             pro=Producer.rmsnorm(hidden, in_norm_next, eps, q=xq, s=xs))
    ch.build()
    ch.run()          # the attention of the next layer then reads `proj`

Every input must be written before `run()` or by a job of a lower level, and nothing
between two jobs may be needed that is not a job: the attention and delta-rule
kernels end a chain.  Levels start at 0 and rise by at most 1 along the list (default:
the previous job's level).  The tensors are bound at `build()`: write new inputs into
the same tensors and call `run()` again, or capture `run()` in a HIP graph.

Every job gives the same bits as the single call with the same arguments (calls with
1-8 rows run the same work units), so a chain equals the engine's call sequence bit
for bit, and row m of an M-row chain equals an M = 1 chain.
"""
from __future__ import annotations

import ctypes

import torch

from . import qlin as C
from .fused import Producer, _CProducer
from .gemm import _check_act, _check_out, _check_quant_out, _check_w8
from .w4 import _check_w4, fill_zeros

__all__ = ["EngineChain"]

QLIN_EJ_GEMM = 1
QLIN_EJ_GATE_UP = 2
QLIN_EJ_GATE_UP_QUANT = 3


class _EJob(ctypes.Structure):
    """include/qlin.h qlin_echain_job."""
    _fields_ = [
        ("kind", ctypes.c_int),
        ("a_q", ctypes.c_void_p), ("a_s", ctypes.c_void_p),
        ("pro", _CProducer),
        ("K", ctypes.c_int), ("N", ctypes.c_int), ("group", ctypes.c_int),
        ("w", ctypes.c_void_p), ("scale", ctypes.c_void_p), ("zero", ctypes.c_void_p),
        ("w2", ctypes.c_void_p), ("scale2", ctypes.c_void_p), ("zero2", ctypes.c_void_p),
        ("scale_dtype", ctypes.c_int),
        ("out", ctypes.c_void_p), ("ldo", ctypes.c_int64),
        ("residual", ctypes.c_void_p), ("ldr", ctypes.c_int64),
        ("out_q", ctypes.c_void_p), ("out_s", ctypes.c_void_p),
        ("level", ctypes.c_int),
    ]


def _bind(L):
    if getattr(L, "_echain_bound", False):
        return
    P = ctypes.POINTER(_EJob)
    L.qlin_echain_bytes.restype = ctypes.c_size_t
    L.qlin_echain_bytes.argtypes = [P, ctypes.c_int, ctypes.c_int]
    L.qlin_echain_init.restype = ctypes.c_int
    L.qlin_echain_init.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                   ctypes.c_void_p]
    L.qlin_echain_run.restype = ctypes.c_int
    L.qlin_echain_run.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    L._echain_bound = True


def _is_w4(b) -> bool:
    return b.dtype == torch.uint8


class EngineChain:
    """A run of engine-signature linears in one launch (see the module docstring)."""

    def __init__(self, M: int):
        if not 1 <= M <= 8:
            raise ValueError("an engine chain computes 1-8 rows (decode)")
        self.M = M
        self._jobs: list[_EJob] = []
        self._keep: list = []
        self.plan = None
        self.level = 0
        self.device = None
        self.w4 = None

    # ------------------------------------------------------------------ jobs
    def _acts(self, a_q, a_s, pro, K_hint=None):
        """(K, producer struct or None) of a job's activations."""
        if pro is not None:
            if a_q is not None or a_s is not None:
                raise ValueError("a job with a producer takes a_q = a_s = None (pass q / s to the Producer "
                                 "to keep the codes)")
            if not isinstance(pro, Producer):
                raise ValueError("pro must be a kernels.fused.Producer")
            if pro.rows < self.M:
                raise ValueError(f"the producer makes {pro.rows} rows, the chain computes {self.M}")
            return pro.cols, pro
        M, K = _check_act(a_q, a_s)
        if M < self.M:
            raise ValueError(f"a_q has {M} rows, the chain computes {self.M}")
        return K, None

    def _weights(self, name, w, s, z, K, group=None):
        """(N, group (0 = W8)) of one weight."""
        if _is_w4(w):
            N, g = _check_w4(name, w, s, z, K, group)
            return N, g
        if z is not None:
            raise ValueError(f"zeros of {name} apply to W4 weights only")
        return _check_w8(name, w, s, K), 0

    def _append(self, job: _EJob, level, pro, emit, tensors, device):
        if self.plan is not None:
            raise RuntimeError("the chain is built; make a new one to add jobs")
        lvl = self.level if level is None else int(level)
        job.level = lvl
        if pro is not None:
            p = pro.c_struct()
            if not emit:
                p.q = None
                p.s = None
            job.pro = p
            tensors = (*tensors, *pro.tensors())
        w4 = job.group != 0
        if self.w4 is None:
            self.w4 = w4
        elif self.w4 != w4:
            raise ValueError("a chain holds W8 jobs or W4 jobs, not both")
        C.require_cuda(*tensors)
        if self.device is None:
            self.device = device
        self._jobs.append(job)
        self._keep.extend(t for t in tensors if t is not None)
        self.level = lvl

    def gemm_i8(self, a_q, a_s, b, b_s, out, residual=None, b_z=None, *, pro=None, level=None):
        """out[M,N] (bf16) = (a_q * a_s) @ dequant(b) (+ residual), as kernels/gemm.py:60-92
        (W8) or kernels/w4.py:139-166 (uint8 packed `b`, group scales, zeros `b_z`).
        `residual` may be `out`."""
        K, pro = self._acts(a_q, a_s, pro)
        N, g = self._weights("b", b, b_s, b_z, K)
        _check_out("out", out, self.M, N)
        if residual is not None:
            _check_out("residual", residual, self.M, N)
        j = _EJob(kind=QLIN_EJ_GEMM, a_q=C.ptr(a_q), a_s=C.ptr(a_s), K=K, N=N, group=g, w=C.ptr(b),
                  scale=C.ptr(b_s), zero=C.ptr(b_z), scale_dtype=C.dtype_code(b_s), out=C.ptr(out),
                  ldo=out.stride(0), residual=C.ptr(residual),
                  ldr=residual.stride(0) if residual is not None else 0)
        self._append(j, level, pro, True, (a_q, a_s, b, b_s, b_z, out, residual), out.device)
        return self

    def proj3(self, a_q, a_s, w1, s1, w2, s2, w3, s3, out, z1=None, z2=None, z3=None, *, pro=None,
              level=None):
        """proj3 (kernels/gemm.py:290-312, kernels/w4.py:220-251): up to three linears of the
        same activations into column ranges [0, N1), [N1, N1 + N2), [N1 + N2, NT) of `out`.
        One job per projection, all at one level; a producer's codes are kept (q / s)
        by the first.  Zeros given for only some projections follow the reference's
        fill rule (kernels/w4.py fill_zeros)."""
        K, pro = self._acts(a_q, a_s, pro)
        z1, z2, z3 = fill_zeros((z1, z2, z3), (s1, s2 if w2 is not None else None, s3 if w3 is not None else None),
                                next((z for z in (z1, z2, z3) if z is not None), None))
        lvl = self.level if level is None else int(level)
        segs, col, g0 = [], 0, None
        for name, w, s, z in (("w1", w1, s1, z1), ("w2", w2, s2, z2), ("w3", w3, s3, z3)):
            if w is None:
                continue
            N, g = self._weights(name, w, s, z, K, g0 if g0 else None)
            g0 = g if g0 is None else g0
            segs.append((w, s, z, N, col))
            col += N
        if not segs:
            raise ValueError("proj3 needs at least one projection")
        _check_out("out", out, self.M, col)
        es = out.element_size()
        for i, (w, s, z, N, c0) in enumerate(segs):
            j = _EJob(kind=QLIN_EJ_GEMM, a_q=C.ptr(a_q), a_s=C.ptr(a_s), K=K, N=N, group=g0, w=C.ptr(w),
                      scale=C.ptr(s), zero=C.ptr(z), scale_dtype=C.dtype_code(s),
                      out=out.data_ptr() + c0 * es, ldo=out.stride(0), residual=None, ldr=0)
            self._append(j, lvl, pro, i == 0, (a_q, a_s, w, s, z, out), out.device)
        return self

    def mlp_gate_up_quant(self, a_q, a_s, wg, wsg, wu, wsu, out_q, out_s, zg=None, zu=None, *, pro=None,
                          level=None):
        """h = silu(a @ Wg) * (a @ Wu), rounded through bf16 and requantized per 64 columns
        into out_q int8 [M, N] / out_s fp32 [M, N/64] (kernels/gemm.py:214-231,
        kernels/w4.py:300-323); one of zg / zu alone stands in for the other (fill_zeros)."""
        K, pro = self._acts(a_q, a_s, pro)
        zg, zu = fill_zeros((zg, zu), (wsg, wsu), zg if zg is not None else zu)
        N, g = self._weights("wg", wg, wsg, zg, K)
        Nu, gu = self._weights("wu", wu, wsu, zu, K, g if g else None)
        if Nu != N or gu != g or wsg.dtype != wsu.dtype:
            raise ValueError("gate and up must have the same shape, group and scale dtype")
        if out_q.shape[0] < self.M or out_s.shape[0] < self.M:
            raise ValueError(f"out_q / out_s need {self.M} rows")
        _check_quant_out(out_q, out_s, out_q.shape[0], N)
        j = _EJob(kind=QLIN_EJ_GATE_UP_QUANT, a_q=C.ptr(a_q), a_s=C.ptr(a_s), K=K, N=N, group=g, w=C.ptr(wg),
                  scale=C.ptr(wsg), zero=C.ptr(zg), w2=C.ptr(wu), scale2=C.ptr(wsu), zero2=C.ptr(zu),
                  scale_dtype=C.dtype_code(wsg), out_q=C.ptr(out_q), out_s=C.ptr(out_s))
        self._append(j, level, pro, True, (a_q, a_s, wg, wsg, zg, wu, wsu, zu, out_q, out_s), out_q.device)
        return self

    def mlp_gate_up(self, a_q, a_s, wg, wsg, wu, wsu, out, zg=None, zu=None, *, pro=None, level=None):
        """out[M, N] (bf16) = silu(a @ Wg) * (a @ Wu) (kernels/gemm.py:140-151); zeros as
        mlp_gate_up_quant."""
        K, pro = self._acts(a_q, a_s, pro)
        zg, zu = fill_zeros((zg, zu), (wsg, wsu), zg if zg is not None else zu)
        N, g = self._weights("wg", wg, wsg, zg, K)
        Nu, gu = self._weights("wu", wu, wsu, zu, K, g if g else None)
        if Nu != N or gu != g or wsg.dtype != wsu.dtype:
            raise ValueError("gate and up must have the same shape, group and scale dtype")
        _check_out("out", out, self.M, N)
        j = _EJob(kind=QLIN_EJ_GATE_UP, a_q=C.ptr(a_q), a_s=C.ptr(a_s), K=K, N=N, group=g, w=C.ptr(wg),
                  scale=C.ptr(wsg), zero=C.ptr(zg), w2=C.ptr(wu), scale2=C.ptr(wsu), zero2=C.ptr(zu),
                  scale_dtype=C.dtype_code(wsg), out=C.ptr(out), ldo=out.stride(0))
        self._append(j, level, pro, True, (a_q, a_s, wg, wsg, zg, wu, wsu, zu, out), out.device)
        return self

    # ------------------------------------------------------------------ plan and launch
    def build(self):
        """Validate the jobs and write the plan to device memory (once)."""
        if not self._jobs:
            raise ValueError("empty chain")
        L = C.lib()
        _bind(L)
        arr = (_EJob * len(self._jobs))(*self._jobs)
        n = L.qlin_echain_bytes(arr, len(self._jobs), self.M)
        if n == 0:
            C.check(C.QLIN_ERR_INVALID, "qlin_echain_bytes")
        plan = torch.empty(n, dtype=torch.uint8, device=self.device) if self.plan is None else self.plan
        C.check(L.qlin_echain_init(arr, len(self._jobs), self.M, C.ptr(plan), n,
                                   C.current_stream(self.device)), "qlin_echain_init")
        self.plan = plan
        return self

    def run(self):
        """Every job, one launch, on the current stream."""
        if self.plan is None:
            self.build()
        L = C.lib()
        C.check(L.qlin_echain_run(C.ptr(self.plan), C.current_stream(self.device)),
                "qlin_echain_run")

    def wait_error(self) -> int:
        """1 if a wait of the last finished launch gave up (a dependency, or a split tile's
        partial sums), else 0 (reads device memory; synchronizes with the current stream).
        After a 1 the plan must be written again (build()) before the next launch: its
        partial-sum slots may not be empty."""
        return int(self.plan[20:24].view(torch.int32).item())

    def run_checked(self):
        """run(), then wait for it and raise if a wait gave up (the plan is written again
        first, so the chain can be launched once more)."""
        self.run()
        if self.wait_error():
            self.build()
            raise RuntimeError("engine chain: a wait gave up (a job read inputs that no lower level wrote in time, "
                               "or a split tile's partial sums did not arrive)")

    @property
    def nbytes(self) -> int:
        return 0 if self.plan is None else self.plan.numel()
