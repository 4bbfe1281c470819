"""CPU tests of the C-ABI boundary (no GPU needed): libqlin.so loads, exports every
function include/qlin.h declares, and rejects bad arguments with the documented
status codes before launching anything; the Python shims validate shapes and dtypes
and raise ValueError like the reference's wrappers would fail on bad input."""
from __future__ import annotations

import ctypes
import pathlib
import re

import pytest
import torch

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "qlin.h"


def _lib():
    from qwen35_amd.kernels import qlin
    return qlin, qlin.lib()


def declared_functions():
    src = HEADER.read_text()
    return re.findall(r"^\s*(?:int|const char\*|size_t)\s+(qlin_\w+)\s*\(", src, re.M)


def test_header_declares_the_abi():
    names = declared_functions()
    assert len(names) == 39
    for n in ("qlin_echain_bytes", "qlin_echain_init", "qlin_echain_run","qlin_rmsnorm_quant", "qlin_gate_mul_quant", "qlin_norm_gated_quant", "qlin_pro_exp_f32",
              "qlin_pro_gemm_i8", "qlin_pro_gemm_w4", "qlin_pro_proj3_i8", "qlin_pro_proj3_w4",
              "qlin_pro_mlp_gate_up_quant_i8", "qlin_pro_mlp_gate_up_quant_w4",
              "qlin_gemm_i8", "qlin_gemm_i8_noalloc", "qlin_chain_bytes", "qlin_chain_init", "qlin_chain_run",
              "qlin_gemm_w4", "qlin_proj3_i8", "qlin_proj3_w4",
              "qlin_mlp_gate_up_quant_i8", "qlin_mlp_gate_up_quant_w4", "qlin_linear_w8",
              "qlin_linear_w4", "qlin_w4_unpack", "qlin_w4_dequant_f32",
              "qlin_requant_w4_sym", "qlin_requant_w8_row", "qlin_w4_repack_gptq",
              "qlin_w4_repack_awq", "qlin_w4_zeros_unpack", "qlin_w4_repack_ct"):
        assert n in names


def test_library_exports_every_declared_symbol():
    qlin, L = _lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert missing == []
    assert set(declared_functions()) == set(qlin.EXPORTS)


def test_version_and_workspace():
    _, L = _lib()
    assert L.qlin_version() == 1
    assert L.qlin_workspace_bytes() == 256 << 20
    # every entry point clears the calling thread's message; an empty call succeeds
    assert L.qlin_w4_unpack(None, 0, 0, None, None) == 0
    assert L.qlin_last_error() == b""


I64 = ctypes.c_int64
SZ = ctypes.c_size_t
FAKE = ctypes.c_void_p(0x10000)      # aligned non-null pointer, never dereferenced


def test_null_activations_rejected():
    qlin, L = _lib()
    rc = L.qlin_gemm_i8(None, None, 1, 128, FAKE, FAKE, qlin.QLIN_F32, 64, FAKE, I64(64), None, I64(0),
                        None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_INVALID
    assert b"null activations" in L.qlin_last_error()


def test_bad_k_rejected():
    qlin, L = _lib()
    rc = L.qlin_gemm_i8(FAKE, FAKE, 1, 96, FAKE, FAKE, qlin.QLIN_F32, 64, FAKE, I64(64), None, I64(0),
                        None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED
    assert b"K=96" in L.qlin_last_error()


def test_element_misalignment_rejected():
    """Any N and any 16-byte misalignment are valid engine calls (they run on the edge
    kernel); a pointer off its own element size, or a row stride below N, is refused
    before any launch."""
    qlin, L = _lib()
    odd = ctypes.c_void_p(0x10001)
    rc = L.qlin_gemm_i8(FAKE, FAKE, 1, 128, FAKE, odd, qlin.QLIN_F32, 40, FAKE, I64(40), None, I64(0),
                        None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED and b"scales must be aligned" in L.qlin_last_error()
    rc = L.qlin_gemm_i8(FAKE, FAKE, 1, 128, FAKE, FAKE, qlin.QLIN_F32, 40, odd, I64(40), None, I64(0),
                        None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED and b"out must be 2-byte aligned" in L.qlin_last_error()
    rc = L.qlin_gemm_i8(FAKE, odd, 1, 128, FAKE, FAKE, qlin.QLIN_F32, 40, FAKE, I64(40), None, I64(0),
                        None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED and b"a_s must be 4-byte aligned" in L.qlin_last_error()
    rc = L.qlin_gemm_i8(FAKE, FAKE, 1, 128, FAKE, FAKE, qlin.QLIN_F32, 40, FAKE, I64(39), None, I64(0),
                        None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_INVALID and b"row stride" in L.qlin_last_error()


def test_bad_group_rejected():
    qlin, L = _lib()
    rc = L.qlin_gemm_w4(FAKE, FAKE, 1, 256, FAKE, FAKE, qlin.QLIN_BF16, None, 48, 64, FAKE, I64(64), None,
                        I64(0), None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED and b"group 48" in L.qlin_last_error()
    rc = L.qlin_linear_w4(FAKE, qlin.QLIN_F16, 1, 192, I64(192), FAKE, FAKE, qlin.QLIN_F16, None, 128, 64,
                          FAKE, qlin.QLIN_F16, I64(64), None, I64(0), None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_INVALID and b"not a multiple of the group" in L.qlin_last_error()


def test_bad_dtypes_rejected():
    qlin, L = _lib()
    rc = L.qlin_linear_w8(FAKE, qlin.QLIN_F32, 1, 128, I64(128), FAKE, FAKE, qlin.QLIN_F16, 64, FAKE,
                          qlin.QLIN_F16, I64(64), None, I64(0), None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED and b"activation dtype" in L.qlin_last_error()
    rc = L.qlin_linear_w8(FAKE, qlin.QLIN_F16, 1, 128, I64(128), FAKE, FAKE, 9, 64, FAKE,
                          qlin.QLIN_F16, I64(64), None, I64(0), None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED and b"scale dtype" in L.qlin_last_error()


def test_zero_sized_calls_are_no_ops():
    qlin, L = _lib()
    assert L.qlin_gemm_i8(None, None, 0, 128, None, None, qlin.QLIN_F32, 64, None, I64(64), None, I64(0),
                          None, SZ(0), None) == 0
    assert L.qlin_w4_unpack(None, 0, 16, None, None) == 0


def test_proj3_zero_mixing_rejected():
    qlin, L = _lib()
    rc = L.qlin_proj3_w4(FAKE, FAKE, 1, 128, FAKE, FAKE, FAKE, 64, FAKE, FAKE, None, 64, None, None, None, 0,
                         qlin.QLIN_BF16, 128, FAKE, I64(128), None, SZ(0), None)
    assert rc == qlin.QLIN_ERR_INVALID and b"zeros" in L.qlin_last_error()


# ---------------------------------------------------------------- Python shim validation

def test_shims_validate_before_launch():
    from qwen35_amd.kernels import gemm, linear, w4
    a = torch.zeros((2, 128), dtype=torch.int8)
    s = torch.zeros((2, 2), dtype=torch.float32)
    b = torch.zeros((128, 64), dtype=torch.int8)
    bs = torch.zeros(64, dtype=torch.float32)
    out = torch.zeros((2, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="a_s must be"):
        gemm.gemm_i8(a, s[:, :1], b, bs, out)
    with pytest.raises(ValueError, match="out must be"):
        gemm.gemm_i8(a, s, b, bs, out.float())
    with pytest.raises(ValueError, match="GPU"):
        gemm.gemm_i8(a, s, b, bs, out)                 # CPU tensors
    p = torch.zeros((64, 64), dtype=torch.uint8)
    ps = torch.zeros((1, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="zeros"):
        w4.gemm_w4(a, s, p, ps, out, b_z=torch.zeros((2, 64), dtype=torch.uint8))
    x = torch.zeros((2, 128), dtype=torch.float32)
    with pytest.raises(ValueError, match="float16"):
        linear.linear_w8(x, b, bs.half(), out.half())


def test_stream_of_rejects_host_tensors():
    """The current-stream lookup (torch's raw-stream binding) refuses a tensor that is
    not on a GPU instead of handing a host pointer's call a stream."""
    from qwen35_amd.kernels import qlin
    with pytest.raises(ValueError, match="GPU"):
        qlin.stream_of(torch.zeros(4))
    with pytest.raises(ValueError, match="GPU"):
        qlin.current_stream(-1)


def test_w4_dispatch_follows_weight_dtype():
    """uint8 weights route gemm_i8 / proj3 / mlp_gate_up_quant to the W4 path
    (kernels/gemm.py:15-17): the W4 validator's message proves the route."""
    from qwen35_amd.kernels import gemm
    a = torch.zeros((2, 128), dtype=torch.int8)
    s = torch.zeros((2, 2), dtype=torch.float32)
    p = torch.zeros((32, 64), dtype=torch.uint8)        # wrong K/2 on purpose
    ps = torch.zeros((1, 64), dtype=torch.bfloat16)
    out = torch.zeros((2, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match=r"uint8 \[K/2=64"):
        gemm.gemm_i8(a, s, p, ps, out)
    with pytest.raises(ValueError, match=r"uint8 \[K/2=64"):
        gemm.proj3(a, s, p, ps, None, None, None, None, out)


def test_chain_validation_without_gpu():
    """qlin_chain_bytes validates the job list on the host: a level that jumps by 2, a
    W4 group other than 128 and a misaligned pointer are refused with a message."""
    qlin, L = _lib()
    from qwen35_amd.kernels import chain as CH
    CH._bind(L)

    def job(level=0, group=0, K=2048, N=512, x=0x10000):
        return CH._Job(x=x, ldx=K, w=0x20000, scale=0x30000, scale_dtype=qlin.QLIN_F16, zero=None, K=K, N=N,
                       group=group, out=0x40000, out_dtype=qlin.QLIN_F16, ldo=N, residual=None, ldr=0,
                       level=level)
    ok = (CH._Job * 2)(job(0), job(1))
    assert L.qlin_chain_bytes(ok, 2, 4) > 0
    bad = (CH._Job * 2)(job(0), job(2))
    assert L.qlin_chain_bytes(bad, 2, 4) == 0
    assert b"level" in L.qlin_last_error()
    assert L.qlin_chain_bytes((CH._Job * 1)(job(group=64)), 1, 1) == 0
    assert b"group" in L.qlin_last_error()
    assert L.qlin_chain_bytes((CH._Job * 1)(job(x=0x10008)), 1, 1) == 0
    assert b"aligned" in L.qlin_last_error()
    assert L.qlin_chain_bytes((CH._Job * 1)(job()), 1, 17) == 0


def test_echain_validation_without_gpu():
    """qlin_echain_bytes validates an engine chain on the host: the struct layout the
    Python binding declares, the level rule, W8 and W4 jobs not mixed, rows 1-8, a W4
    group that is not a multiple of 64, gate/up + quant needing N % 64 == 0, a producer
    job that also names activations, and a bad producer (head size)."""
    qlin, L = _lib()
    from qwen35_amd.kernels import echain as EC
    from qwen35_amd.kernels import fused as FU
    EC._bind(L)

    def job(kind=EC.QLIN_EJ_GEMM, level=0, group=0, K=2048, N=512, aq=0x10000, pro=None):
        j = EC._EJob(kind=kind, a_q=aq, a_s=0x11000 if aq else None, K=K, N=N, group=group, w=0x20000,
                     scale=0x30000, scale_dtype=qlin.QLIN_BF16, out=0x40000, ldo=N, level=level)
        if kind != EC.QLIN_EJ_GEMM:
            j.w2, j.scale2, j.out_q, j.out_s = 0x50000, 0x60000, 0x70000, 0x80000
        if pro is not None:
            j.pro = pro
        return j

    def nbytes(*jobs, M=4):
        return L.qlin_echain_bytes((EC._EJob * len(jobs))(*jobs), len(jobs), M)

    assert nbytes(job(), job(EC.QLIN_EJ_GATE_UP_QUANT, level=1, N=6144), job(level=2)) > 0
    assert nbytes(job(), job(level=2)) == 0 and b"levels" in L.qlin_last_error()
    assert nbytes(job(), job(group=128, level=1)) == 0 and b"W8 jobs or W4" in L.qlin_last_error()
    assert nbytes(job(), M=9) == 0 and b"1-8" in L.qlin_last_error()
    assert nbytes(job(group=96, K=2880)) == 0 and b"group" in L.qlin_last_error()
    assert nbytes(job(EC.QLIN_EJ_GATE_UP_QUANT, N=528)) == 0 and b"N % 64" in L.qlin_last_error()
    rms = FU._CProducer(kind=1, x=0x90000, ldx=2048, x_dtype=qlin.QLIN_BF16, g=None, ldg=0, w=0xA0000,
                        w_dtype=qlin.QLIN_BF16, hd=0, one_plus=1, eps=1e-6, q=None, s=None)
    assert nbytes(job(aq=None, pro=rms)) > 0
    assert nbytes(job(pro=rms)) == 0 and b"a_q" in L.qlin_last_error()
    ng = FU._CProducer(kind=3, x=0x90000, ldx=2048, x_dtype=qlin.QLIN_BF16, g=0xB0000, ldg=8192, w=0xA0000,
                       w_dtype=qlin.QLIN_BF16, hd=64, one_plus=0, eps=1e-6, q=None, s=None)
    assert nbytes(job(aq=None, pro=ng)) == 0 and b"head size 64" in L.qlin_last_error()


def test_producer_validation_without_gpu():
    """The activation producers refuse bad arguments on the host with a message: K not a
    multiple of 64, an fp32 input, a norm_gated head size the reference's kernel cannot
    serve (64), a gate stride under 2 N, and missing q / s."""
    qlin, L = _lib()
    F = ctypes.c_float
    rc = L.qlin_rmsnorm_quant(FAKE, I64(96), qlin.QLIN_BF16, FAKE, qlin.QLIN_BF16, 1, 96, F(1e-6), 1, FAKE, FAKE,
                              None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED and b"K=96" in L.qlin_last_error()
    rc = L.qlin_rmsnorm_quant(FAKE, I64(128), qlin.QLIN_F32, FAKE, qlin.QLIN_BF16, 1, 128, F(1e-6), 1, FAKE, FAKE,
                              None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED and b"activation dtype" in L.qlin_last_error()
    rc = L.qlin_norm_gated_quant(FAKE, FAKE, I64(128), qlin.QLIN_BF16, FAKE, qlin.QLIN_BF16, 1, 128, 64, F(1e-6),
                                 FAKE, FAKE, None)
    assert rc == qlin.QLIN_ERR_UNSUPPORTED and b"head size 64" in L.qlin_last_error()
    rc = L.qlin_gate_mul_quant(FAKE, I64(256), FAKE, I64(256), qlin.QLIN_BF16, 1, 256, 128, FAKE, FAKE, None)
    assert rc == qlin.QLIN_ERR_INVALID and b"2 K" in L.qlin_last_error()
    rc = L.qlin_rmsnorm_quant(FAKE, I64(128), qlin.QLIN_BF16, FAKE, qlin.QLIN_BF16, 1, 128, F(1e-6), 1, None, None,
                              None)
    assert rc == qlin.QLIN_ERR_INVALID and b"null q" in L.qlin_last_error()


def test_fused_producer_validation_without_gpu():
    """A fused linear without a producer, or without q / s and without a workspace for the
    codes, is refused before anything is launched."""
    qlin, L = _lib()
    from qwen35_amd.kernels import fused as FU
    f = FU._fn("qlin_pro_gemm_i8")
    rc = f(None, 1, 128, FAKE, FAKE, qlin.QLIN_F32, 64, FAKE, 64, None, 0, None, 0, None)
    assert rc == qlin.QLIN_ERR_INVALID and b"null producer" in L.qlin_last_error()
    p = FU._CProducer(kind=1, x=0x10000, ldx=128, x_dtype=qlin.QLIN_BF16, g=None, ldg=0, w=0x20000,
                      w_dtype=qlin.QLIN_BF16, hd=0, one_plus=1, eps=1e-6, q=None, s=None)
    rc = f(ctypes.byref(p), 1, 128, FAKE, FAKE, qlin.QLIN_F32, 64, FAKE, 64, None, 0, None, 0, None)
    assert rc == qlin.QLIN_ERR_WORKSPACE and b"workspace" in L.qlin_last_error()
    p.kind = 7
    rc = f(ctypes.byref(p), 1, 128, FAKE, FAKE, qlin.QLIN_F32, 64, FAKE, 64, None, 0, None, 0, None)
    assert rc == qlin.QLIN_ERR_INVALID and b"producer kind" in L.qlin_last_error()
