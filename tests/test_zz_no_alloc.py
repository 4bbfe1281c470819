"""qlin_gemm_i8_noalloc (no counterpart in the reference: the allocation-free form of
qlin_gemm_i8 for callers that cannot allocate device memory) against qlin_gemm_i8 with
the library's workspace, called through the C ABI: the same bits, on consecutive calls
that leave the shared scratch in different states.
"""
from __future__ import annotations

import pytest
import torch

import helpers as H

pytestmark = pytest.mark.gpu


def _noalloc(a, as_, b, bs, out, residual=None):
    from qwen35_amd.kernels import qlin as C
    M, K = a.shape
    N = b.shape[1]
    C.call("qlin_gemm_i8_noalloc", C.ptr(a), C.ptr(as_), M, K, C.ptr(b), C.ptr(bs), C.dtype_code(bs), N,
           C.ptr(out), out.stride(0), C.ptr(residual), residual.stride(0) if residual is not None else 0,
           C.stream_of(out))
    return out


def _with_workspace(a, as_, b, bs, out, residual=None):
    from qwen35_amd.kernels import gemm
    return gemm.gemm_i8(a, as_, b, bs, out, residual=residual)


# (M, K, N): a prefill chunk of the down projection whose split-K partials exceed the
# 8 MiB scratch in one launch (so it runs in blocks of rows), then smaller calls: a
# best-of decode step, a remainder chunk, and a single-row decode
CALLS = [(700, 6144, 2048), (4, 2048, 2048), (188, 2048, 6144), (1, 6144, 2048)]


@pytest.mark.parametrize("first,second", [(0, 1), (2, 3), (1, 3)])
def test_noalloc_matches_workspace_entry_point(first, second):
    for i, (M, K, N) in enumerate((CALLS[first], CALLS[second])):
        a, as_ = H.engine_act(M, K, seed=700 + i)
        b, bs = H.engine_w8(K, N, seed=701 + i)
        hid = torch.randn((M, N), generator=H.gen(702 + i)).to(torch.bfloat16).cuda()
        a, as_, b, bs = a.cuda(), as_.cuda(), b.cuda(), bs.cuda()
        ref = hid.clone()
        _with_workspace(a, as_, b, bs, ref, residual=ref)        # residual in place
        got = hid.clone()
        _noalloc(a, as_, b, bs, got, residual=got)
        plain_ref = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        plain = torch.empty_like(plain_ref)
        _with_workspace(a, as_, b, bs, plain_ref)
        _noalloc(a, as_, b, bs, plain)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (M, K, N)
        assert torch.equal(plain, plain_ref), (M, K, N)


def test_noalloc_rejects_a_call_beyond_the_scratch(monkeypatch):
    """Eight forced K splits of 65536 columns need 32 MiB of partials for 16 rows: more
    than the scratch holds, so the call fails with a message before it launches anything."""
    monkeypatch.setenv("QLIN_ENGINE_SPLITS", "8")
    M, K, N = 16, 2048, 65536
    a, as_ = H.engine_act(M, K, seed=710)
    b, bs = H.engine_w8(K, N, seed=711)
    out = torch.zeros((M, N), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="workspace"):
        _noalloc(a.cuda(), as_.cuda(), b.cuda(), bs.cuda(), out)
    torch.cuda.synchronize()
    assert int(out.view(torch.int16).abs().sum()) == 0
