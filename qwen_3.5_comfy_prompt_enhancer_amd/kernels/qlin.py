"""ctypes binding of libqlin.so and the launch plumbing of the quantized-linear
kernels (the launch/config helpers the reference keeps in kernels/common.py).

The device helpers the reference's kernels/common.py defines as Triton functions --
`swizzle` (12-21), `round_i8` (24-29), `silu` (32-34) -- live in HIP in
`csrc/qlin_dev.h`.  This module holds:

* loading `libqlin.so` with ctypes and declaring its C ABI (include/qlin.h);
* tensor -> pointer / dtype-code marshalling and the current HIP stream;
* the split-K workspace of each (device, stream) (allocated once, zero-filled, reused);
* status code -> exception (ValueError for bad arguments, RuntimeError otherwise).

There is no fallback: if the library is missing or no GPU is present, the
entry points raise.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import threading

import torch

from .common import GROUP  # noqa: F401  (re-exported)

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libqlin.so"

QLIN_OK = 0
QLIN_ERR_INVALID = -1
QLIN_ERR_UNSUPPORTED = -2
QLIN_ERR_HIP = -3
QLIN_ERR_WORKSPACE = -4

QLIN_F16 = 1
QLIN_BF16 = 2
QLIN_F32 = 3

_DT = {torch.float16: QLIN_F16, torch.bfloat16: QLIN_BF16, torch.float32: QLIN_F32}

_lib = None
_lib_lock = threading.Lock()

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_S = ctypes.c_size_t

# argument lists of the C ABI (include/qlin.h); every entry point returns int
_SIGS = {
    "qlin_gemm_i8": [_P, _P, _I, _I, _P, _P, _I, _I, _P, _L, _P, _L, _P, _S, _P],
    "qlin_gemm_i8_noalloc": [_P, _P, _I, _I, _P, _P, _I, _I, _P, _L, _P, _L, _P],
    "qlin_gemm_w4": [_P, _P, _I, _I, _P, _P, _I, _P, _I, _I, _P, _L, _P, _L, _P, _S, _P],
    "qlin_proj3_i8": [_P, _P, _I, _I, _P, _P, _I, _P, _P, _I, _P, _P, _I, _I, _P, _L, _P, _S, _P],
    "qlin_proj3_w4": [_P, _P, _I, _I, _P, _P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I,
                      _P, _L, _P, _S, _P],
    "qlin_mlp_gate_up_i8": [_P, _P, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P, _S, _P],
    "qlin_mlp_gate_up_w4": [_P, _P, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _S, _P],
    "qlin_mlp_gate_up_quant_i8": [_P, _P, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P, _P, _S, _P],
    "qlin_mlp_gate_up_quant_w4": [_P, _P, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P,
                                  _P, _S, _P],
    "qlin_linear_w8": [_P, _I, _I, _I, _L, _P, _P, _I, _I, _P, _I, _L, _P, _L, _P, _S, _P],
    "qlin_linear_w4": [_P, _I, _I, _I, _L, _P, _P, _I, _P, _I, _I, _P, _I, _L, _P, _L, _P, _S, _P],
    "qlin_w4_unpack": [_P, _I, _I, _P, _P],
    "qlin_w4_dequant_f32": [_P, _P, _I, _P, _I, _I, _I, _P, _P],
    "qlin_w8_dequant_f32": [_P, _P, _I, _I, _I, _P, _P],
    "qlin_requant_w4_sym": [_P, _I, _I, _I, _P, _P, _P],
    "qlin_requant_w8_row": [_P, _I, _I, _P, _P, _P],
    "qlin_w4_repack_gptq": [_P, _I, _I, _P, _P],
    "qlin_w4_repack_awq": [_P, _I, _I, _P, _P],
    "qlin_w4_zeros_unpack": [_P, _I, _I, _I, _I, _P, _P],
    "qlin_w4_repack_ct": [_P, _I, _I, _I, _P, _P],
    "qlin_rmsnorm_quant": [_P, _L, _I, _P, _I, _I, _I, ctypes.c_float, _I, _P, _P, _P],
    "qlin_gate_mul_quant": [_P, _L, _P, _L, _I, _I, _I, _I, _P, _P, _P],
    "qlin_norm_gated_quant": [_P, _P, _L, _I, _P, _I, _I, _I, _I, ctypes.c_float, _P, _P, _P],
    "qlin_pro_exp_f32": [_P, _P, _I, _P],
}

# the decode-chain entry points are declared in kernels/chain.py and kernels/echain.py (they
# take a struct array),
# the fused-producer linears in kernels/fused.py (they take a struct)
EXPORTS = ("qlin_version", "qlin_last_error", "qlin_workspace_bytes", *_SIGS,
           "qlin_chain_bytes", "qlin_chain_init", "qlin_chain_run",
           "qlin_echain_bytes", "qlin_echain_init", "qlin_echain_run",
           "qlin_pro_gemm_i8", "qlin_pro_gemm_w4", "qlin_pro_proj3_i8", "qlin_pro_proj3_w4",
           "qlin_pro_mlp_gate_up_quant_i8", "qlin_pro_mlp_gate_up_quant_w4")


def lib() -> ctypes.CDLL:
    """The loaded libqlin.so (raises ImportError if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} not found: build it with "
                    "`python qwen_3.5_comfy_prompt_enhancer_amd/build.py`")
            L = ctypes.CDLL(str(LIB_PATH))
            L.qlin_version.restype = ctypes.c_int
            L.qlin_version.argtypes = []
            L.qlin_last_error.restype = ctypes.c_char_p
            L.qlin_last_error.argtypes = []
            L.qlin_workspace_bytes.restype = ctypes.c_size_t
            L.qlin_workspace_bytes.argtypes = []
            for name, args in _SIGS.items():
                f = getattr(L, name)
                f.restype = ctypes.c_int
                f.argtypes = args
            _lib = L
    return _lib


def ptr(t) -> int | None:
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else t.data_ptr()


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


# The current stream's raw handle without building a torch Stream object (0.1 us
# against 2-3 us for torch.cuda.current_stream(), which is most of a call's host time
# otherwise); the public API where this build of torch lacks the binding.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream(device: torch.device | int) -> int:
    """The current HIP stream of a device (torch.device or index), as the hipStream_t
    the C ABI takes."""
    idx = device if isinstance(device, int) else device.index
    if idx is None:
        idx = torch.cuda.current_device()
    if idx < 0:
        raise ValueError("tensors must be on the GPU")
    if _raw_stream is not None:
        return int(_raw_stream(idx))
    return torch.cuda.current_stream(torch.device("cuda", idx)).cuda_stream


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of `t`'s device, as the hipStream_t the C ABI takes."""
    return current_stream(t.get_device())


def check(status: int, name: str) -> None:
    if status == QLIN_OK:
        return
    msg = lib().qlin_last_error().decode(errors="replace") or name
    if status in (QLIN_ERR_INVALID, QLIN_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)


_ws: dict[tuple[int, int], torch.Tensor] = {}
_ws_lock = threading.Lock()
_capture_streams: dict[int, torch.cuda.Stream] = {}


def workspace(device: torch.device, stream: int | None = None) -> torch.Tensor:
    """Split-K workspace of (device, stream), zero-filled once; the kernels leave their
    arrival counters at zero after every call, so it is never cleared again.

    Each stream gets its own, so calls running at the same time on two streams never
    share arrival counters or partial sums.  A call under HIP graph capture uses the
    workspace of the capturing stream, which must exist before capture starts (a
    zero-fill cannot go into the graph): capture with `capture()` below, or call
    `bind_workspace(stream)` first.  A graph replays with the workspace it was captured
    with, so graphs captured on one stream must not be replayed at the same time as each
    other or as calls on that stream."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if stream is None:
        stream = current_stream(idx)
    key = (idx, int(stream))
    w = _ws.get(key)
    if w is not None:
        return w
    with _ws_lock:
        w = _ws.get(key)
        if w is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "quantized-linear call under HIP graph capture on a stream without a workspace: capture "
                    "with kernels.qlin.capture(graph), or call kernels.qlin.bind_workspace(stream) before "
                    "capturing")
            nbytes = lib().qlin_workspace_bytes()
            w = torch.zeros(nbytes, dtype=torch.uint8, device=torch.device("cuda", idx))
            _ws[key] = w
    return w


def bind_workspace(stream: torch.cuda.Stream) -> torch.Tensor:
    """Allocate (once) the workspace of `stream`, outside graph capture, so that calls
    captured on it later find it."""
    return workspace(stream.device, stream.cuda_stream)


def capture(graph: torch.cuda.CUDAGraph, stream: torch.cuda.Stream | None = None, **kw):
    """`torch.cuda.graph(graph, stream=...)` on a stream that has a workspace: `stream`
    (bound here if it has none), or a capture stream of the current device's own.
    Graphs captured on the same stream share its workspace (see `workspace`)."""
    if stream is None:
        idx = torch.cuda.current_device()
        stream = _capture_streams.get(idx)
        if stream is None:
            stream = torch.cuda.Stream(device=idx)
            _capture_streams[idx] = stream
    bind_workspace(stream)
    return torch.cuda.graph(graph, stream=stream, **kw)


def require_cuda(*ts) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("all tensors must be on the GPU")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev


def require_contig(name: str, t) -> None:
    if t is not None and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def require_rowmajor(name: str, t) -> None:
    """2-D with unit column stride (rows may be strided)."""
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError(f"{name} must be a 2-D row-major matrix")


def call(name: str, *args) -> None:
    """Invoke one C entry point and raise on a non-zero status."""
    check(getattr(lib(), name)(*args), name)
