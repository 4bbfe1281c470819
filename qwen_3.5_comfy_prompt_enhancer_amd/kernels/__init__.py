"""gfx950 quantized-linear kernels behind the engine's call signatures.

`gemm` and `w4` mirror the reference's kernels/gemm.py and kernels/w4.py; `linear`
holds the A16 (fp16-activation) weight-only core; `layout` the unpack / dequant
checks; `qlin` loads libqlin.so; `common` holds GROUP.
"""
from .common import GROUP  # noqa: F401
