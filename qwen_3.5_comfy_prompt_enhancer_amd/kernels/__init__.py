"""gfx950 quantized-linear kernels behind the engine's call signatures.

`gemm` and `w4` mirror the reference's kernels/gemm.py and kernels/w4.py, `norm` the
activation producers of its kernels/norm.py; `fused` runs a producer and a linear in
one call; `linear` holds the A16 (fp16-activation) weight-only core; `chain` whole
decode steps in one launch; `layout` the unpack / dequant checks and load-time
layout producers; `qlin` loads libqlin.so; `common` holds GROUP.
"""
from .common import GROUP  # noqa: F401
