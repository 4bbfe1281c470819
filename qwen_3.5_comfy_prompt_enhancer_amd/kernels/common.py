"""Constants shared with the engine (kernels/common.py:5-9 of the reference).

In a drop-in install the reference's own kernels/common.py (which also carries the
Triton helpers its norm / attention kernels use) stays in place; it defines the same
GROUP.  The launch plumbing of the quantized linears lives in `qlin.py`.
"""

# Activation quantization granularity: one fp32 scale per 64 int8 values along K
# (kernels/common.py:5-7).
GROUP = 64
