"""MI355X (gfx950) rebuild of the Qwen3.5 prompt-enhancer engine's quantized-linear path.

`kernels.gemm` / `kernels.w4` keep the engine's call signatures (gemm_i8, proj3,
mlp_gate_up, mlp_gate_up_quant and their W4 twins); `kernels.linear` holds the
fp16-activation weight-only core.  The engine's call sites (engine.py:221-374) use
these functions unchanged.  All of them launch the hand-written HIP kernels of
kernels/libqlin.so.
"""
__version__ = "0.1.0"
