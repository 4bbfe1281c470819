"""Seeded synthetic inputs in the engine layouts, shared by the parity tests and bench.

Distributions follow the workload definitions: fp16 activations N(0, 1); int8 weights
uniform on [-127, 127] with per-output-column fp16 scales |N(0, 0.02)| / 127; W4
nibbles uniform on [0, 15], packed two per byte along K (even k in the low nibble),
group-128 fp16 scales |N(0, 0.02)| / 7, zero point 8.  Everything is generated on the
CPU with a seeded torch.Generator so the oracle and the GPU see identical bits.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import ref_cpu as R


def gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def act_f16(M: int, K: int, seed: int) -> torch.Tensor:
    return torch.randn((M, K), generator=gen(seed)).to(torch.float16)


def w8(K: int, N: int, seed: int):
    """int8 [K, N] (engine layout; the logical [N, K] weight transposed) + fp16 [N]."""
    g = gen(seed)
    w_nk = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = (torch.randn(N, generator=g) * 0.02).abs() / 127
    return w_nk.t().contiguous(), s.to(torch.float16)


def w4(K: int, N: int, seed: int, group: int = 128, zeros: str = "none"):
    """packed uint8 [K/2, N] + fp16 scales [K/group, N] (+ uint8 zeros [K/group, N]).
    zeros: "none" (z = 8 implied), "eight" (explicit tensor of 8), "random"."""
    g = gen(seed)
    # a uniform byte is two independent uniform nibbles (low = even k, high = odd k)
    packed = torch.randint(0, 256, (K // 2, N), generator=g, dtype=torch.uint8)
    s = ((torch.randn((K // group, N), generator=g) * 0.02).abs() / 7).to(torch.float16)
    if zeros == "none":
        z = None
    elif zeros == "eight":
        z = torch.full((K // group, N), 8, dtype=torch.uint8)
    else:
        z = torch.randint(0, 16, (K // group, N), generator=g, dtype=torch.int32).to(torch.uint8)
    return packed, s, z


def engine_act(M: int, K: int, seed: int):
    """int8 a_q [M, K] and fp32 a_s [M, K/64] (.dev/test_kernels.py:34-36)."""
    g = gen(seed)
    a = torch.randint(-127, 127, (M, K), generator=g, dtype=torch.int8)
    s = torch.rand((M, K // 64), generator=g) * 0.02
    return a, s


def engine_w8(K: int, N: int, seed: int):
    """int8 [K, N] and fp32 per-column scales (.dev/test_kernels.py:35-37)."""
    g = gen(seed)
    b = torch.randint(-127, 127, (K, N), generator=g, dtype=torch.int8)
    s = torch.rand(N, generator=g) * 0.002
    return b, s


def np_(t):
    """torch CPU tensor -> numpy (bf16 as uint16 bit patterns)."""
    if t is None:
        return None
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def sample_cols(N: int, max_cols: int, seed: int = 0) -> np.ndarray:
    """All columns if N <= max_cols, else a sorted random subset of whole 16-column
    blocks (columns are independent, so the oracle only needs those)."""
    if N <= max_cols:
        return np.arange(N)
    rng = np.random.default_rng(seed)
    blocks = rng.choice(N // 16, size=max_cols // 16, replace=False)
    blocks.sort()
    return (blocks[:, None] * 16 + np.arange(16)[None, :]).reshape(-1)


def linear_w8_ref_cols(x, w, s, cols, residual=None):
    return R.linear_w8_ref(np_(x), np_(w)[:, cols], np_(s)[cols],
                           None if residual is None else np_(residual)[:, cols])


def linear_w4_ref_cols(x, packed, s, z, cols, residual=None):
    zz = None if z is None else np_(z)[:, cols]
    return R.linear_w4_ref(np_(x), np_(packed)[:, cols], np_(s)[:, cols], zz,
                           None if residual is None else np_(residual)[:, cols])


def to_f32(t) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def half_ulp(ref, dtype) -> np.ndarray:
    """Half a unit in the last place of `ref` in the 16-bit output type."""
    mant = {torch.float16: 10, torch.bfloat16: 7}[dtype]
    a = np.abs(np.asarray(ref, dtype=np.float64))
    _, e = np.frexp(a)                      # a = m * 2**e, m in [0.5, 1)
    ulp = np.ldexp(1.0, e - 1 - mant)
    if dtype == torch.float16:
        ulp = np.maximum(ulp, 2.0 ** -24)  # subnormal spacing
    return 0.5 * ulp


def assert_out_close(y: torch.Tensor, ref, tol: float = 2e-3) -> None:
    """The kernel's result must be within `tol * max|ref|` of the fp32 oracle before
    it is rounded to the 16-bit output type; the rounding adds at most half an ulp.
    (A bf16 output alone carries up to 2**-8 relative rounding, so a plain 2e-3
    normalized bound could not hold for it.)"""
    y32 = y.detach().float().cpu().numpy().astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    allowed = tol * np.abs(ref).max() + half_ulp(ref, y.dtype)
    err = np.abs(y32 - ref)
    bad = err > allowed
    if bad.any():
        i = np.unravel_index(np.argmax(err - allowed), err.shape)
        raise AssertionError(
            f"{int(bad.sum())} elements out of tolerance; worst at {i}: y={y32[i]} ref={ref[i]} "
            f"allowed={allowed[i]:.3e}; max_rel_err={R.max_rel_err(y32, ref):.3e} "
            f"rel_l2={R.rel_l2(y32, ref):.3e}")
