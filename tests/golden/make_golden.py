"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no GEMM-level golden data (its kernel tests draw random CUDA
tensors and only print errors), so these vectors are produced by the oracle from
seeded numpy inputs; the oracle itself is pinned by tests/test_oracle.py.  Each .npz
holds the inputs and the expected outputs of one case.  bf16 tensors are stored as
uint16 bit patterns.
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import ref_cpu as R  # noqa: E402


def _rng(seed):
    return np.random.default_rng(seed)


def cases():
    out = {}
    # every byte value, two packed rows -> four nibble rows
    b = np.tile(np.arange(256, dtype=np.uint8), (2, 1))
    out["w4_unpack_all_bytes"] = dict(packed=b, nib=R.unpack_w4(b))

    r = _rng(101)
    x = r.standard_normal((3, 256)).astype(np.float16)
    w = r.integers(-127, 128, size=(256, 64), dtype=np.int8)
    s = (np.abs(r.normal(0, 0.02, 64)) / 127).astype(np.float16)
    out["a16_w8"] = dict(x=x, w=w, s=s, y=R.linear_w8_ref(x, w, s))

    r = _rng(102)
    x = r.standard_normal((3, 256)).astype(np.float16)
    p = r.integers(0, 256, size=(128, 64), dtype=np.uint8)
    s = (np.abs(r.normal(0, 0.02, (2, 64))) / 7).astype(np.float16)
    z = r.integers(0, 16, size=(2, 64), dtype=np.uint8)
    out["a16_w4_g128_zeros"] = dict(x=x, w=p, s=s, z=z, y=R.linear_w4_ref(x, p, s, z),
                                    dq=R.dequant_w4_f32(p, s, z))

    r = _rng(103)
    a = r.integers(-127, 127, size=(5, 256), dtype=np.int8)
    a_s = (r.random((5, 4)) * 0.02).astype(np.float32)
    bw = r.integers(-127, 127, size=(256, 64), dtype=np.int8)
    bs = (r.random(64) * 0.002).astype(np.float32)
    res = R.f32_to_bf16_bits(r.standard_normal((5, 64)).astype(np.float32))
    out["engine_gemm_i8_res"] = dict(a_q=a, a_s=a_s, b=bw, b_s=bs, res=res,
                                     y=R.gemm_i8_ref(a, a_s, bw, bs, residual=res))

    r = _rng(104)
    a = r.integers(-127, 127, size=(4, 256), dtype=np.int8)
    a_s = (r.random((4, 4)) * 0.02).astype(np.float32)
    p = r.integers(0, 256, size=(128, 64), dtype=np.uint8)
    s = R.f32_to_bf16_bits((np.abs(r.normal(0, 0.02, (4, 64))) / 7).astype(np.float32))  # G = 64
    z = r.integers(0, 16, size=(4, 64), dtype=np.uint8)
    out["engine_gemm_w4_g64_zeros"] = dict(a_q=a, a_s=a_s, b=p, b_s=s, b_z=z,
                                           y=R.gemm_w4_ref(a, a_s, p, s, b_z=z))

    r = _rng(105)
    a = r.integers(-127, 127, size=(3, 128), dtype=np.int8)
    a_s = (r.random((3, 2)) * 0.02).astype(np.float32)
    ws = [r.integers(-127, 127, size=(128, n), dtype=np.int8) for n in (64, 32, 32)]
    ss = [(r.random(w_.shape[1]) * 0.002).astype(np.float32) for w_ in ws]
    out["engine_proj3_i8"] = dict(a_q=a, a_s=a_s, w1=ws[0], s1=ss[0], w2=ws[1], s2=ss[1], w3=ws[2],
                                  s3=ss[2], y=R.proj3_ref(a, a_s, ws[0], ss[0], ws[1], ss[1], ws[2], ss[2]))

    r = _rng(106)
    a = r.integers(-127, 127, size=(3, 256), dtype=np.int8)
    a_s = (r.random((3, 4)) * 0.02).astype(np.float32)
    wg = r.integers(-127, 127, size=(256, 128), dtype=np.int8)
    wu = r.integers(-127, 127, size=(256, 128), dtype=np.int8)
    sg = (r.random(128) * 0.002).astype(np.float32)
    su = (r.random(128) * 0.002).astype(np.float32)
    h = R.mlp_gate_up_ref(a, a_s, wg, sg, wu, su)
    q, qs = R.mlp_gate_up_quant_ref(a, a_s, wg, sg, wu, su)
    out["engine_gate_up_quant_i8"] = dict(a_q=a, a_s=a_s, wg=wg, sg=sg, wu=wu, su=su, h=h, q=q, qs=qs)
    return out


def main():
    for name, arrays in cases().items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(name, {k: (v.dtype.name, v.shape) for k, v in arrays.items()})


if __name__ == "__main__":
    main()
