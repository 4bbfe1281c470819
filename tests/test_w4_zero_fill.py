"""W4 calls with zeros for only some of their weights (host logic, no GPU).

The reference runs such a call with zeros for every weight: each missing zero tensor
is replaced by the first given one (kernels/w4.py:235-241 for proj3_w4, 309-314 for
mlp_gate_up_quant_w4), which the kernel reads at `Z + srow * SW + cn` with the
weight's own row stride SW = N and column cn (kernels/w4.py:82-83).  `fill_zeros`
hands the kernels exactly those values as an explicit [K/group, N] tensor.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch


def _w4():
    from qwen35_amd.kernels import w4
    return w4


def _z(rows, n, seed):
    return torch.randint(0, 16, (rows, n), generator=torch.Generator().manual_seed(seed), dtype=torch.uint8)


def test_all_or_none_pass_through():
    w4 = _w4()
    s1, s2 = torch.zeros(16, 64), torch.zeros(16, 32)
    z1, z2 = _z(16, 64, 1), _z(16, 32, 2)
    assert w4.fill_zeros((None, None), (s1, s2), None) == [None, None]
    out = w4.fill_zeros((z1, z2), (s1, s2), z1)
    assert out[0] is z1 and out[1] is z2


def test_missing_zeros_read_the_fill_with_their_own_strides():
    w4 = _w4()
    rows = 16
    z1 = _z(rows, 64, 3)
    s = (torch.zeros(rows, 64), torch.zeros(rows, 48), torch.zeros(rows, 16))
    out = w4.fill_zeros((z1, None, None), s, z1)
    flat = z1.numpy().reshape(-1)
    for z, n in zip(out[1:], (48, 16)):
        assert z.dtype == torch.uint8 and tuple(z.shape) == (rows, n) and z.is_contiguous()
        # the element the reference's kernel loads for group row r, column c
        want = np.array([[flat[r * n + c] for c in range(n)] for r in range(rows)], dtype=np.uint8)
        assert np.array_equal(z.numpy(), want)
    # an absent projection (no scale) gets no zeros
    out = w4.fill_zeros((z1, None, None), (s[0], s[1], None), z1)
    assert out[2] is None


def test_gate_up_one_zero_tensor_stands_in_for_the_other():
    w4 = _w4()
    s = torch.zeros(16, 64)
    zg = _z(16, 64, 4)
    g, u = w4.fill_zeros((zg, None), (s, s), zg)
    assert g is zg and torch.equal(u, zg)
    g, u = w4.fill_zeros((None, zg), (s, s), zg)
    assert torch.equal(g, zg) and u is zg


def test_fill_too_small_is_refused():
    """A wider missing grid than the given zeros: the reference would read past the end
    of the given tensor; refused before any launch."""
    w4 = _w4()
    z2 = _z(16, 32, 5)
    with pytest.raises(ValueError, match="cannot stand in"):
        w4.fill_zeros((None, z2, None), (torch.zeros(16, 64), torch.zeros(16, 32), None), z2)
