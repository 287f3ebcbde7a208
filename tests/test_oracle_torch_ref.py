"""Pins oracle/torch_ref.py (the torch-CPU restatement of the reference's
dequantize + F.linear that bench.py times as the CPU baseline): its
dequantized weights equal the C / numpy oracle's bit for bit (both are exact
products q * s), with padding sliced off, and its linear agrees with the
float64 product to fp32 accuracy."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import gaussian
from oracle import quant, torch_ref


@pytest.mark.parametrize("k,g", [(256, 128), (300, 128), (96, 32), (7, 2)])
def test_int4_dequant_matches_oracle(k, g):
    w = gaussian((37, k), seed=k + g)
    p, s, kp = quant.c_quantize_int4(w, g)
    got = torch_ref.dequantize_int4(torch.from_numpy(p), torch.from_numpy(s), k, g).numpy()
    ref = quant.c_dequantize_int4(p, s, k, g)
    assert got.shape == (37, k)
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def test_int8_dequant_matches_oracle():
    w = gaussian((41, 333), seed=5)
    p, s = quant.c_quantize_int8(w)
    got = torch_ref.dequantize_int8(torch.from_numpy(p), torch.from_numpy(s)).numpy()
    ref = quant.c_dequantize_int8(p, s)
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_linear_matches_float64(scheme):
    n, k, m = 64, 384, 5
    w = gaussian((n, k), seed=9)
    x = gaussian((m, k), seed=10, std=1.0)
    b = gaussian((n,), seed=11)
    if scheme == "int8":
        p, s = quant.c_quantize_int8(w)
        w_hat = quant.c_dequantize_int8(p, s)
    else:
        p, s, _ = quant.c_quantize_int4(w, 128)
        w_hat = quant.c_dequantize_int4(p, s, k, 128)
    y = torch_ref.linear(torch.from_numpy(x), torch.from_numpy(p), torch.from_numpy(s), scheme, k,
                         128, torch.from_numpy(b)).numpy()
    y64 = quant.linear_f64(x, w_hat, b)
    mag = np.abs(x.astype(np.float64)) @ np.abs(w_hat.astype(np.float64)).T + np.abs(b)
    assert (np.abs(y - y64) / mag).max() < 1e-5
