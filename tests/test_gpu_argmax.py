"""Greedy token of a quantized projection (engine/model.py:151 logits,
:187/:200 ``int(logits[..].argmax())``) computed in the dequant-GEMV epilogue.

Bars: the fused tokens equal torch.argmax over the logits the same call
returns (bit-identical logits, so exact), and over the float64 reference
logits; ties go to the first index; a NaN row returns torch's answer.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import gaussian
from kshipra_amd.quantization import (quantize_int4_per_group, quantize_int8_per_channel,
                                      quantized_linear, quantized_linear_argmax)
from oracle import quant

pytestmark = pytest.mark.gpu


def _qw(w, scheme, gpu):
    wt = torch.from_numpy(w).to(gpu)
    return quantize_int8_per_channel(wt) if scheme == "int8" else quantize_int4_per_group(wt, 128)


@pytest.mark.parametrize("scheme", ["int8", "int4"])
@pytest.mark.parametrize("m,n,k", [(1, 1000, 512), (3, 5, 256), (16, 4099, 640), (17, 777, 384),
                                   (40, 2100, 1024), (200, 515, 256), (1, 70000, 128)])
def test_fused_argmax_matches_logits(gpu, scheme, m, n, k):
    w = gaussian((n, k), seed=n + k)
    b = gaussian((n,), seed=n)
    qw = _qw(w, scheme, gpu)
    x = torch.from_numpy(gaussian((m, k), seed=m, std=1.0)).to(gpu)
    bt = torch.from_numpy(b).to(gpu)
    tok, logits = quantized_linear_argmax(x, qw, bt, return_logits=True)
    assert tok.dtype == torch.int64 and tok.shape == (m,)
    assert torch.equal(tok, logits.argmax(dim=-1))
    assert torch.equal(logits, quantized_linear(x, qw, bt))
    tok_only = quantized_linear_argmax(x, qw, bt)                # logits never written
    assert torch.equal(tok_only, tok)
    if scheme == "int8":
        w_hat = quant.c_dequantize_int8(*quant.c_quantize_int8(w))
    else:
        p, s, _ = quant.c_quantize_int4(w, 128)
        w_hat = quant.c_dequantize_int4(p, s, k, 128)
    y64 = quant.linear_f64(x.cpu().numpy(), w_hat, b)
    assert np.array_equal(tok.cpu().numpy(), y64.argmax(axis=-1))


@pytest.mark.parametrize("scheme", ["int8", "int4"])
@pytest.mark.parametrize("m", [1, 20])
def test_ties_go_to_the_first_index(gpu, scheme, m):
    """Identical rows give bit-identical logits: the smaller index wins,
    also across tiles and workgroups."""
    n, k = 5000, 256
    w = gaussian((n, k), seed=3) * 0.1
    hot = np.abs(gaussian((k,), seed=4, std=1.0)) + 0.5
    for r in (4321, 700, 4999, 33):
        w[r] = hot                                              # four identical maxima
    qw = _qw(w, scheme, gpu)
    x = torch.ones(m, k, device=gpu)
    tok, logits = quantized_linear_argmax(x, qw, return_logits=True)
    assert (logits[:, [33, 700, 4321, 4999]] == logits[:, 33:34]).all()
    assert (tok == 33).all()


def test_nan_row_follows_torch(gpu):
    w = gaussian((3000, 256), seed=8)
    qw = quantize_int4_per_group(torch.from_numpy(w).to(gpu), 128)
    x = torch.randn(3, 256, device=gpu)
    x[1, 17] = float("nan")
    tok, logits = quantized_linear_argmax(x, qw, return_logits=True)
    assert torch.isnan(logits[1]).all()
    assert torch.equal(tok, logits.argmax(dim=-1))


def test_batched_shape(gpu):
    w = gaussian((900, 128), seed=9)
    qw = quantize_int8_per_channel(torch.from_numpy(w).to(gpu))
    x = torch.randn(2, 3, 128, device=gpu)
    tok = quantized_linear_argmax(x, qw)
    assert tok.shape == (2, 3)
    assert torch.equal(tok, quantized_linear(x, qw).argmax(dim=-1))
