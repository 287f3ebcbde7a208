"""GPU parity: quantize / pack / dequantize are bit-exact with the oracle.

Bar: payload and scales byte-identical to the C restatement of
engine/quantization.py:196-344 on the same seeded fp32 inputs, including
every adversarial branch (ties, zero rows, fp16-scale underflow -> +-inf ->
clamp, subnormal and overflowing scales), the configs' full shapes, fp16 /
bf16 inputs, strided inputs, and 24 seeded random shapes and value mixes
(scales 2^-30 .. 2^30, zero / constant / outlier / tie rows) at every group
size.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import LLAMA3_8B_SHAPES, adversarial_rows, gaussian, with_outliers
from kshipra_amd.quantization import (QuantizationError, _dequantize_int4_per_group,
                                      _dequantize_int8_per_channel, _validate_weight,
                                      quantize_int4_per_group, quantize_int8_per_channel)
from oracle import quant

pytestmark = pytest.mark.gpu


def _check_int8(w_np: np.ndarray, qw) -> None:
    q_ref, s_ref = quant.c_quantize_int8(w_np)
    assert qw.payload.dtype == torch.int8 and qw.scales.dtype == torch.float16
    assert np.array_equal(qw.scales.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(qw.payload.cpu().numpy(), q_ref)


def _check_int4(w_np: np.ndarray, qw, g: int) -> None:
    p_ref, s_ref, kp = quant.c_quantize_int4(w_np, g)
    assert qw.in_features_padded == kp and qw.group_size == g
    assert np.array_equal(qw.scales.cpu().numpy().view(np.uint16), s_ref.view(np.uint16))
    assert np.array_equal(qw.payload.cpu().numpy(), p_ref)


def _random_weight(i: int):
    """Seeded shape and value mix: Gaussian rows at scales 2^-30 .. 2^30,
    some rows with outliers, all-zero rows, rows of one repeated value and
    rows that put values exactly on rounding ties of their own scale."""
    rng = np.random.default_rng(31337 + i)
    n = int(rng.integers(1, 700))
    k = int(rng.integers(1, 3000)) if i % 3 else int(rng.choice([128, 896, 4096]))
    w = (rng.standard_normal((n, k)) * float(2.0 ** rng.integers(-30, 31))).astype(np.float32)
    for r in rng.choice(n, size=min(n, 4), replace=False):
        kind = int(rng.integers(4))
        if kind == 0:
            w[r] = 0.0
        elif kind == 1:
            w[r] = np.float32(rng.standard_normal())
        elif kind == 2:
            w[r, rng.integers(k)] *= 1000.0
        else:                                   # multiples of half a step of the row's int8 scale
            amax = max(float(np.abs(w[r]).max()), 1e-30)
            step = amax / 127.0
            w[r] = (rng.integers(-254, 255, size=k) * 0.5 * step).astype(np.float32)
    return w


@pytest.mark.parametrize("i", range(24))
def test_random_shapes_bit_exact(gpu, i):
    """Seeded random shapes and value mixes: INT8, and INT4 at a random
    supported group size, byte-identical with the oracle."""
    w = _random_weight(i)
    wd = torch.from_numpy(w).to(gpu)
    _check_int8(w, quantize_int8_per_channel(wd))
    g = [2, 32, 64, 128, 256][i % 5]
    _check_int4(w, quantize_int4_per_group(wd, g), g)


@pytest.mark.parametrize("k", [1, 7, 64, 128, 200, 896, 1000])
def test_int8_adversarial_bit_exact(gpu, k):
    w = adversarial_rows(np.random.default_rng(k), k)
    _check_int8(w, quantize_int8_per_channel(torch.from_numpy(w).to(gpu)))


@pytest.mark.parametrize("k,g", [(1, 128), (100, 128), (128, 128), (500, 128), (896, 128),
                                 (96, 32), (130, 2), (500, 256), (300, 64)])
def test_int4_adversarial_bit_exact(gpu, k, g):
    w = adversarial_rows(np.random.default_rng(k * 7 + g), k)
    _check_int4(w, quantize_int4_per_group(torch.from_numpy(w).to(gpu), g), g)


def test_config1_int8_qwen_gate(gpu):
    """INT8 [4864 x 896] N(0, 0.02), seed 0."""
    w = gaussian((4864, 896), seed=0)
    _check_int8(w, quantize_int8_per_channel(torch.from_numpy(w).to(gpu)))


@pytest.mark.parametrize("name", ["q_proj", "k_proj", "gate_proj", "down_proj"])
def test_llama3_8b_shapes_bit_exact(gpu, name):
    n, k = LLAMA3_8B_SHAPES[name]
    w = with_outliers(gaussian((n, k), seed=10 + list(LLAMA3_8B_SHAPES).index(name)), seed=1)
    wt = torch.from_numpy(w).to(gpu)
    _check_int8(w, quantize_int8_per_channel(wt))
    _check_int4(w, quantize_int4_per_group(wt, 128), 128)


def test_lm_head_shape_bit_exact(gpu):
    w = gaussian((128256, 4096), seed=5)
    wt = torch.from_numpy(w).to(gpu)
    _check_int4(w, quantize_int4_per_group(wt, 128), 128)
    _check_int8(w, quantize_int8_per_channel(wt))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float64])
def test_low_and_high_precision_inputs(gpu, dtype):
    """``w.to(float32)`` first (engine/quantization.py:205): fp16/bf16 -> fp32
    is exact; fp64 is rounded by torch exactly as the reference does."""
    w = torch.from_numpy(adversarial_rows(np.random.default_rng(1), 384)[:7]).to(dtype)
    w32 = w.to(torch.float32).numpy()
    _check_int8(w32, quantize_int8_per_channel(w.to(gpu)))
    _check_int4(w32, quantize_int4_per_group(w.to(gpu), 128), 128)


def test_strided_and_transposed_inputs(gpu):
    base = torch.from_numpy(gaussian((96, 640), seed=3)).to(gpu)
    view = base[:, 64:564]                                   # ldw = 640 > K = 500
    _check_int8(view.cpu().numpy(), quantize_int8_per_channel(view))
    _check_int4(view.cpu().numpy(), quantize_int4_per_group(view, 128), 128)
    tr = torch.from_numpy(gaussian((300, 200), seed=4)).to(gpu).t()   # column-major
    _check_int8(tr.cpu().numpy(), quantize_int8_per_channel(tr))


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
def test_non_finite_rejected(gpu, bad):
    w = torch.randn(33, 300)
    w[17, 211] = bad
    wg = w.to(gpu)
    with pytest.raises(QuantizationError):
        quantize_int8_per_channel(wg)
    with pytest.raises(QuantizationError):
        quantize_int4_per_group(wg, 128)
    with pytest.raises(QuantizationError):
        _validate_weight(wg)
    _validate_weight(torch.randn(33, 300, device=gpu))       # finite: no error


def test_dequantize_exact_and_rounded(gpu):
    w = adversarial_rows(np.random.default_rng(8), 500)
    w = w[np.isfinite(quant.c_quantize_int8(w)[1].astype(np.float32))]   # drop inf-scale rows
    wt = torch.from_numpy(w).to(gpu)
    q8 = quantize_int8_per_channel(wt)
    ref8 = quant.c_dequantize_int8(*quant.c_quantize_int8(w))
    got = _dequantize_int8_per_channel(q8).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref8.view(np.uint32))
    q4 = quantize_int4_per_group(wt, 128)
    p, s, _ = quant.c_quantize_int4(w, 128)
    ref4 = quant.c_dequantize_int4(p, s, 500, 128)
    got4 = _dequantize_int4_per_group(q4).cpu().numpy()
    assert got4.shape == (w.shape[0], 500)
    assert np.array_equal(got4.view(np.uint32), ref4.view(np.uint32))
    for dt in (torch.float16, torch.bfloat16):           # one RNE rounding of the exact product
        assert torch.equal(q8.dequantize(dt).cpu(), torch.from_numpy(ref8).to(dt))
        assert torch.equal(q4.dequantize(dt).cpu(), torch.from_numpy(ref4).to(dt))
    assert q8.dequantize().dtype == torch.float16           # the reference's default
    assert torch.equal(q8.dequantize(torch.float64).cpu(), torch.from_numpy(ref8).double())


def test_reference_known_answers_on_gpu(gpu):
    """Kshipra tests/test_quantization.py:212-245 on the GPU path."""
    qw = quantize_int8_per_channel(torch.tensor([[1.5]], device=gpu))
    w_hat = qw.dequantize(dtype=torch.float32)
    assert w_hat.shape == (1, 1)
    assert abs(float(w_hat) - 1.5) / 1.5 < 1e-3
    assert int(qw.payload.item()) == 127
    qw = quantize_int4_per_group(torch.tensor([[0.5], [-0.3]], device=gpu), 128)
    assert qw.dequantize(dtype=torch.float32).shape == (2, 1)
    qw = quantize_int8_per_channel(torch.zeros(4, 128, device=gpu))
    assert torch.all(qw.dequantize(dtype=torch.float32) == 0)
    qw = quantize_int4_per_group(torch.randn(16, 100, device=gpu), 128)
    assert qw.in_features_padded == 128


def test_storage_and_half_scale_bound(gpu):
    """tests/test_quantization.py:37-104 on GPU-quantized weights."""
    torch.manual_seed(0)
    w = torch.randn(4096, 4096, device=gpu)
    q8 = quantize_int8_per_channel(w)
    assert q8.storage_bytes() == 4096 * 4096 + 4096 * 2
    q4 = quantize_int4_per_group(w, 128)
    assert q4.storage_bytes() == 4096 * 2048 + 4096 * 32 * 2
    assert q4.storage_bytes() * 8 / w.numel() == pytest.approx(4.125, abs=1e-3)
    torch.manual_seed(1)
    w = torch.randn(64, 512, device=gpu)
    q = quantize_int8_per_channel(w)
    err = (w - q.dequantize(torch.float32)).abs().amax(dim=1)
    assert torch.all(err <= q.scales.float() / 2 + 1e-6)
    torch.manual_seed(2)
    w = torch.randn(32, 512, device=gpu)
    q = quantize_int4_per_group(w, 128)
    err = (w - q.dequantize(torch.float32)).abs().view(32, 4, 128).amax(dim=-1)
    assert torch.all(err <= q.scales.float() / 2 + 1e-6)
