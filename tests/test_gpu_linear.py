"""GPU parity: the fused dequant-matmul vs the oracle.

Reference value: ``x @ (q * s)^T + b`` in float64 over the oracle's exact
dequantized weight (engine/quantization.py:394-396 evaluated without
rounding).  Bars, written per test:

* norm-wise:     max|y - y64| / max|y64|            <= 1e-4   (the target is 1e-3)
* element-wise:  |y - y64| <= 1e-4 * (|x| @ |w_hat|^T + |b|)  (condition-aware,
                 so outputs that cancel to ~0 are still checked)

The measured worst case of every test is printed (``-s``) and recorded in the
design notes.  Bias / no bias, N not a multiple of 16, strided and 3-D inputs,
both MFMA paths (M <= 16 skinny, M > 16 tiled GEMM) and the generic fallback
(other group sizes, K not a multiple of 64) are covered.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn

from cases import LLAMA3_8B_SHAPES, gaussian, with_outliers
from kshipra_amd.quantization import (FusedQuantizedLinear, QuantizedLinear,
                                      quantize_int4_per_group, quantize_int8_per_channel,
                                      quantized_linear, quantized_linear_argmax)
from oracle import quant

pytestmark = pytest.mark.gpu

NORM_TOL = 1e-4
ELEM_TOL = 1e-4


def _reference(x: np.ndarray, w: np.ndarray, scheme: str, g: int, b):
    if scheme == "int8":
        w_hat = quant.c_dequantize_int8(*quant.c_quantize_int8(w))
    else:
        p, s, _ = quant.c_quantize_int4(w, g)
        w_hat = quant.c_dequantize_int4(p, s, w.shape[1], g)
    y64 = quant.linear_f64(x, w_hat, b)
    mag = np.abs(x.astype(np.float64)) @ np.abs(w_hat.astype(np.float64)).T
    if b is not None:
        mag = mag + np.abs(b.astype(np.float64))
    return y64, mag


def _compare(y: torch.Tensor, y64: np.ndarray, mag: np.ndarray, label: str):
    yn = y.detach().cpu().numpy().astype(np.float64).reshape(y64.shape)
    err = np.abs(yn - y64)
    norm_err = err.max() / max(np.abs(y64).max(), 1e-30)
    elem_err = (err / np.maximum(mag, 1e-30)).max()
    print(f"[{label}] norm-wise {norm_err:.3e}  element-wise {elem_err:.3e}", flush=True)
    assert norm_err <= NORM_TOL, (label, norm_err)
    assert elem_err <= ELEM_TOL, (label, elem_err)
    return norm_err


def _run(gpu, m, n, k, scheme, g=128, bias=True, seed=0, outliers=False):
    """Quantize one seeded weight, run every batch size in ``m`` (int or list)."""
    ms = [m] if isinstance(m, int) else list(m)
    w = gaussian((n, k), seed=seed)
    if outliers:
        w = with_outliers(w, seed + 1)
    b = gaussian((n,), seed=seed + 3) if bias else None
    wt = torch.from_numpy(w).to(gpu)
    qw = quantize_int8_per_channel(wt) if scheme == "int8" else quantize_int4_per_group(wt, g)
    del wt
    worst = 0.0
    for mm in ms:
        x = gaussian((mm, k), seed=seed + 2 + mm, std=1.0)
        y = quantized_linear(torch.from_numpy(x).to(gpu), qw,
                             None if b is None else torch.from_numpy(b).to(gpu))
        torch.cuda.synchronize()
        y64, mag = _reference(x, w, scheme, g, b)
        worst = max(worst, _compare(y, y64, mag, f"{scheme} m={mm} n={n} k={k} g={g}"))
    return worst


@pytest.mark.parametrize("scheme", ["int8", "int4"])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 13, 16])
def test_skinny_paths(gpu, scheme, m):
    _run(gpu, m, 272, 896, scheme, seed=m)              # K = 896: 7 groups / 14 windows
    _run(gpu, m, 100, 4864, scheme, seed=m + 50)        # N % 16 != 0, odd unit counts
    # INT4: K = 4000 ends 32 columns into its last group (the tail is staged as
    # zeros; regression for stale staging there); INT8 takes the generic path
    _run(gpu, m, 200, 4000, scheme, seed=m + 90)


@pytest.mark.parametrize("m,n,k,scheme", [
    (3, 4096, 14336, "int8"),    # down_proj at the split's smallest M
    (5, 4096, 14336, "int8"),    # two workgroups per CU from M = 5: 8 slices
    (6, 4096, 14336, "int4"),
    (4, 4096, 14336, "int4"),    # down_proj: 4 K slices of 28 groups
    (8, 4096, 14336, "int8"),    # 8 slices of 28 windows
    (16, 4096, 14336, "int4"),   # split rows (no hi / lo pairing), 16 slices
    (12, 1000, 8100, "int4"),    # K tail inside the last slice, N % 64 != 0
    (5, 300, 9024, "int8"),      # 47 slices of 3 windows
    (2, 4096, 14336, "int4"),    # below the split's M: whole-K workgroups
    (8, 28672, 4096, "int4"),    # below the split's K: whole-K workgroups
    (2, 28672, 4096, "int8"),    # M <= 4: two tiles per workgroup, LDS staging
    (4, 14336, 4096, "int4"),    # 66 KiB staged per workgroup, two per CU
])
def test_skinny_k_split(gpu, m, n, k, scheme):
    """Skinny launches whose K is split across workgroup rows (partials in the
    workspace, reduced in slice order with the bias), and their unsplit
    neighbours: aligned activations with bias, unaligned without."""
    w = gaussian((n, k), seed=n + k + m)
    b = gaussian((n,), seed=n + k + m + 1)
    wt = torch.from_numpy(w).to(gpu)
    qw = quantize_int8_per_channel(wt) if scheme == "int8" else quantize_int4_per_group(wt, 128)
    del wt
    xs = torch.from_numpy(gaussian((m, k + 1), seed=n + k + m + 2, std=1.0)).to(gpu)
    for name, x, bias in (("aligned", xs[:, :k].contiguous(), b), ("unaligned", xs[:, 1:], None)):
        y = quantized_linear(x, qw, None if bias is None else torch.from_numpy(bias).to(gpu))
        torch.cuda.synchronize()
        y64, mag = _reference(x.cpu().numpy(), w, scheme, 128, bias)
        _compare(y, y64, mag, f"k-split {scheme} m={m} n={n} k={k} {name}")


@pytest.mark.parametrize("n,k,scheme", [
    (6144, 4096, "int4"), (6150, 4096, "int8"),   # q+k+v; last workgroup with one partial tile
    (14336, 4096, "int8"), (6200, 4096, "int4"),  # gate / up; N % 32 == 24
])
def test_m1_two_tile_waves(gpu, n, k, scheme):
    """M = 1 with two 16-column tiles per wave (8-wave workgroups): bias and
    no bias, aligned and unaligned activations, and the fused greedy argmax
    over the same launch shape."""
    w = gaussian((n, k), seed=n + k)
    b = gaussian((n,), seed=n + k + 1)
    wt = torch.from_numpy(w).to(gpu)
    qw = quantize_int8_per_channel(wt) if scheme == "int8" else quantize_int4_per_group(wt, 128)
    del wt
    xs = torch.from_numpy(gaussian((1, k + 1), seed=n + k + 2, std=1.0)).to(gpu)
    for name, x, bias in (("aligned", xs[:, :k].contiguous(), b), ("unaligned", xs[:, 1:], None)):
        bt = None if bias is None else torch.from_numpy(bias).to(gpu)
        y = quantized_linear(x, qw, bt)
        torch.cuda.synchronize()
        y64, mag = _reference(x.cpu().numpy(), w, scheme, 128, bias)
        _compare(y, y64, mag, f"two-tile {scheme} n={n} k={k} {name}")
        tok = quantized_linear_argmax(x, qw, bt).reshape(-1).cpu()
        assert torch.equal(tok, y.argmax(dim=-1).reshape(-1).cpu()), name


@pytest.mark.parametrize("scheme", ["int8", "int4"])
@pytest.mark.parametrize("m", [17, 32, 40, 64, 100, 256, 512])
def test_gemm_paths(gpu, scheme, m):
    _run(gpu, m, 320, 1024, scheme, seed=m)
    _run(gpu, m, 250, 640, scheme, seed=m + 9, bias=False)


@pytest.mark.parametrize("m", [24, 48, 70])
def test_gemm_padded_k(gpu, m):
    # INT4 K = 904 pads to 1024: the last stage holds 8-column chunks past K.
    _run(gpu, m, 48, 904, "int4", seed=m + 3)
    # Long K, few tiles: many K splits reduced in order.
    _run(gpu, m, 40, 8192, "int8", seed=m + 4)


@pytest.mark.parametrize("m,n,k,scheme", [(130, 80, 100, "int4"), (129, 300, 128, "int8"),
                                          (200, 70, 1280, "int4"), (256, 528, 384, "int8")])
def test_gemm_prefill_kernel_edges(gpu, m, n, k, scheme):
    """Prefill-sized M through the producer/consumer kernel: one or few K
    stages (shorter than the LDS ring), partial row and column tiles, splits."""
    _run(gpu, m, n, k, scheme, seed=m + n)


@pytest.mark.parametrize("m,n,k", [(512, 14400, 512), (300, 28700, 256)])
def test_gemm_wide_consumer_tiles(gpu, m, n, k):
    """INT4 grids that fill the GPU without a K split run 7 consumer waves
    (448-column tiles): last column tile partial, last row tile partial."""
    _run(gpu, m, n, k, "int4", seed=m + k)


@pytest.mark.parametrize("m,n,k,g,scheme", [(16, 512, 512, 32, "int4"), (3, 512, 512, 256, "int4"),
                                            (40, 96, 500, 128, "int4"), (4, 70, 100, 128, "int8"),
                                            (33, 70, 100, 64, "int4"), (2, 16, 1, 128, "int4"),
                                            (1, 1, 1, 128, "int8")])
def test_generic_fallback(gpu, m, n, k, g, scheme):
    _run(gpu, m, n, k, scheme, g=g, seed=k)


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_config1_matvec(gpu, scheme):
    """INT8 [4864 x 896] N(0, 0.02) seed 0 with x ~ N(0, 1) (and the INT4 twin)."""
    w = gaussian((4864, 896), seed=0)
    x = (torch.randn(896, generator=torch.Generator().manual_seed(1))).numpy()
    wt = torch.from_numpy(w).to(gpu)
    qw = quantize_int8_per_channel(wt) if scheme == "int8" else quantize_int4_per_group(wt, 128)
    y = quantized_linear(torch.from_numpy(x).to(gpu), qw)            # 1-D input
    assert y.shape == (4864,)
    y64, mag = _reference(x[None], w, scheme, 128, None)
    _compare(y[None], y64, mag, f"config1 {scheme}")


@pytest.mark.parametrize("scheme", ["int8", "int4"])
@pytest.mark.parametrize("name", list(LLAMA3_8B_SHAPES))
def test_llama3_8b_full_shapes(gpu, scheme, name):
    """Every Llama-3-8B projection at M = 1, 8, 32, 64 (continuous-batching decode)."""
    n, k = LLAMA3_8B_SHAPES[name]
    seed = 100 + list(LLAMA3_8B_SHAPES).index(name)
    _run(gpu, [1, 8, 32, 64], n, k, scheme, seed=seed, bias=False, outliers=(scheme == "int4"))


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_prefill_chunk_mlp(gpu, scheme):
    """INT4/INT8 prefill GEMM on the Llama-3-8B MLP with outliers: X [512 x 4096]
    through gate/up [14336 x 4096], then [512 x 14336] through down."""
    _run(gpu, 512, 14336, 4096, scheme, seed=3, bias=False, outliers=True)
    _run(gpu, 512, 4096, 14336, scheme, seed=4, bias=False, outliers=True)


def test_strided_and_batched_inputs(gpu):
    w = gaussian((200, 384), seed=1)
    qw = quantize_int4_per_group(torch.from_numpy(w).to(gpu), 128)
    xb = torch.from_numpy(gaussian((2, 5, 512), seed=2, std=1.0)).to(gpu)
    x = xb[..., 64:448]                                         # ldx = 512, 3-D
    y = quantized_linear(x, qw)
    assert y.shape == (2, 5, 200)
    y64, mag = _reference(x.reshape(10, 384).cpu().numpy(), w, "int4", 128, None)
    _compare(y.reshape(10, 200), y64, mag, "strided 3-D")
    assert quantized_linear(x[:, :0], qw).shape == (2, 0, 200)     # empty batch


def test_deterministic(gpu):
    for m in (1, 8, 64):
        w = torch.from_numpy(gaussian((4096, 4096), seed=m)).to(gpu)
        x = torch.randn(m, 4096, device=gpu)
        for qw in (quantize_int8_per_channel(w), quantize_int4_per_group(w, 128)):
            a, b = quantized_linear(x, qw), quantized_linear(x, qw)
            assert torch.equal(a, b)


def test_linearity_full_size(gpu):
    """Size-independent property at the Llama down shape: f(x1 + x2) = f(x1) + f(x2)."""
    w = torch.from_numpy(gaussian((4096, 14336), seed=9)).to(gpu)
    x1, x2 = torch.randn(1, 14336, device=gpu), torch.randn(1, 14336, device=gpu)
    for qw in (quantize_int8_per_channel(w), quantize_int4_per_group(w, 128)):
        lhs = quantized_linear(x1 + x2, qw)
        rhs = quantized_linear(x1, qw) + quantized_linear(x2, qw)
        assert ((lhs - rhs).abs().max() / rhs.abs().max()).item() < 1e-5


def test_low_precision_activations(gpu):
    w = torch.from_numpy(gaussian((256, 512), seed=5)).to(gpu)
    x = torch.randn(4, 512, device=gpu)
    qw = quantize_int4_per_group(w, 128)
    y32 = quantized_linear(x, qw)
    for dt in (torch.float16, torch.bfloat16):
        y = quantized_linear(x.to(dt), qw)
        assert y.dtype == dt
        ref = quantized_linear(x.to(dt).float(), qw)
        assert torch.equal(y, ref.to(dt))
    assert (y32 - quantized_linear(x.half(), qw).float()).abs().max() < 0.05


# ---------------------------------------------------------------------- #
# Kshipra tests/test_quantization.py:125-181 on the GPU path
# ---------------------------------------------------------------------- #


def _rel_l2(ref, y):
    return float((y - ref).norm() / ref.norm().clamp_min(1e-12))


def test_int8_linear_matches_fp32_reference(gpu):
    torch.manual_seed(4)
    lin = nn.Linear(512, 512, bias=True).to(gpu)
    x = torch.randn(16, 512, device=gpu)
    with torch.no_grad():
        y_ref = lin(x)
        y = QuantizedLinear(lin, scheme="int8")(x)
    assert _rel_l2(y_ref, y) < 2e-2


def test_int4_linear_matches_fp32_reference(gpu):
    torch.manual_seed(5)
    lin = nn.Linear(512, 512, bias=True).to(gpu)
    x = torch.randn(16, 512, device=gpu)
    with torch.no_grad():
        y_ref = lin(x)
        y = QuantizedLinear(lin, scheme="int4", group_size=128)(x)
    assert _rel_l2(y_ref, y) < 2.5e-1


def test_tighter_group_beats_looser_group(gpu):
    torch.manual_seed(6)
    lin = nn.Linear(512, 512, bias=False).to(gpu)
    x = torch.randn(16, 512, device=gpu)
    with torch.no_grad():
        y_ref = lin(x)
        r32 = _rel_l2(y_ref, QuantizedLinear(lin, "int4", 32)(x))
        r256 = _rel_l2(y_ref, QuantizedLinear(lin, "int4", 256)(x))
    assert r32 < r256


def test_linear_without_bias_and_repr(gpu):
    torch.manual_seed(7)
    lin = nn.Linear(128, 256, bias=False).to(gpu)
    x = torch.randn(4, 128, device=gpu)
    q = QuantizedLinear(lin, scheme="int8")
    assert q.bias is None
    with torch.no_grad():
        assert _rel_l2(lin(x), q(x)) < 2e-2
    assert "scheme=int8" in repr(q) and "storage_bytes=" in repr(q)


@pytest.mark.parametrize("scheme", ["int8", "int4"])
@pytest.mark.parametrize("m", [1, 5, 24, 100])
def test_fused_projections_match_parts(gpu, scheme, m):
    """q/k/v-like parts (one without bias) fused into one launch: every part's
    output against the float64 reference and against its own launch."""
    k = 896
    shapes = [(896, k, True), (128, k, False), (128, k, True)]
    lins = []
    for i, (n, kk, has_b) in enumerate(shapes):
        lin = nn.Linear(kk, n, bias=has_b, device=gpu)
        with torch.no_grad():
            lin.weight.copy_(torch.from_numpy(gaussian((n, kk), seed=40 + i)))
            if has_b:
                lin.bias.copy_(torch.from_numpy(gaussian((n,), seed=50 + i)))
        lins.append((lin, QuantizedLinear(lin, scheme=scheme)))
    fused = FusedQuantizedLinear([q for _, q in lins])
    x = torch.from_numpy(gaussian((m, k), seed=60 + m, std=1.0)).to(gpu)
    outs = fused(x)
    assert [o.shape for o in outs] == [(m, n) for n, _, _ in shapes]
    for (lin, q), o in zip(lins, outs):
        w = lin.weight.detach().cpu().numpy()
        b = lin.bias.detach().cpu().numpy() if lin.bias is not None else None
        y64, mag = _reference(x.cpu().numpy(), w, scheme, 128, b)
        _compare(o, y64, mag, f"fused part {scheme} m={m} n={w.shape[0]}")
        sep = q(x)
        assert torch.allclose(o, sep, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_operand_checks_before_launch(gpu, scheme):
    """Operands the kernels cannot read as given are converted or refused on
    the host, before any launch: a bias or scales left on the CPU raise
    RuntimeError (as F.linear does for mixed devices), float32 scales that
    fp16 holds exactly and a non-contiguous payload give the same result,
    inexact float32 scales raise QuantizationError."""
    from kshipra_amd.quantization import QuantizationError, QuantizedWeight
    n, k = 96, 256
    w = gaussian((n, k), seed=77)
    wt = torch.from_numpy(w).to(gpu)
    qw = quantize_int8_per_channel(wt) if scheme == "int8" else quantize_int4_per_group(wt, 128)
    x = torch.from_numpy(gaussian((3, k), seed=78, std=1.0)).to(gpu)
    b = torch.from_numpy(gaussian((n,), seed=79)).to(gpu)
    ref = quantized_linear(x, qw, b)
    with pytest.raises(RuntimeError):
        quantized_linear(x, qw, b.cpu())
    with pytest.raises(RuntimeError):
        quantized_linear(x, QuantizedWeight(qw.payload, qw.scales.cpu(), qw.scheme, qw.original_shape,
                                            qw.group_size, qw.in_features_padded), b)
    s32 = QuantizedWeight(qw.payload, qw.scales.float(), qw.scheme, qw.original_shape,
                          qw.group_size, qw.in_features_padded)
    assert torch.equal(quantized_linear(x, s32, b), ref)
    bad = QuantizedWeight(qw.payload, qw.scales.float() * (1 + 2 ** -20), qw.scheme,
                          qw.original_shape, qw.group_size, qw.in_features_padded)
    with pytest.raises(QuantizationError):
        quantized_linear(x, bad, b)
    strided = qw.payload.t().contiguous().t()                  # same values, column-major
    assert not strided.is_contiguous()
    nc = QuantizedWeight(strided, qw.scales, qw.scheme, qw.original_shape, qw.group_size,
                         qw.in_features_padded)
    assert torch.equal(quantized_linear(x, nc, b), ref)
    lin = nn.Linear(k, n, device=gpu)
    ql = QuantizedLinear(lin, scheme).cpu()                     # moves the bias buffer only
    with pytest.raises(RuntimeError):
        ql(x)


@pytest.mark.parametrize("n", [28672, 26000])
def test_single_row_wide(gpu, n):
    """INT4 M = 1 at the fused gate/up width [28672 x 4096] (more waves than
    one round of the chip holds) and at a ragged N; aligned and unaligned
    activations, bias."""
    _run(gpu, 1, n, 4096, "int4", bias=True, seed=n)
    w = gaussian((n, 4096), seed=n + 1)
    qw = quantize_int4_per_group(torch.from_numpy(w).to(gpu), 128)
    xs = torch.from_numpy(gaussian((1, 4097), seed=n + 2, std=1.0)).to(gpu)
    y = quantized_linear(xs[:, 1:], qw)
    torch.cuda.synchronize()
    y64, mag = _reference(xs[:, 1:].cpu().numpy(), w, "int4", 128, None)
    _compare(y, y64, mag, f"wide unaligned n={n}")
