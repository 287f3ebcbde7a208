"""GPU parity of the dequant-matmul over the whole fp32 activation range.

The reference forward is ``F.linear(x, w_hat, b)`` in fp32
(engine/quantization.py:394-396), exact in its products for every finite x.
The MFMA paths feed x to fp16 matrix cores as hi + lo halves of x scaled by a
per-row (or per row-slice) power of two; these tests drive that scaling at the
edges of the fp32 range on every path that stages activations:

* skinny M = 1 (single-row instances, INT4) and the general instances (INT8);
* skinny M = 2..16 with pre-loads only and with the remainder (unaligned x);
* skinny with the staging pre-pass (rows too long for LDS);
* skinny with K split across workgroups (down_proj shapes);
* the tiled GEMM (M = 17..64) and the warp-specialised GEMM (prefill);
* the SiLU-gated gate / up epilogue and the fused greedy argmax.

Inputs: N(0, 1) rows scaled by 2^+-30, 2^+-100, 1e5, 1e-6, 2^-140 (fp32
subnormals), rows mixing 1e-6 and 6e4 entries, all-zero rows, and a batch
whose rows differ by 2^60 in magnitude.  Bars are the linear tests' own
(float64 reference over the exact dequantized weight): max|y - y64| /
max|y64| <= 1e-4 and |y - y64| <= 1e-4 (|x| @ |w_hat|^T) element-wise, no
NaN or inf where the reference is finite.  Non-finite activations must give
the reference's IEEE pattern (+-inf, or NaN for inf * 0 and inf - inf).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import gaussian
from kshipra_amd import _lib
from kshipra_amd.quantization import (interleave_gate_up, quantize_int4_per_group,
                                      quantize_int8_per_channel, quantized_gate_up_silu,
                                      quantized_linear, quantized_linear_argmax)
from oracle import quant

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _w_hat(w: np.ndarray, scheme: str) -> np.ndarray:
    if scheme == "int8":
        return quant.c_dequantize_int8(*quant.c_quantize_int8(w)).astype(np.float64)
    p, s, _ = quant.c_quantize_int4(w, 128)
    return quant.c_dequantize_int4(p, s, w.shape[1], 128).astype(np.float64)


def _quantize(w: np.ndarray, scheme: str, gpu):
    wt = torch.from_numpy(w).to(gpu)
    return quantize_int8_per_channel(wt) if scheme == "int8" else quantize_int4_per_group(wt, 128)


def _scaled_inputs(m: int, k: int, seed: int):
    """(label, x fp32 [m, k]) pairs covering the range edges."""
    base = gaussian((m, k), seed=seed, std=1.0).astype(np.float64)
    out = []
    for label, f in (("x2^30", 2.0 ** 30), ("x2^-30", 2.0 ** -30), ("x2^100", 2.0 ** 100),
                     ("x2^-100", 2.0 ** -100), ("x1e5", 1e5), ("x1e-6", 1e-6),
                     ("subnormal", 2.0 ** -140)):
        out.append((label, (base * f).astype(np.float32)))
    mixed = (base * 1e-6).astype(np.float32)
    rng = np.random.default_rng(seed)
    hot = rng.random((m, k)) < 0.02
    mixed[hot] = (np.sign(base[hot]) * 6e4).astype(np.float32)
    out.append(("mixed 1e-6 / 6e4", mixed))
    rows = base.copy()
    rows *= (2.0 ** (60 * (np.arange(m) % 3 - 1)))[:, None]      # rows at 2^-60, 1, 2^60
    if m > 1:
        rows[m // 2] = 0.0                                         # an all-zero row
    out.append(("rows 2^-60 / 1 / 2^60 + zero row", rows.astype(np.float32)))
    return out


def _check(y: np.ndarray, x: np.ndarray, w_hat: np.ndarray, label: str):
    x64 = x.astype(np.float64)
    y64 = x64 @ w_hat.T
    mag = np.abs(x64) @ np.abs(w_hat).T
    y = y.astype(np.float64).reshape(y64.shape)
    assert np.isfinite(y).all(), f"{label}: non-finite output where the reference is finite"
    # fp32 cannot hold an output below 2^-126 to 1e-4 relative.  There the
    # kernels round each wave's and each K slice's partial sum once (at most
    # 16 waves + 16 slices + the output), 2^-150 each: allow 2^-144 absolute
    # on top of the bars (the fp32 reference rounds every one of its K
    # products at that spacing).
    err = np.maximum(np.abs(y - y64) - 2.0 ** -144, 0.0)
    # norm-wise per row: rows of very different magnitude are each held to the bar
    rmax = np.maximum(np.abs(y64).max(axis=1, keepdims=True), 1e-300)
    norm = (err / rmax)[np.abs(y64).max(axis=1) > 0].max(initial=0.0)
    elem = np.where(mag > 0, err / np.where(mag > 0, mag, 1.0), err).max()
    zero_rows = ~np.any(x64 != 0, axis=1)
    assert not np.any(y[zero_rows]), f"{label}: an all-zero row gave a nonzero output"
    print(f"[range {label}] norm-wise {norm:.3e} element-wise {elem:.3e}", flush=True)
    assert norm <= TOL and elem <= TOL, (label, norm, elem)


# (m, n, k, scheme, aligned): which staging path each one takes is asserted
# through the workspace size where the library exposes it.
CASES = [
    (1, 4096, 4096, "int4", True),      # single-row skinny instance
    (1, 28672, 4096, "int4", True),     # single-row, wider than one round of waves
    (1, 4096, 4096, "int8", True),      # general skinny instance at M = 1
    (3, 1024, 4096, "int4", True),      # pre-loads cover every entry
    (8, 1024, 4096, "int8", False),     # remainder staging (unaligned x)
    (13, 512, 4096, "int4", False),     # split hi / lo rows, remainder
    (8, 20480, 4096, "int4", True),     # staging pre-pass (workspace)
    (8, 4096, 14336, "int8", True),     # K split across workgroups
    (6, 4096, 14336, "int4", False),
    (32, 2048, 4096, "int4", True),     # tiled GEMM
    (64, 2048, 4096, "int8", False),
    (96, 2048, 4096, "int4", True),     # warp-specialised GEMM
    (80, 1024, 2048, "int8", True),
]


@pytest.mark.parametrize("m,n,k,scheme,aligned", CASES)
def test_linear_activation_range(gpu, m, n, k, scheme, aligned):
    w = gaussian((n, k), seed=n + k + m)
    qw = _quantize(w, scheme, gpu)
    w_hat = _w_hat(w, scheme)
    if (m, n) == (8, 20480):
        assert _lib.load().kq_linear_workspace_bytes(4, m, n, k, 128) > 0   # pre-pass staging
    for label, x in _scaled_inputs(m, k, seed=m + k):
        xt = torch.from_numpy(np.concatenate([np.zeros((m, 1), np.float32), x], 1)).to(gpu)
        xin = xt[:, 1:] if not aligned else xt[:, 1:].contiguous()
        y = quantized_linear(xin, qw)
        torch.cuda.synchronize()
        _check(y.cpu().numpy(), x, w_hat, f"{scheme} m={m} n={n} k={k} {label}")


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_bias_with_scaled_activations(gpu, scheme):
    """The bias is added after the scale is undone: with x at 2^30 and the
    bias at the same magnitude both contribute."""
    m, n, k = 4, 512, 1024
    w = gaussian((n, k), seed=5)
    b = (gaussian((n,), seed=6, std=1.0) * 2.0 ** 30).astype(np.float32)
    x = (gaussian((m, k), seed=7, std=1.0) * 2.0 ** 30).astype(np.float32)
    qw = _quantize(w, scheme, gpu)
    for mm in (m, 40):
        xs = np.tile(x, (mm // m, 1))
        y = quantized_linear(torch.from_numpy(xs).to(gpu), qw, torch.from_numpy(b).to(gpu)).cpu().numpy()
        w_hat = _w_hat(w, scheme)
        y64 = xs.astype(np.float64) @ w_hat.T + b
        mag = np.abs(xs.astype(np.float64)) @ np.abs(w_hat).T + np.abs(b)
        elem = (np.abs(y - y64) / mag).max()
        print(f"[range bias {scheme} m={mm}] element-wise {elem:.3e}", flush=True)
        assert elem <= TOL


@pytest.mark.parametrize("scheme", ["int8", "int4"])
@pytest.mark.parametrize("m", [1, 5, 24])
def test_gate_up_silu_activation_range(gpu, scheme, m):
    """SiLU pair epilogue (skinny) and the pairing kernel (GEMM) with x at
    2^-40 and 2^20: the gate sees the unscaled products."""
    nh, k = 512, 1024
    wg, wu = gaussian((nh, k), seed=21), gaussian((nh, k), seed=22)
    qw = interleave_gate_up(_quantize(wg, scheme, gpu), _quantize(wu, scheme, gpu))
    hg, hu = _w_hat(wg, scheme), _w_hat(wu, scheme)
    for f in (2.0 ** -40, 2.0 ** -8, 2.0 ** 20):
        x = (gaussian((m, k), seed=23, std=1.0) * f).astype(np.float32)
        a = quantized_gate_up_silu(torch.from_numpy(x).to(gpu), qw).cpu().numpy().astype(np.float64)
        x64 = x.astype(np.float64)
        g, u = x64 @ hg.T, x64 @ hu.T
        mg, mu = np.abs(x64) @ np.abs(hg).T, np.abs(x64) @ np.abs(hu).T
        with np.errstate(over="ignore"):
            sig = 1.0 / (1.0 + np.exp(-g))
        a64 = g * sig * u
        bound = np.abs(sig * (1.0 + g * (1.0 - sig))) * np.abs(u) * mg + np.abs(g * sig) * mu
        assert np.isfinite(a).all()
        elem = (np.abs(a - a64) / np.maximum(bound, 1e-300)).max()
        print(f"[range silu {scheme} m={m} x{f:.1e}] element-wise {elem:.3e}", flush=True)
        assert elem <= TOL


@pytest.mark.parametrize("scheme", ["int8", "int4"])
@pytest.mark.parametrize("m", [1, 32])
def test_argmax_activation_range(gpu, scheme, m):
    """Greedy tokens at x scaled by 2^-100 and 2^100 equal the float64 argmax
    (and the unscaled input's tokens: the scaling is exact)."""
    n, k = 6000, 512
    w = gaussian((n, k), seed=31)
    qw = _quantize(w, scheme, gpu)
    w_hat = _w_hat(w, scheme)
    x = gaussian((m, k), seed=32, std=1.0)
    ref = (x.astype(np.float64) @ w_hat.T).argmax(axis=1)
    for f in (1.0, 2.0 ** -100, 2.0 ** 100):
        xs = (x.astype(np.float64) * f).astype(np.float32)
        tok = quantized_linear_argmax(torch.from_numpy(xs).to(gpu), qw).cpu().numpy()
        assert np.array_equal(tok, ref), (f, np.nonzero(tok != ref))


@pytest.mark.parametrize("m,n,k,scheme", [(1, 512, 1024, "int4"), (1, 512, 1024, "int8"),
                                          (8, 512, 1024, "int4"), (40, 512, 1024, "int8")])
def test_non_finite_activations(gpu, m, n, k, scheme):
    """Rows holding +-inf or NaN: the reference's fp32 products give +-inf, or
    NaN for inf * 0 and opposite infinities, in a pattern float64 reproduces;
    a finite row in the same batch stays exact."""
    w = gaussian((n, k), seed=41)
    qw = _quantize(w, scheme, gpu)
    w_hat = _w_hat(w, scheme)
    x = gaussian((m, k), seed=42, std=1.0)
    x[0, 3] = np.inf
    if m > 2:
        x[1, 7] = np.nan
        x[2, 5], x[2, 9] = np.inf, -np.inf
    y = quantized_linear(torch.from_numpy(x).to(gpu), qw).cpu().numpy().astype(np.float64)
    with np.errstate(invalid="ignore"):
        y64 = x.astype(np.float64) @ w_hat.T
    for r in range(min(m, 3)):
        assert np.array_equal(np.isnan(y[r]), np.isnan(y64[r])), r
        fin = ~np.isnan(y64[r])
        assert np.array_equal(y[r][fin], y64[r][fin]), r          # +-inf, same signs
    if m > 3:
        _check(y[3:], x[3:], w_hat, f"{scheme} m={m} finite rows beside non-finite ones")
