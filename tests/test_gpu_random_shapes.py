"""GPU parity over seeded random shapes: the dequant-matmul (and its fused
SiLU-gated and greedy-argmax forms) vs the float64 oracle.

Every case draws a scheme (INT8 per-channel / INT4 G=128), a batch M that
lands on each kernel family (single-row, skinny hi/lo and split, tiled GEMM,
warp-specialised GEMM), N from 1 to 2600 (any residue mod 16), K from the
Llama-3 / Qwen2.5 sizes or arbitrary (INT4 padded groups, INT8 windows that
do not divide K: the generic kernel), an activation scale from 2^-40 to 2^40
and bias on or off.  Bars as in test_gpu_linear.py: norm-wise and
condition-aware element-wise error <= 1e-4 against x @ (q * s)^T + b in
float64 over the oracle's exact dequantized weight
(engine/quantization.py:394-396 evaluated without rounding).  The SiLU-gated
pairs use test_gpu_gate_up_silu.py's bar (the linear bar carried through
silu(g) * u); the fused argmax must return the same tokens with and without
its logits, the first index of the maximum of those logits, logits within
the linear bar of the float64 product, and a chosen logit within the linear
bar of the float64 maximum.  (Its logits equal quantized_linear's bit for
bit except where quantized_linear splits K across workgroups -- M >= 3 with
K >= 8192 -- and adds the slices in another order.)
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import gaussian
from kshipra_amd.quantization import (interleave_gate_up, quantize_int4_per_group,
                                      quantize_int8_per_channel, quantized_gate_up_silu,
                                      quantized_linear, quantized_linear_argmax)
from oracle import quant

pytestmark = pytest.mark.gpu

TOL = 1e-4
N_CASES = 200


def _case(i: int):
    rng = np.random.default_rng(7919 * i + 13)
    scheme = "int4" if i % 2 else "int8"
    m = int(rng.choice([1, 1, 1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 24, 31, 32, 33, 40, 64, 65, 80]))
    n = int(rng.integers(1, 2600))
    k = int(rng.choice([64, 128, 256, 384, 512, 896, 1024, 1536, 2048, 3072, 4096, 4864, 8192, 14336]))
    if rng.random() < 0.25:
        k = int(rng.integers(8, 5000))
    scale = float(rng.choice([1.0, 1.0, 1e-6, 1e5, 2.0 ** 40, 2.0 ** -40]))
    bias = bool(rng.random() < 0.5)
    return scheme, m, n, k, scale, bias


@pytest.mark.parametrize("block", range(4))
def test_random_shapes(gpu, block):
    worst = 0.0
    for i in range(block * N_CASES // 4, (block + 1) * N_CASES // 4):
        scheme, m, n, k, scale, bias = _case(i)
        label = f"case {i}: {scheme} m={m} n={n} k={k} scale={scale:g} bias={bias}"
        w = gaussian((n, k), seed=i)
        x = (gaussian((m, k), seed=10_000 + i, std=1.0) * scale).astype(np.float32)
        b = gaussian((n,), seed=20_000 + i) if bias else None
        wd = torch.from_numpy(w).to(gpu)
        if scheme == "int8":
            qw = quantize_int8_per_channel(wd)
            w_hat = quant.c_dequantize_int8(*quant.c_quantize_int8(w))
        else:
            qw = quantize_int4_per_group(wd, 128)
            p, s, _ = quant.c_quantize_int4(w, 128)
            w_hat = quant.c_dequantize_int4(p, s, k, 128)
        y = quantized_linear(torch.from_numpy(x).to(gpu), qw, torch.from_numpy(b).to(gpu) if bias else None)
        yn = y.cpu().numpy().astype(np.float64)
        y64 = quant.linear_f64(x, w_hat, b)
        mag = np.abs(x.astype(np.float64)) @ np.abs(w_hat.astype(np.float64)).T
        if bias:
            mag = mag + np.abs(b.astype(np.float64))
        err = np.abs(yn - y64)
        norm_err = err.max() / max(np.abs(y64).max(), 1e-300)
        elem_err = (err / np.maximum(mag, 1e-300)).max()
        assert np.isfinite(yn).all(), label
        assert norm_err <= TOL and elem_err <= TOL, (label, norm_err, elem_err)
        worst = max(worst, norm_err, elem_err)
    print(f"[random shapes block {block}] worst {worst:.3e}", flush=True)


def _dequantized(w: np.ndarray, scheme: str) -> np.ndarray:
    if scheme == "int8":
        return quant.c_dequantize_int8(*quant.c_quantize_int8(w)).astype(np.float64)
    p, s, _ = quant.c_quantize_int4(w, 128)
    return quant.c_dequantize_int4(p, s, w.shape[1], 128).astype(np.float64)


def _quantized(w: np.ndarray, scheme: str, gpu):
    wd = torch.from_numpy(w).to(gpu)
    return quantize_int8_per_channel(wd) if scheme == "int8" else quantize_int4_per_group(wd, 128)


@pytest.mark.parametrize("block", range(2))
def test_random_gate_up_silu(gpu, block):
    worst = 0.0
    for i in range(block * 40, (block + 1) * 40):
        scheme, m, _, k, scale, bias = _case(1000 + i)
        nh = 16 * int(np.random.default_rng(i).integers(1, 180))
        label = f"case {i}: {scheme} m={m} nh={nh} k={k} scale={scale:g} bias={bias}"
        wg, wu = gaussian((nh, k), seed=30_000 + i), gaussian((nh, k), seed=40_000 + i)
        bg, bu = gaussian((nh,), seed=50_000 + i), gaussian((nh,), seed=60_000 + i)
        qw = interleave_gate_up(_quantized(wg, scheme, gpu), _quantized(wu, scheme, gpu))
        x = (gaussian((m, k), seed=70_000 + i, std=1.0) * scale).astype(np.float32)
        b = None
        if bias:
            b = torch.stack([torch.from_numpy(bg).reshape(-1, 16), torch.from_numpy(bu).reshape(-1, 16)],
                            dim=1).reshape(-1).to(gpu)
        a = quantized_gate_up_silu(torch.from_numpy(x).to(gpu), qw, b).cpu().numpy().astype(np.float64)
        x64 = x.astype(np.float64)
        hg, hu = _dequantized(wg, scheme), _dequantized(wu, scheme)
        gv, uv = x64 @ hg.T, x64 @ hu.T
        mg, mu = np.abs(x64) @ np.abs(hg).T, np.abs(x64) @ np.abs(hu).T
        if bias:
            gv, uv, mg, mu = gv + bg, uv + bu, mg + np.abs(bg), mu + np.abs(bu)
        with np.errstate(over="ignore"):
            sig = 1.0 / (1.0 + np.exp(-gv))
        silu = gv * sig
        dsilu = sig * (1.0 + gv * (1.0 - sig))
        a64 = silu * uv
        mag = np.abs(dsilu) * np.abs(uv) * mg + np.abs(silu) * mu
        err = np.abs(a - a64)
        norm_err = err.max() / max(np.abs(a64).max(), 1e-300)
        elem_err = (err / (mag + 1e-300)).max()
        assert np.isfinite(a).all(), label
        assert norm_err <= TOL and elem_err <= TOL, (label, norm_err, elem_err)
        worst = max(worst, norm_err, elem_err)
    print(f"[random gate/up silu block {block}] worst {worst:.3e}", flush=True)


@pytest.mark.parametrize("block", range(2))
def test_random_argmax(gpu, block):
    for i in range(block * 40, (block + 1) * 40):
        scheme, m, n, k, scale, bias = _case(2000 + i)
        n = 2 * n + 1
        label = f"case {i}: {scheme} m={m} n={n} k={k} scale={scale:g} bias={bias}"
        w = gaussian((n, k), seed=80_000 + i)
        x = (gaussian((m, k), seed=90_000 + i, std=1.0) * scale).astype(np.float32)
        b = gaussian((n,), seed=95_000 + i) if bias else None
        qw = _quantized(w, scheme, gpu)
        xd = torch.from_numpy(x).to(gpu)
        bd = torch.from_numpy(b).to(gpu) if bias else None
        tok, logits = quantized_linear_argmax(xd, qw, bd, return_logits=True)
        tok_only = quantized_linear_argmax(xd, qw, bd)
        assert torch.equal(tok, tok_only), label
        assert torch.equal(tok, logits.argmax(dim=-1)), label
        w_hat = _dequantized(w, scheme)
        y64 = quant.linear_f64(x, w_hat, b)
        mag = np.abs(x.astype(np.float64)) @ np.abs(w_hat).T
        if bias:
            mag = mag + np.abs(b.astype(np.float64))
        err = np.abs(logits.cpu().numpy().astype(np.float64) - y64)
        assert (err <= TOL * np.maximum(mag, 1e-300)).all(), (label, (err / np.maximum(mag, 1e-300)).max())
        t = tok.cpu().numpy()
        rows = np.arange(m)
        gap = y64.max(axis=1) - y64[rows, t]
        assert (gap <= 2 * TOL * mag.max(axis=1)).all(), (label, gap.max())
