"""GPU parity of the SiLU-gated gate / up projection (the MLP input
``silu(gate_proj(x)) * up_proj(x)`` of the layer engine/model.py:147 runs,
with gate_proj / up_proj quantized as at engine/model.py:80-91).

Reference: float64 ``silu(g) * u`` with g, u the float64 products of x and
the oracle's exact dequantized weights (plus bias).  Bars:

* norm-wise:    max|a - a64| / max|a64| <= 1e-4;
* element-wise: |a - a64| <= 1e-4 * (|silu'(g)| |u| mg + |silu(g)| mu) + 1e-30,
  with mg = |x| @ |w_g|^T + |b_g| (mu likewise): the linear path's bar
  carried through the product, so outputs near zero are still checked.

Covers the skinny path (M <= 8 hi / lo rows, M = 9..16 split rows), the GEMM
path plus the pairing kernel (M > 16), the generic path (G = 32), bias / no
bias, unaligned activations, and the module against two projections + torch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from cases import gaussian
from kshipra_amd.quantization import (FusedGateUpSiLU, QuantizedLinear, interleave_gate_up,
                                      quantize_int4_per_group, quantize_int8_per_channel,
                                      quantized_gate_up_silu)
from oracle import quant

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _what(w: np.ndarray, scheme: str, g: int) -> np.ndarray:
    if scheme == "int8":
        return quant.c_dequantize_int8(*quant.c_quantize_int8(w)).astype(np.float64)
    p, s, _ = quant.c_quantize_int4(w, g)
    return quant.c_dequantize_int4(p, s, w.shape[1], g).astype(np.float64)


def _reference(x, wg, wu, bg, bu, scheme, g):
    x64 = x.astype(np.float64)
    hg, hu = _what(wg, scheme, g), _what(wu, scheme, g)
    gv, uv = x64 @ hg.T, x64 @ hu.T
    mg, mu = np.abs(x64) @ np.abs(hg).T, np.abs(x64) @ np.abs(hu).T
    if bg is not None:
        gv, uv = gv + bg, uv + bu
        mg, mu = mg + np.abs(bg), mu + np.abs(bu)
    sig = 1.0 / (1.0 + np.exp(-gv))
    silu = gv * sig
    dsilu = sig * (1.0 + gv * (1.0 - sig))
    return silu * uv, np.abs(dsilu) * np.abs(uv) * mg + np.abs(silu) * mu


def _quantize(w: torch.Tensor, scheme: str, g: int):
    return quantize_int8_per_channel(w) if scheme == "int8" else quantize_int4_per_group(w, g)


@pytest.mark.parametrize("m,nh,k,scheme,g", [
    (1, 14336, 4096, "int4", 128),   # Llama-3-8B gate / up at M = 1
    (1, 14336, 4096, "int8", 128),
    (3, 1024, 896, "int4", 128),     # hi / lo rows, K = 7 groups
    (8, 512, 1024, "int8", 128),
    (13, 256, 1024, "int4", 128),    # split rows (M = 9..16)
    (24, 320, 640, "int8", 128),     # GEMM path + pairing kernel
    (100, 512, 1024, "int4", 128),
    (4, 96, 512, "int4", 32),        # generic path + pairing kernel
])
def test_gate_up_silu_matches_reference(gpu, m, nh, k, scheme, g):
    wg, wu = gaussian((nh, k), seed=nh + k), gaussian((nh, k), seed=nh + k + 1)
    bg, bu = gaussian((nh,), seed=nh + 2), gaussian((nh,), seed=nh + 3)
    qg = _quantize(torch.from_numpy(wg).to(gpu), scheme, g)
    qu = _quantize(torch.from_numpy(wu).to(gpu), scheme, g)
    qw = interleave_gate_up(qg, qu)
    xs = gaussian((m, k + 1), seed=m + k, std=1.0)
    xg = torch.from_numpy(xs).to(gpu)
    bias = torch.stack([torch.from_numpy(bg).reshape(-1, 16), torch.from_numpy(bu).reshape(-1, 16)],
                       dim=1).reshape(-1).to(gpu)
    for name, x, b in (("aligned+bias", xg[:, :k].contiguous(), bias), ("unaligned", xg[:, 1:], None)):
        a = quantized_gate_up_silu(x, qw, b)
        torch.cuda.synchronize()
        a64, mag = _reference(x.cpu().numpy(), wg, wu, bg if b is not None else None,
                              bu if b is not None else None, scheme, g)
        err = np.abs(a.cpu().numpy().astype(np.float64) - a64)
        norm = err.max() / max(np.abs(a64).max(), 1e-30)
        elem = (err / (mag + 1e-30)).max()
        print(f"[gate/up silu {scheme} m={m} nh={nh} k={k} g={g} {name}] "
              f"norm-wise {norm:.3e} element-wise {elem:.3e}", flush=True)
        assert norm <= TOL and elem <= TOL, (name, norm, elem)


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_fused_module_matches_two_projections(gpu, scheme):
    """FusedGateUpSiLU against QuantizedLinear gate / up + F.silu(g) * u
    (the reference's MLP body) on one MLP's shapes, 3-D input."""
    torch.manual_seed(11)
    gate = nn.Linear(896, 4864, bias=False, device=gpu)
    up = nn.Linear(896, 4864, bias=False, device=gpu)
    qg, qu = QuantizedLinear(gate, scheme), QuantizedLinear(up, scheme)
    fused = FusedGateUpSiLU(qg, qu)
    x = torch.randn(2, 3, 896, device=gpu)
    with torch.no_grad():
        ref = F.silu(qg(x)) * qu(x)
        out = fused(x)
    assert out.shape == (2, 3, 4864)
    scale = ref.abs().max().item()
    assert (out - ref).abs().max().item() <= 1e-5 * scale
    assert "storage_bytes" in repr(fused)
