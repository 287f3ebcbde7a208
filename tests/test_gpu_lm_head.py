"""Vocab projection (lm_head) on the Llama-3-8B shape [128256 x 4096] with
greedy argmax (engine/model.py:187,200: ``int(logits[0, -1].argmax())``,
first index on ties).

W ~ N(0, 0.02) (seeded torch CPU generator), quantized INT8 per-channel and
INT4 G=128 on the GPU; h ~ N(0, 1) at M = 1 and M = 32.  Checks:

* the GPU payload and scales are bit-identical to the oracle's quantization of
  the same fp32 bytes;
* logits are within the linear-path bars (norm-wise and element-wise 1e-4)
  of the float64 value of the reference forward (exact dequantized weight);
* the greedy token of every row equals the argmax of the float64 logits and of
  the reference's own fp32 order (materialise w_hat, then an fp32 matmul),
  both via torch.argmax over the logits and via the argmax fused into the
  projection (quantized_linear_argmax).
  The smallest float64 top-2 gap over the rows is printed next to the largest
  logit error, so a run shows by how much the comparison clears a near-tie.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kshipra_amd.quantization import (quantize_int4_per_group, quantize_int8_per_channel,
                                      quantized_linear, quantized_linear_argmax)
from oracle import quant

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN = 128256, 4096
ROWS_PER_CHUNK = 16384


@pytest.fixture(scope="module")
def lm_head_weight():
    g = torch.Generator().manual_seed(55)
    w = torch.randn(VOCAB, HIDDEN, generator=g) * 0.02
    h = torch.randn(32, HIDDEN, generator=torch.Generator().manual_seed(56))
    return w.numpy(), h.numpy()


def _reference_logits(payload, scales, scheme, h):
    """float64 logits, the reference's fp32 logits, and the float64 |h| @ |w_hat|^T bound."""
    m = h.shape[0]
    y64 = np.empty((m, VOCAB), np.float64)
    y32 = np.empty((m, VOCAB), np.float32)
    mag = np.empty((m, VOCAB), np.float64)
    h64 = h.astype(np.float64)
    for r0 in range(0, VOCAB, ROWS_PER_CHUNK):
        r1 = min(VOCAB, r0 + ROWS_PER_CHUNK)
        if scheme == "int8":
            w_hat = quant.c_dequantize_int8(payload[r0:r1], scales[r0:r1])
        else:
            w_hat = quant.c_dequantize_int4(payload[r0:r1], scales[r0:r1], HIDDEN, 128)
        y32[:, r0:r1] = quant.linear_f32(h, w_hat)
        w64 = w_hat.astype(np.float64)
        y64[:, r0:r1] = h64 @ w64.T
        mag[:, r0:r1] = np.abs(h64) @ np.abs(w64).T
    return y64, y32, mag


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_lm_head_greedy_argmax(gpu, lm_head_weight, scheme):
    w, h = lm_head_weight
    wt = torch.from_numpy(w).to(gpu)
    qw = quantize_int8_per_channel(wt) if scheme == "int8" else quantize_int4_per_group(wt, 128)
    del wt
    payload = qw.payload.cpu().numpy()
    scales = qw.scales.cpu().numpy()          # float16

    # Bit-exact packing against the oracle on the same fp32 bytes.
    if scheme == "int8":
        p_ref, s_ref = quant.c_quantize_int8(w)
    else:
        p_ref, s_ref, _ = quant.c_quantize_int4(w, 128)
    assert np.array_equal(payload.view(np.uint8), p_ref.view(np.uint8))
    assert np.array_equal(scales.view(np.uint16), s_ref.view(np.uint16))

    y64, y32, mag = _reference_logits(payload, scales, scheme, h)
    for m in (1, 32):
        hx = torch.from_numpy(h[:m]).to(gpu)
        logits = quantized_linear(hx, qw)
        tok = logits.argmax(dim=-1).cpu().numpy()
        yn = logits.cpu().numpy().astype(np.float64)
        err = np.abs(yn - y64[:m])
        norm_err = err.max() / np.abs(y64[:m]).max()
        elem_err = (err / mag[:m]).max()
        ref64_tok = y64[:m].argmax(axis=-1)
        ref32_tok = y32[:m].argmax(axis=-1)
        top2 = np.sort(y64[:m], axis=-1)[:, -2:]
        gap = top2[:, 1] - top2[:, 0]
        print(f"[lm_head {scheme} m={m}] norm-wise {norm_err:.3e} element-wise {elem_err:.3e} "
              f"max |logit error| {err.max():.3e} min top-2 gap {gap.min():.3e}", flush=True)
        assert norm_err <= 1e-4 and elem_err <= 1e-4
        assert np.array_equal(tok, ref64_tok), (tok, ref64_tok)
        assert np.array_equal(tok, ref32_tok), (tok, ref32_tok)
        # the same tokens from the argmax fused into the projection
        fused = quantized_linear_argmax(hx, qw).cpu().numpy()
        assert np.array_equal(fused, ref64_tok), (fused, ref64_tok)
