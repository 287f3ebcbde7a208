"""Quantized weights from disk straight into HBM (the load path of the
on-disk format): GPU memory holds only payload + scales -- the reference's
"INT4 loads with at least 50 MiB less than FP16" (Kshipra
tests/test_quantization.py:286-362, host RSS there) restated for device
memory -- and a decoder rebuilt from its saved quantized weights generates
the same tokens."""

from __future__ import annotations

import torch
import pytest

from cases import QWEN05B, decoder_weights
from kshipra_amd.checkpoint import (load_quantized, load_quantized_weights, save_quantized,
                                    save_quantized_weights)
from kshipra_amd.model import DecoderConfig, DecoderLM
from kshipra_amd.quantization import quantize_int4_per_group, quantized_linear

pytestmark = pytest.mark.gpu


def _load_delta(gpu, fn):
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(gpu)
    torch.cuda.reset_peak_memory_stats(gpu)
    obj = fn()
    torch.cuda.synchronize()
    return obj, torch.cuda.memory_allocated(gpu) - base, torch.cuda.max_memory_allocated(gpu) - base


def test_int4_loads_into_hbm_without_materialising(gpu, tmp_path):
    torch.manual_seed(0)
    w16 = torch.randn(8192, 8192, dtype=torch.float16)
    torch.save(w16, str(tmp_path / "w_fp16.pt"))
    qw = quantize_int4_per_group(w16.to(gpu), 128)
    save_quantized(qw, str(tmp_path / "w_int4.pt"))
    x = torch.randn(4, 8192, device=gpu)
    y_before = quantized_linear(x, qw)
    del qw
    torch.cuda.empty_cache()

    q2, d4, peak4 = _load_delta(gpu, lambda: load_quantized(str(tmp_path / "w_int4.pt"), gpu))
    slack = 2 * 1024 * 1024                               # allocator rounding
    assert d4 <= q2.storage_bytes() + slack and peak4 <= q2.storage_bytes() + slack
    w2, d16, _ = _load_delta(gpu, lambda: torch.load(str(tmp_path / "w_fp16.pt"), map_location=gpu,
                                                      weights_only=True))
    assert d16 - d4 > 50 * 1024 * 1024
    assert torch.equal(quantized_linear(x, q2), y_before)   # same bytes, same kernel, same result
    del w2


@pytest.mark.parametrize("scheme", ["int4", "int8"])
def test_decoder_from_saved_quantized_weights(gpu, tmp_path, scheme):
    cfg = dict(QWEN05B, num_layers=4, vocab_size=32000)
    w = {k: torch.from_numpy(v) for k, v in decoder_weights(cfg, seed=5).items()}
    lm = DecoderLM(DecoderConfig(**cfg), w, scheme, gpu, max_seq=32)
    toks, _ = lm.generate([3, 14, 15, 92], 6)
    qws = lm.quantized_weights()
    plain = {k: v for k, v in w.items() if not any(k == f"{n}.weight" for n in qws)}
    path = str(tmp_path / "model.safetensors")
    save_quantized_weights(qws, path, plain)
    stored = sum(q.storage_bytes() for q in qws.values())
    del lm
    loaded, extra = load_quantized_weights(path, gpu)
    assert sum(q.storage_bytes() for q in loaded.values()) == stored
    lm2 = DecoderLM(DecoderConfig(**cfg), extra, scheme, gpu, max_seq=32, quantized=loaded, fuse=True)
    toks2, _ = lm2.generate([3, 14, 15, 92], 6)
    assert toks2 == toks


@pytest.mark.parametrize("scheme,n,k", [("int8", 1024, 896), ("int4", 1024, 896), ("int4", 640, 1000)])
@pytest.mark.parametrize("m", [1, 8, 40])
def test_oracle_bytes_from_disk_match_float64(gpu, tmp_path, scheme, n, k, m):
    """The oracle's quantized bytes saved as the reference's bare
    ``{"payload", "scales"}`` dict (tests/test_quantization.py:312), loaded
    straight into HBM and multiplied by the HIP kernel: the output equals the
    float64 product of the oracle's exact dequantized weight within the
    linear path's bars (1e-4 norm-wise and element-wise)."""
    import numpy as np
    from cases import gaussian
    from oracle import quant

    w = gaussian((n, k), seed=n + k + m)
    b = gaussian((n,), seed=n + 1)
    if scheme == "int8":
        p, s = quant.c_quantize_int8(w)
        w_hat = quant.c_dequantize_int8(p, s)
    else:
        p, s, _ = quant.c_quantize_int4(w, 128)
        w_hat = quant.c_dequantize_int4(p, s, k, 128)
    path = str(tmp_path / "w.pt")
    torch.save({"payload": torch.from_numpy(p), "scales": torch.from_numpy(s)}, path)
    qw = load_quantized(path, gpu, in_features=k)
    assert qw.payload.device == gpu and qw.scales.device == gpu
    assert np.array_equal(qw.payload.cpu().numpy(), p)
    x = gaussian((m, k), seed=m, std=1.0)
    y = quantized_linear(torch.from_numpy(x).to(gpu), qw, torch.from_numpy(b).to(gpu))
    y = y.cpu().numpy().astype(np.float64)
    y64 = quant.linear_f64(x, w_hat, b)
    mag = np.abs(x.astype(np.float64)) @ np.abs(w_hat.astype(np.float64)).T + np.abs(b)
    err = np.abs(y - y64)
    norm, elem = err.max() / np.abs(y64).max(), (err / mag).max()
    print(f"[disk {scheme} m={m} n={n} k={k}] norm-wise {norm:.3e} element-wise {elem:.3e}", flush=True)
    assert norm <= 1e-4 and elem <= 1e-4
