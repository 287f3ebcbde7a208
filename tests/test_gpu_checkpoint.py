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
