"""On-disk quantized format (host side): the reference's {"payload", "scales"}
dict (Kshipra tests/test_quantization.py:312) plus metadata, and the
safetensors model file; round trips are bit-exact and the INT4 file of an
8192 x 8192 fp16 weight is > 50 MiB smaller than the fp16 file
(tests/test_quantization.py:319-324)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from cases import gaussian
from kshipra_amd.checkpoint import (load_quantized, load_quantized_weights, save_quantized,
                                    save_quantized_weights)
from kshipra_amd.quantization import QuantizationError, QuantizedWeight
from oracle import quant


def _oracle_qw(w: np.ndarray, scheme: str) -> QuantizedWeight:
    if scheme == "int8":
        p, s = quant.c_quantize_int8(w)
        return QuantizedWeight(torch.from_numpy(p), torch.from_numpy(s), "int8_per_channel", w.shape)
    p, s, kp = quant.c_quantize_int4(w, 128)
    return QuantizedWeight(torch.from_numpy(p), torch.from_numpy(s), "int4_per_group", w.shape, 128, kp)


def _same(a: QuantizedWeight, b: QuantizedWeight) -> None:
    assert a.scheme == b.scheme and tuple(a.original_shape) == tuple(b.original_shape)
    assert a.group_size == b.group_size and a.in_features_padded == b.in_features_padded
    assert a.payload.dtype == b.payload.dtype and torch.equal(a.payload.cpu(), b.payload.cpu())
    assert torch.equal(a.scales.cpu().view(torch.int16), b.scales.cpu().view(torch.int16))


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_reference_dict_round_trip(tmp_path, scheme):
    qw = _oracle_qw(gaussian((48, 300), seed=1), scheme)
    path = str(tmp_path / "w.pt")
    save_quantized(qw, path)
    d = torch.load(path, weights_only=True)
    assert {"payload", "scales"} <= set(d)             # the reference's own keys
    _same(load_quantized(path), qw)


def test_int4_file_is_smaller_than_fp16(tmp_path):
    torch.manual_seed(0)
    w16 = torch.randn(8192, 8192, dtype=torch.float16)
    torch.save(w16, str(tmp_path / "w_fp16.pt"))
    qw = _oracle_qw(w16.float().numpy(), "int4")
    save_quantized(qw, str(tmp_path / "w_int4.pt"))
    fp16_size = os.path.getsize(tmp_path / "w_fp16.pt")
    int4_size = os.path.getsize(tmp_path / "w_int4.pt")
    assert fp16_size > int4_size + 50 * 1024 * 1024
    assert int4_size < qw.storage_bytes() + 64 * 1024      # payload + scales + a small header


def test_safetensors_model_file(tmp_path):
    ws = {"layers.0.q_proj": _oracle_qw(gaussian((64, 128), seed=2), "int4"),
          "layers.0.k_proj": _oracle_qw(gaussian((16, 128), seed=3), "int8")}
    extra = {"norm.weight": torch.ones(128), "layers.0.q_proj.bias": torch.arange(64.0)}
    path = str(tmp_path / "model.safetensors")
    save_quantized_weights(ws, path, extra)
    got, got_extra = load_quantized_weights(path)
    assert set(got) == set(ws) and set(got_extra) == set(extra)
    for k in ws:
        _same(got[k], ws[k])
    for k in extra:
        assert torch.equal(got_extra[k], extra[k])


def test_loader_validates(tmp_path):
    qw = _oracle_qw(gaussian((8, 256), seed=4), "int4")
    d = {"payload": qw.payload, "scales": qw.scales[:, :1].contiguous(), "scheme": qw.scheme,
         "original_shape": [8, 256], "group_size": 128, "in_features_padded": 256}
    torch.save(d, str(tmp_path / "bad.pt"))
    with pytest.raises(QuantizationError):                # scales shape disagrees with the payload
        load_quantized(str(tmp_path / "bad.pt"))
    d.pop("scheme")
    torch.save(d, str(tmp_path / "partial.pt"))
    with pytest.raises(QuantizationError, match="lacks"):  # metadata present but incomplete
        load_quantized(str(tmp_path / "partial.pt"))


@pytest.mark.parametrize("scheme,k", [("int8", 300), ("int4", 256), ("int4", 300)])
def test_reference_bare_dict(tmp_path, scheme, k):
    """The reference's own file (tests/test_quantization.py:312 saves
    ``{"payload", "scales"}`` and nothing else): scheme, shape and group size
    are inferred; a padded INT4 K comes from the caller."""
    qw = _oracle_qw(gaussian((24, k), seed=k), scheme)
    path = str(tmp_path / "bare.pt")
    torch.save({"payload": qw.payload, "scales": qw.scales}, path)
    padded = scheme == "int4" and k % 128 != 0
    _same(load_quantized(path, in_features=k if padded else None), qw)
    if padded:
        got = load_quantized(path)                           # K read as the padded width
        assert got.original_shape == (24, qw.in_features_padded)
        assert torch.equal(got.payload, qw.payload)
        with pytest.raises(QuantizationError):
            load_quantized(path, in_features=k - 128)        # outside the last group
    if scheme == "int4":
        with pytest.raises(QuantizationError):
            load_quantized(path, in_features=k if padded else None, group_size=64)
    else:
        with pytest.raises(QuantizationError):
            load_quantized(path, in_features=k + 1)
    torch.save({"payload": qw.payload.to(torch.int16), "scales": qw.scales}, path)
    with pytest.raises(QuantizationError):
        load_quantized(path)
