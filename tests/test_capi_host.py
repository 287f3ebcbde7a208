"""CPU-only checks of the C-ABI library and the host-side logic.

No GPU is touched: the library is loaded, every symbol the header declares is
resolved, and only entry points whose argument validation fails on the host
(before any HIP call) are invoked.
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch
import torch.nn as nn

from kshipra_amd import _lib
from kshipra_amd.quantization import (QuantizationError, QuantizedLinear, QuantizedWeight,
                                      _validate_weight, quantize_int4_per_group,
                                      quantize_int8_per_channel)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kshipra_quant.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(kq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    syms = header_symbols()
    assert len(syms) >= 10
    for name in syms:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
    assert sorted(n for n, _, _ in _lib.SIGNATURES) == syms


def test_version():
    assert _lib.load().kq_version() == _lib.ABI_VERSION


def test_workspace_query_is_host_only():
    lib = _lib.load()
    # M = 1 INT4 / INT8 on Llama-3-8B shapes: activations fit in LDS, no workspace
    assert lib.kq_linear_workspace_bytes(4, 1, 14336, 4096, 128) == 0
    assert lib.kq_linear_workspace_bytes(8, 1, 4096, 14336, 0) == 0
    # M = 8, K = 4096: 132 KiB of staged activations per workgroup; 256
    # workgroups (one per CU) stage in LDS, 448 (a second round) in the
    # workspace, 4 bytes per activation, then one scale exponent per row
    assert lib.kq_linear_workspace_bytes(8, 8, 4096, 4096, 0) == 0
    assert lib.kq_linear_workspace_bytes(8, 8, 28672, 4096, 0) == 4 * 8 * 4096 + 4 * 8
    # K = 14336, M >= 3: K split into slices staged in LDS; the workspace
    # holds one fp32 partial output per slice (8 slices at M = 8, 4 at M = 4 and 3)
    assert lib.kq_linear_workspace_bytes(4, 8, 4096, 14336, 128) == 8 * 4 * 8 * 4096
    assert lib.kq_linear_workspace_bytes(8, 4, 4096, 14336, 0) == 4 * 4 * 4 * 4096
    assert lib.kq_linear_workspace_bytes(8, 3, 4096, 14336, 0) == 4 * 4 * 3 * 4096
    # ... below M = 3, whole-K workgroups stage x in LDS: no workspace
    assert lib.kq_linear_workspace_bytes(4, 2, 4096, 14336, 128) == 0
    # GEMM path: operand planes for M rounded up to the 64-row tile, then one
    # scale exponent per padded row
    assert lib.kq_linear_workspace_bytes(4, 512, 14336, 4096, 128) == 4 * 512 * 4096 + 4 * 512
    assert lib.kq_linear_workspace_bytes(4, 100, 64, 256, 128) == 4 * 128 * 256 + 4 * 128
    # generic path (G != 128) needs none
    assert lib.kq_linear_workspace_bytes(4, 64, 512, 512, 32) == 0
    assert lib.kq_linear_workspace_bytes(4, 0, 10, 10, 128) == 0


@pytest.mark.parametrize("call", [
    lambda L: L.kq_quantize_int4(None, 0, 4, 128, 128, 3, None, None, None, None),
    lambda L: L.kq_quantize_int4(1, 0, 4, 128, 128, 0, 1, 1, 1, None),
    lambda L: L.kq_quantize_int4(1, 0, 4, 128, 128, 127, 1, 1, 1, None),
    lambda L: L.kq_quantize_int8(1, 7, 4, 128, 128, 1, 1, 1, None),
    lambda L: L.kq_quantize_int8(1, 0, 0, 128, 128, 1, 1, 1, None),
    lambda L: L.kq_quantize_int8(1, 0, 4, 128, 64, 1, 1, 1, None),
    lambda L: L.kq_dequantize_int4(1, 1, 4, 100, 128, 256, 1, 0, None),
    lambda L: L.kq_dequantize_int8(1, 1, 4, 100, 1, 9, None),
    lambda L: L.kq_linear_int8(1, 1, 10, 1, 1, None, 1, 20, 20, 100, None, 0, None),
    lambda L: L.kq_linear_int4(1, 1, 128, 1, 1, 128, 100, None, 1, 20, 20, 100, None, 0, None),
    lambda L: L.kq_linear_int4(1, 1, 128, 1, 1, 3, 128, None, 1, 20, 20, 128, None, 0, None),
    lambda L: L.kq_linear_argmax_int8(1, 1, 100, 1, 1, None, None, 0, 20, 100, None, None, 0, None),
    lambda L: L.kq_linear_argmax_int8(1, 70000, 100, 1, 1, None, None, 0, 20, 100, 1, None, 0, None),
    lambda L: L.kq_linear_argmax_int8(1, 1, 100, 1, 1, None, 1, 10, 20, 100, 1, None, 0, None),
    lambda L: L.kq_linear_argmax_int4(1, 1, 128, 1, 1, 5, 130, None, None, 0, 20, 128, 1, None, 0, None),
])
def test_argument_errors_are_reported_before_launch(call):
    lib = _lib.load()
    status = call(lib)
    assert status == _lib.KQ_ERR_ARG
    assert lib.kq_last_error() not in (None, b"")


def test_missing_workspace_is_reported():
    lib = _lib.load()
    # M = 8, N = 28672, K = 4096 needs a workspace; pointers are never dereferenced
    st = lib.kq_linear_int8(1, 8, 4096, 1, 1, None, 1, 28672, 28672, 4096, None, 0, None)
    assert st == _lib.KQ_ERR_WORKSPACE
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.check(st)


def test_argmax_needs_its_workspace():
    lib = _lib.load()
    # partial argmax pairs of the 16-column tiles: 8016 x 8 bytes at M = 1 (256-byte rounded)
    assert lib.kq_linear_argmax_workspace_bytes(4, 1, 128256, 4096, 128) == (8016 * 8 + 255) // 256 * 256
    # GEMM path: linear workspace + partials + a logits buffer
    assert lib.kq_linear_argmax_workspace_bytes(8, 32, 1000, 256, 0) > 32 * 1000 * 4
    st = lib.kq_linear_argmax_int8(1, 1, 4096, 1, 1, None, None, 0, 128256, 4096, 1, None, 0, None)
    assert st == _lib.KQ_ERR_WORKSPACE


def test_status_mapping():
    with pytest.raises(QuantizationError):
        _lib.check(_lib.KQ_ERR_ARG)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.KQ_ERR_HIP)
    _lib.check(_lib.KQ_OK)


# ---------------------------------------------------------------------- #
# Python API: host-side validation (Kshipra tests/test_quantization.py
# :189-245 restated where it needs no GPU)
# ---------------------------------------------------------------------- #


def test_odd_and_zero_group_size_rejected():
    w = torch.randn(4, 128)
    for g in (127, 0, -2):
        with pytest.raises(QuantizationError):
            quantize_int4_per_group(w, group_size=g)


def test_bad_rank_and_empty_rejected():
    for w in (torch.randn(8), torch.randn(2, 3, 4), torch.empty(0, 4), torch.empty(4, 0)):
        with pytest.raises(QuantizationError):
            quantize_int8_per_channel(w)
        with pytest.raises(QuantizationError):
            _validate_weight(w)


def test_bad_scheme_and_module_type_rejected():
    with pytest.raises(QuantizationError):
        QuantizedLinear(nn.Linear(8, 8), scheme="int3")
    with pytest.raises(QuantizationError):
        QuantizedLinear(nn.Conv1d(8, 8, 1), scheme="int8")


def test_cpu_tensors_fail_loudly():
    """There is no CPU fallback: compute on a CPU tensor raises."""
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        quantize_int8_per_channel(torch.randn(4, 8))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        quantize_int4_per_group(torch.randn(4, 8))


def test_quantized_weight_validation():
    """engine/quantization.py:108-152 checks, with host tensors."""
    ok8 = QuantizedWeight(torch.zeros(3, 5, dtype=torch.int8), torch.zeros(3, dtype=torch.float16),
                          "int8_per_channel", (3, 5))
    assert ok8.storage_bytes() == 15 + 6
    ok4 = QuantizedWeight(torch.zeros(3, 64, dtype=torch.uint8), torch.zeros(3, 1, dtype=torch.float16),
                          "int4_per_group", (3, 100), 128, 128)
    assert ok4.storage_bytes() == 3 * 64 + 3 * 2
    bad = [
        dict(payload=torch.zeros(3, 5, dtype=torch.int8), scales=torch.zeros(3, dtype=torch.float16),
             scheme="int2", original_shape=(3, 5)),
        dict(payload=torch.zeros(3, 5, dtype=torch.int8), scales=torch.zeros(4, dtype=torch.float16),
             scheme="int8_per_channel", original_shape=(3, 5)),
        dict(payload=torch.zeros(3, 5, dtype=torch.uint8), scales=torch.zeros(3, dtype=torch.float16),
             scheme="int8_per_channel", original_shape=(3, 5)),
        dict(payload=torch.zeros(3, 5, dtype=torch.int8), scales=torch.zeros(3, 1, dtype=torch.float16),
             scheme="int8_per_channel", original_shape=(3, 5)),
        dict(payload=torch.zeros(3, 4, dtype=torch.int8), scales=torch.zeros(3, dtype=torch.float16),
             scheme="int8_per_channel", original_shape=(3, 5)),
        dict(payload=torch.zeros(3, 64, dtype=torch.int8), scales=torch.zeros(3, 1, dtype=torch.float16),
             scheme="int4_per_group", original_shape=(3, 100), group_size=128, in_features_padded=128),
        dict(payload=torch.zeros(3, 64, dtype=torch.uint8), scales=torch.zeros(3, 1, dtype=torch.float16),
             scheme="int4_per_group", original_shape=(3, 100)),
        dict(payload=torch.zeros(3, 64, dtype=torch.uint8), scales=torch.zeros(3, 2, dtype=torch.float16),
             scheme="int4_per_group", original_shape=(3, 100), group_size=128, in_features_padded=128),
        dict(payload=torch.zeros(3, 63, dtype=torch.uint8), scales=torch.zeros(3, 1, dtype=torch.float16),
             scheme="int4_per_group", original_shape=(3, 100), group_size=128, in_features_padded=128),
    ]
    for kw in bad:
        with pytest.raises(QuantizationError):
            QuantizedWeight(**kw)


def test_header_cites_reference_for_every_compute_entry_point():
    text = open(HEADER).read()
    for name in ("kq_quantize_int8", "kq_quantize_int4", "kq_dequantize_int8", "kq_dequantize_int4",
                 "kq_linear_int8", "kq_linear_int4", "kq_check_finite"):
        block = text[:text.index(name + "(")].rsplit("/*", 1)[-1]
        assert "engine/quantization.py" in block, name
    for name in ("kq_linear_argmax_int8", "kq_linear_argmax_int4",
                 "kq_linear_silu_mul_int8", "kq_linear_silu_mul_int4"):
        block = text[:text.index(name + "(")].rsplit("/*", 1)[-1]
        assert "engine/model.py" in block, name


def _oracle_qw(w, scheme):
    import numpy as np
    from oracle import quant
    if scheme == "int8":
        p, s = quant.c_quantize_int8(w)
        return QuantizedWeight(torch.from_numpy(p), torch.from_numpy(s), "int8_per_channel", w.shape)
    p, s, kp = quant.c_quantize_int4(w, 128)
    return QuantizedWeight(torch.from_numpy(np.ascontiguousarray(p)), torch.from_numpy(s),
                           "int4_per_group", w.shape, 128, kp)


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_row_stacking_equals_quantizing_the_stacked_weight(scheme):
    """concat_quantized (the fused q/k/v and gate/up weight) is bit-identical to
    quantizing the row-stacked fp32 weight, padding columns included."""
    import numpy as np
    from cases import gaussian
    from kshipra_amd.quantization import concat_quantized
    parts = [gaussian((n, 300), seed=70 + i) for i, n in enumerate((64, 16, 16))]
    fused = concat_quantized([_oracle_qw(w, scheme) for w in parts])
    whole = _oracle_qw(np.concatenate(parts, axis=0), scheme)
    assert fused.original_shape == whole.original_shape == (96, 300)
    assert torch.equal(fused.payload, whole.payload)
    assert torch.equal(fused.scales.view(torch.int16), whole.scales.view(torch.int16))
    assert fused.storage_bytes() == whole.storage_bytes()


def test_concat_rejects_mismatched_parts():
    import numpy as np
    from cases import gaussian
    from kshipra_amd.quantization import concat_quantized
    a = _oracle_qw(gaussian((16, 256), seed=1), "int4")
    b = _oracle_qw(gaussian((16, 384), seed=2), "int4")
    c = _oracle_qw(gaussian((16, 256), seed=3), "int8")
    for bad in ([a, b], [a, c], []):
        with pytest.raises(QuantizationError):
            concat_quantized(bad)
    with pytest.raises(QuantizationError):
        from kshipra_amd.quantization import FusedQuantizedLinear
        FusedQuantizedLinear([nn.Linear(4, 4)])


@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_gate_up_interleave_is_a_row_permutation(scheme):
    """interleave_gate_up equals quantizing the fp32 weight whose rows are the
    gate / up rows interleaved by 16-row tiles, bit for bit."""
    import numpy as np
    from cases import gaussian
    from kshipra_amd.quantization import interleave_gate_up
    g, u = gaussian((48, 300), seed=80), gaussian((48, 300), seed=81)
    fused = interleave_gate_up(_oracle_qw(g, scheme), _oracle_qw(u, scheme))
    rows = np.concatenate([np.concatenate([g[16 * b:16 * b + 16], u[16 * b:16 * b + 16]])
                           for b in range(3)])
    whole = _oracle_qw(rows, scheme)
    assert fused.original_shape == (96, 300)
    assert torch.equal(fused.payload, whole.payload)
    assert torch.equal(fused.scales.view(torch.int16), whole.scales.view(torch.int16))


def test_gate_up_interleave_rejects():
    from cases import gaussian
    from kshipra_amd.quantization import FusedGateUpSiLU, interleave_gate_up
    a = _oracle_qw(gaussian((32, 256), seed=1), "int4")
    for bad in (_oracle_qw(gaussian((32, 384), seed=2), "int4"),   # in_features
                _oracle_qw(gaussian((48, 256), seed=3), "int4"),   # out_features
                _oracle_qw(gaussian((32, 256), seed=4), "int8")):  # scheme
        with pytest.raises(QuantizationError):
            interleave_gate_up(a, bad)
    odd = _oracle_qw(gaussian((24, 256), seed=5), "int4")           # not 16-row tiles
    with pytest.raises(QuantizationError):
        interleave_gate_up(odd, odd)
    with pytest.raises(QuantizationError):
        FusedGateUpSiLU(nn.Linear(4, 4), nn.Linear(4, 4))


def test_silu_mul_workspace_and_argument_errors():
    lib = _lib.load()
    # M = 1 gate / up of Llama-3-8B: pairs of tiles in LDS, no workspace
    assert lib.kq_linear_silu_mul_workspace_bytes(4, 1, 14336, 4096, 128) == 0
    # GEMM path: operand planes (64-row tile) + the interleaved product
    ws = lib.kq_linear_silu_mul_workspace_bytes(4, 64, 14336, 4096, 128)
    assert ws >= 4 * 64 * 4096 + 4 * 64 * 2 * 14336
    # out_features not a multiple of 16, ldact too small, null act
    assert lib.kq_linear_silu_mul_int8(1, 1, 64, 1, 1, None, 1, 24, 24, 64, None, 0, None) == _lib.KQ_ERR_ARG
    assert lib.kq_linear_silu_mul_int8(1, 1, 64, 1, 1, None, 1, 16, 32, 64, None, 0, None) == _lib.KQ_ERR_ARG
    assert lib.kq_linear_silu_mul_int4(1, 1, 128, 1, 1, 128, 128, None, None, 32, 32, 128, None, 0,
                                       None) == _lib.KQ_ERR_ARG
    assert lib.kq_last_error() not in (None, b"")


def test_graph_workspaces_are_retained(monkeypatch):
    """Calls under HIP graph capture get workspaces that no eager call or
    other capture shares and that are never released while a graph may
    replay: a buffer superseded inside a capture is retired, not freed."""
    import weakref

    cid = {"v": None}
    monkeypatch.setattr(_lib, "_capture_id", lambda stream: cid["v"])
    monkeypatch.setattr(_lib, "_alloc", lambda dev, n: torch.empty(n, dtype=torch.uint8))
    monkeypatch.setattr(_lib, "_ws", {})
    monkeypatch.setattr(_lib, "_graph_ws", {})
    monkeypatch.setattr(_lib, "_graph_retired", [])
    dev = torch.device("cuda", 0)
    eager = _lib.workspace(dev, 7, 100)
    assert _lib.workspace(dev, 7, 100) is eager                 # eager calls share per stream
    cid["v"] = 11                                               # capture 11 on stream 7
    g1 = _lib.workspace(dev, 7, 100)
    assert g1 is not eager and _lib.workspace(dev, 7, 50) is g1  # shared within the capture
    g1_ref = weakref.ref(g1)
    g1_big = _lib.workspace(dev, 7, 4 << 20)                    # grows inside the capture
    assert g1_big is not g1
    del g1
    assert g1_ref() is not None                                 # the superseded buffer stays alive
    cid["v"] = 12                                               # another capture
    g2 = _lib.workspace(dev, 7, 100)
    assert g2 is not g1_big and g2 is not eager
    cid["v"] = None                                             # eager again, larger
    eager_big = _lib.workspace(dev, 7, 8 << 20)
    assert eager_big is not eager and eager_big is not g1_big and eager_big is not g2
    assert _lib.workspace(dev, 7, 0) is None
    _lib.release_graph_workspaces()
    assert g1_ref() is None                                     # released on request only


def test_scales_conversion_rules():
    """fp16 scales pass through; other float scales only when fp16 holds them
    exactly (the reference reads them with .to(float32)); others refuse."""
    from kshipra_amd.quantization import QuantizationError, _fp16_scales
    s16 = torch.tensor([0.5, 2.0 ** -20, 65504.0], dtype=torch.float16)
    assert _fp16_scales(s16) is s16 or torch.equal(_fp16_scales(s16), s16)
    assert torch.equal(_fp16_scales(s16.float()), s16)
    sb = torch.tensor([0.5, 2.0 ** -20, 3.0], dtype=torch.bfloat16)
    assert torch.equal(_fp16_scales(sb), sb.half())
    with pytest.raises(QuantizationError):
        _fp16_scales(torch.tensor([0.1], dtype=torch.float32))
    with pytest.raises(QuantizationError):
        _fp16_scales(torch.tensor([1], dtype=torch.int32))
