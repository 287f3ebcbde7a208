"""On-disk format and load path for quantized weights.

* ``save_quantized(qw, path)`` / ``load_quantized(path, device)``: one weight
  as the dict Kshipra's tests save (``torch.save({"payload": ..., "scales":
  ...})``, tests/test_quantization.py:312), plus the metadata a
  ``QuantizedWeight`` needs (``scheme``, ``original_shape``, ``group_size``,
  ``in_features_padded``) so it loads back without the fp32 original.
  ``load_quantized`` also reads the reference's bare ``{"payload",
  "scales"}`` dict: the scheme follows from the payload dtype (int8 ->
  per-channel, uint8 -> packed INT4), the shape from the payload and the
  INT4 group size from ``2 * payload columns / scale columns``; an INT4
  weight whose ``in_features`` was padded needs ``in_features`` from the
  caller (the padding is not recorded in that dict).  Read with
  ``torch.load(weights_only=True)``: nothing in the file is executed.
* ``save_quantized_weights(weights, path)`` / ``load_quantized_weights(path,
  device)``: a name -> ``QuantizedWeight`` mapping (a whole model's
  projections) as one safetensors file, tensors ``<name>.payload`` /
  ``<name>.scales`` and the metadata in the header.

Loading puts only the packed payload and fp16 scales in device memory (the
fp32 / fp16 weight is never materialised), so a quantized model occupies
``sum(qw.storage_bytes())`` of HBM.  Every loaded weight is re-validated by
``QuantizedWeight.__post_init__`` (engine/quantization.py:108-152).
"""

from __future__ import annotations

import json
from typing import Dict, Optional, Union

import torch

from ._errors import QuantizationError
from .quantization import QuantizedWeight

_META_KEYS = ("scheme", "original_shape", "group_size", "in_features_padded")


def _meta(qw: QuantizedWeight) -> dict:
    return {"scheme": qw.scheme, "original_shape": [int(v) for v in qw.original_shape],
            "group_size": qw.group_size, "in_features_padded": qw.in_features_padded}


def _build(payload: torch.Tensor, scales: torch.Tensor, meta: dict) -> QuantizedWeight:
    for key in _META_KEYS:
        if key not in meta:
            raise QuantizationError(f"quantized checkpoint lacks {key!r}")
    return QuantizedWeight(payload=payload, scales=scales, scheme=meta["scheme"],
                           original_shape=tuple(int(v) for v in meta["original_shape"]),
                           group_size=meta["group_size"],
                           in_features_padded=meta["in_features_padded"])


def save_quantized(qw: QuantizedWeight, path: str) -> None:
    """``{"payload", "scales"}`` (the reference's dict) plus metadata."""
    d = {"payload": qw.payload.detach().cpu(), "scales": qw.scales.detach().cpu()}
    d.update(_meta(qw))
    torch.save(d, path)


def _infer_meta(payload: torch.Tensor, scales: torch.Tensor,
                in_features: Optional[int], group_size: Optional[int]) -> dict:
    """Metadata of a bare ``{"payload", "scales"}`` dict (the layouts of
    engine/quantization.py:40-46)."""
    if payload.dim() != 2:
        raise QuantizationError(f"payload must be 2-D, got {tuple(payload.shape)}")
    n, cols = payload.shape
    if payload.dtype == torch.int8:
        k = cols if in_features is None else int(in_features)
        if k != cols:
            raise QuantizationError(f"in_features {k} != INT8 payload columns {cols}")
        return {"scheme": "int8_per_channel", "original_shape": [n, k], "group_size": None,
                "in_features_padded": None}
    if payload.dtype != torch.uint8:
        raise QuantizationError(f"payload dtype {payload.dtype} is neither int8 nor uint8")
    if scales.dim() != 2 or scales.shape[1] == 0:
        raise QuantizationError(f"INT4 scales must be 2-D [out, groups], got {tuple(scales.shape)}")
    kp = 2 * cols
    if kp % scales.shape[1] != 0:
        raise QuantizationError(f"{kp} padded columns do not split into {scales.shape[1]} groups")
    g = kp // scales.shape[1]
    if group_size is not None and int(group_size) != g:
        raise QuantizationError(f"group_size {group_size} != {g} implied by the payload and scales")
    k = kp if in_features is None else int(in_features)
    if not (kp - g < k <= kp):
        raise QuantizationError(f"in_features {k} is inconsistent with {kp} padded columns (G = {g})")
    return {"scheme": "int4_per_group", "original_shape": [n, k], "group_size": g,
            "in_features_padded": kp}


def load_quantized(path: str, device: Union[str, torch.device, None] = None,
                   in_features: Optional[int] = None,
                   group_size: Optional[int] = None) -> QuantizedWeight:
    """One ``QuantizedWeight`` from ``path``, its tensors placed on ``device``.

    Files written by ``save_quantized`` carry their metadata; the reference's
    bare ``{"payload", "scales"}`` dict has it inferred (``in_features`` /
    ``group_size``, when given, are checked against it).
    """
    d = torch.load(path, map_location=device if device is not None else "cpu", weights_only=True)
    if not isinstance(d, dict) or "payload" not in d or "scales" not in d:
        raise QuantizationError(f"{path}: not a quantized weight (expected payload and scales)")
    if any(key in d for key in _META_KEYS):
        qw = _build(d["payload"], d["scales"], d)
        if in_features is not None and int(in_features) != qw.original_shape[1]:
            raise QuantizationError(f"in_features {in_features} != saved {qw.original_shape[1]}")
        return qw
    return _build(d["payload"], d["scales"], _infer_meta(d["payload"], d["scales"], in_features,
                                                         group_size))


def save_quantized_weights(weights: Dict[str, QuantizedWeight], path: str,
                           extra: Optional[Dict[str, torch.Tensor]] = None) -> None:
    """All quantized weights (and optional plain tensors, e.g. norms and
    embeddings) in one safetensors file."""
    from safetensors.torch import save_file
    tensors, meta = {}, {}
    for name, qw in weights.items():
        tensors[f"{name}.payload"] = qw.payload.detach().contiguous().cpu()
        tensors[f"{name}.scales"] = qw.scales.detach().contiguous().cpu()
        meta[name] = _meta(qw)
    for name, t in (extra or {}).items():
        if name in tensors:
            raise QuantizationError(f"duplicate tensor name {name!r}")
        tensors[name] = t.detach().cpu().clone()   # tied tensors (embedding / lm_head) stored apart
    save_file(tensors, path, metadata={"kshipra_quantized": json.dumps(meta)})


def load_quantized_weights(path: str, device: Union[str, torch.device] = "cpu"):
    """Returns ``(weights, extra)``: name -> ``QuantizedWeight`` on ``device``
    and the plain tensors saved alongside."""
    from safetensors import safe_open
    dev = str(device)
    with safe_open(path, framework="pt", device=dev) as f:
        meta = json.loads((f.metadata() or {}).get("kshipra_quantized", "{}"))
        weights = {name: _build(f.get_tensor(f"{name}.payload"), f.get_tensor(f"{name}.scales"), m)
                   for name, m in meta.items()}
        taken = {f"{n}.{s}" for n in meta for s in ("payload", "scales")}
        extra = {k: f.get_tensor(k) for k in f.keys() if k not in taken}
    return weights, extra
