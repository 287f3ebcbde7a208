"""The reference's CPU forward restated in torch (test infrastructure only).

Kshipra's ``QuantizedLinear.forward`` materialises the dequantized weight with
torch CPU ops and calls ``F.linear`` (engine/quantization.py:394-396); the
dequantization is ``q.to(float32) * s`` per output channel for INT8
(:226-230) and, for INT4, unpack the low / high nibbles, interleave them,
restore the sign (u >= 8 -> u - 16), multiply by the group scale expanded
over its G columns and slice off the padding (:321-344).  This module runs
those same tensor operations on the CPU so that ``bench.py`` can time the
reference's own path (torch's intra-op threads, as the reference gets them)
beside the GPU kernels.  It is the timed CPU baseline, never a product path:
``kshipra_amd`` does not import it.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F


def dequantize_int8(payload: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """engine/quantization.py:226-230: fp32 [N, K] = q * s[:, None]."""
    return payload.to(torch.float32) * scales.to(torch.float32).unsqueeze(1)


def dequantize_int4(payload: torch.Tensor, scales: torch.Tensor, in_features: int,
                    group_size: int) -> torch.Tensor:
    """engine/quantization.py:321-344: nibble unpack (low nibble = even
    column), two's-complement sign restore, per-group scale, padding sliced."""
    n, half = payload.shape
    kp = 2 * half
    lo = (payload & 0x0F).to(torch.int16)
    hi = ((payload >> 4) & 0x0F).to(torch.int16)
    u = torch.stack([lo, hi], dim=-1).reshape(n, kp)
    q = torch.where(u >= 8, u - 16, u).to(torch.int8)
    s = scales.to(torch.float32).unsqueeze(-1).expand(-1, -1, group_size).reshape(n, kp)
    return (q.to(torch.float32) * s)[:, :in_features]


def linear(x: torch.Tensor, payload: torch.Tensor, scales: torch.Tensor, scheme: str,
           in_features: int, group_size: int = 128,
           bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """engine/quantization.py:394-396: F.linear(x, dequantize(), bias) in fp32."""
    if scheme == "int8":
        w = dequantize_int8(payload, scales)
    else:
        w = dequantize_int4(payload, scales, in_features, group_size)
    return F.linear(x, w, bias)
