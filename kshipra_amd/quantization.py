"""Weight-only INT8 / INT4 quantization on MI355X -- drop-in for Kshipra's
``engine/quantization.py``.

Same public names, fields, scheme strings, dtypes, shapes, validation and
error types as the reference module:

* ``QuantizationError``            (engine/quantization.py:69-70)
* ``QuantizedWeight``              (:78-172)  payload / scales / scheme /
  original_shape / group_size / in_features_padded; ``storage_bytes()``;
  ``dequantize(dtype=torch.float16)``
* ``_validate_weight``             (:180-188)
* ``quantize_int8_per_channel``    (:196-223)
* ``_dequantize_int8_per_channel`` (:226-230)
* ``quantize_int4_per_group``      (:238-318)
* ``_dequantize_int4_per_group``   (:321-344)
* ``QuantizedLinear``              (:352-403)

Layouts are the reference's: INT8 payload ``int8 [out, in]`` with fp16 scales
``[out]``; INT4 payload ``uint8 [out, in_padded // 2]`` (low nibble = even
column, two's-complement nibbles) with fp16 scales ``[out, in_padded // G]``.

What differs is where the work runs.  Every compute entry point launches a
hand-written gfx950 HIP kernel from ``libkshipra_quant.so`` on the tensor's
device and torch's current stream:

* quantize / pack: bit-exact with the reference (true fp32 division, fp16
  round-to-nearest-even scale, round-half-to-even, NaN -> 0, +-inf -> clamp);
* ``QuantizedLinear.forward``: the fused dequant-matmul -- the packed payload
  is streamed once from HBM and never materialised; fp32 accumulation;
* ``dequantize``: exact ``q * s`` rounded to the requested dtype.

Tensors must live on a ROCm GPU.  A CPU tensor raises ``RuntimeError``: there
is no CPU fallback.  As in the reference, ``QuantizedWeight`` is a plain
attribute of ``QuantizedLinear`` (not a buffer), so move the float module to
the GPU *before* quantizing (engine/model.py:67,77-78 does exactly that).

Activations of dtype float16 / bfloat16 are computed in fp32 and the output is
rounded to the input dtype once (the reference instead rounds the weight to
that dtype first; the fp32 path is the more accurate of the two).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import _lib
from ._errors import QuantizationError

__all__ = [
    "QuantizationError",
    "QuantizedWeight",
    "quantize_int8_per_channel",
    "quantize_int4_per_group",
    "QuantizedLinear",
    "concat_quantized",
    "FusedQuantizedLinear",
    "quantized_linear_argmax",
    "interleave_gate_up",
    "quantized_gate_up_silu",
    "FusedGateUpSiLU",
]


# ---------------------------------------------------------------------- #
# Container (engine/quantization.py:78-172)
# ---------------------------------------------------------------------- #


@dataclass
class QuantizedWeight:
    """A quantized weight tensor plus the metadata needed to dequantize it.

    payload:            ``int8 [out, in]`` (INT8) or ``uint8 [out, in_padded // 2]`` (INT4)
    scales:             fp16 ``[out]`` (INT8) or ``[out, in_padded // group_size]`` (INT4)
    scheme:             ``"int8_per_channel"`` or ``"int4_per_group"``
    original_shape:     ``(out_features, in_features)``
    group_size:         ``G`` for INT4, ``None`` for INT8
    in_features_padded: ``ceil(in / G) * G`` for INT4, ``None`` for INT8
    """

    payload: torch.Tensor
    scales: torch.Tensor
    scheme: str
    original_shape: Tuple[int, int]
    group_size: Optional[int] = None
    in_features_padded: Optional[int] = None

    def __post_init__(self) -> None:
        # Same checks and messages as engine/quantization.py:108-152.
        if self.scheme not in ("int8_per_channel", "int4_per_group"):
            raise QuantizationError(f"unknown scheme {self.scheme!r}")
        out_features, _ = self.original_shape
        if self.scales.shape[0] != out_features:
            raise QuantizationError(
                f"scales.shape[0] = {self.scales.shape[0]} does not match "
                f"out_features = {out_features}")
        if self.scheme == "int8_per_channel":
            if self.payload.dtype != torch.int8:
                raise QuantizationError(f"INT8 payload must be int8, got {self.payload.dtype}")
            if self.scales.dim() != 1:
                raise QuantizationError(
                    f"INT8 scales must be 1-D [out_features], got {tuple(self.scales.shape)}")
            if tuple(self.payload.shape) != tuple(self.original_shape):
                raise QuantizationError(
                    f"INT8 payload shape {tuple(self.payload.shape)} != "
                    f"original_shape {self.original_shape}")
        else:
            if self.payload.dtype != torch.uint8:
                raise QuantizationError(f"INT4 payload must be uint8, got {self.payload.dtype}")
            if self.group_size is None or self.in_features_padded is None:
                raise QuantizationError("INT4 requires group_size and in_features_padded")
            expected_groups = self.in_features_padded // self.group_size
            if tuple(self.scales.shape) != (out_features, expected_groups):
                raise QuantizationError(
                    f"INT4 scales shape {tuple(self.scales.shape)} != "
                    f"({out_features}, {expected_groups})")
            expected_payload_cols = self.in_features_padded // 2
            if tuple(self.payload.shape) != (out_features, expected_payload_cols):
                raise QuantizationError(
                    f"INT4 payload shape {tuple(self.payload.shape)} != "
                    f"({out_features}, {expected_payload_cols})")

    def storage_bytes(self) -> int:
        """Bytes occupied by payload + scales (engine/quantization.py:154-159)."""
        return (self.payload.numel() * self.payload.element_size()
                + self.scales.numel() * self.scales.element_size())

    def dequantize(self, dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """Materialise ``original_shape`` in ``dtype`` (engine/quantization.py:161-172).

        The fp32 product ``q * s`` is exact; it is rounded to ``dtype`` once.
        """
        if self.scheme == "int8_per_channel":
            return _dequantize_int8_per_channel(self, dtype)
        return _dequantize_int4_per_group(self, dtype)


# ---------------------------------------------------------------------- #
# Helpers
# ---------------------------------------------------------------------- #


def _validate_dims(w: torch.Tensor) -> None:
    if w.dim() != 2:
        raise QuantizationError(f"weight must be 2-D, got {w.dim()}-D")
    if w.shape[0] == 0 or w.shape[1] == 0:
        raise QuantizationError(f"weight must have non-zero dims, got {tuple(w.shape)}")


def _weight_view(w: torch.Tensor) -> Tuple[torch.Tensor, int, int]:
    """fp32/fp16/bf16 view with unit column stride, and its kernel dtype code /
    leading dimension.  Other float dtypes are rounded to fp32 first, as
    ``w.to(torch.float32)`` does at engine/quantization.py:205."""
    w = w.detach()
    if w.dtype not in _lib.DTYPE_CODE:
        w = w.to(torch.float32)
    if w.stride(1) != 1 or (w.shape[0] > 1 and w.stride(0) < w.shape[1]):
        w = w.contiguous()
    ld = w.stride(0) if w.shape[0] > 1 else w.shape[1]
    return w, _lib.DTYPE_CODE[w.dtype], ld


def _raise_if_nonfinite(flag: torch.Tensor) -> None:
    if int(flag.item()) != 0:
        raise QuantizationError("weight contains non-finite values")


def _validate_weight(w: torch.Tensor) -> None:
    """engine/quantization.py:180-188: 2-D, non-empty, all finite (GPU pass)."""
    _validate_dims(w)
    _lib.require_device(w, "weight")
    lib = _lib.load()
    wv, code, ld = _weight_view(w)
    flag = torch.empty(1, dtype=torch.int32, device=w.device)
    _lib.check(lib.kq_check_finite(wv.data_ptr(), code, wv.shape[0], wv.shape[1], ld,
                                   flag.data_ptr(), _lib.stream_of(wv)))
    _raise_if_nonfinite(flag)


# ---------------------------------------------------------------------- #
# INT8 per-channel (engine/quantization.py:196-230)
# ---------------------------------------------------------------------- #


def quantize_int8_per_channel(w: torch.Tensor) -> QuantizedWeight:
    """Symmetric per-output-channel INT8 quantization, bit-exact with the reference.

    ``s[r] = fp16(max(max|W[r, :]| / 127, 1e-8))``; ``q = clamp(rint(W / s), -127, 127)``.
    One HIP kernel computes the row maxima, the scales and the payload; the
    finiteness check of :187 is fused into it.
    """
    _validate_dims(w)
    _lib.require_device(w, "weight")
    lib = _lib.load()
    wv, code, ld = _weight_view(w)
    n, k = wv.shape
    payload = torch.empty((n, k), dtype=torch.int8, device=w.device)
    scales = torch.empty((n,), dtype=torch.float16, device=w.device)
    flag = torch.empty(1, dtype=torch.int32, device=w.device)
    _lib.check(lib.kq_quantize_int8(wv.data_ptr(), code, n, k, ld, payload.data_ptr(),
                                    scales.data_ptr(), flag.data_ptr(), _lib.stream_of(wv)))
    _raise_if_nonfinite(flag)
    return QuantizedWeight(payload=payload, scales=scales, scheme="int8_per_channel",
                           original_shape=(int(n), int(k)))


def _out_dtype(dtype: torch.dtype) -> torch.dtype:
    return dtype if dtype in _lib.DTYPE_CODE else torch.float32


def _dequantize_int8_per_channel(qw: QuantizedWeight,
                                 dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """engine/quantization.py:226-230: ``q * s`` (exact in fp32), as ``dtype``."""
    _lib.require_device(qw.payload, "payload")
    lib = _lib.load()
    n, k = qw.original_shape
    od = _out_dtype(dtype)
    out = torch.empty((n, k), dtype=od, device=qw.payload.device)
    p, s = qw.payload.contiguous(), _fp16_scales(qw.scales)
    _lib.check(lib.kq_dequantize_int8(p.data_ptr(), s.data_ptr(), n, k, out.data_ptr(),
                                      _lib.DTYPE_CODE[od], _lib.stream_of(p)))
    return out if od == dtype else out.to(dtype)


# ---------------------------------------------------------------------- #
# INT4 per-group (engine/quantization.py:238-344)
# ---------------------------------------------------------------------- #


def quantize_int4_per_group(w: torch.Tensor, group_size: int = 128) -> QuantizedWeight:
    """Symmetric per-group INT4 quantization with nibble packing, bit-exact.

    ``G`` must be positive and even.  ``in_features`` is right-padded with
    zeros to a multiple of ``G``; ``s[r, g] = fp16(max(max|group| / 7, 1e-8))``;
    ``q = clamp(rint(W / s), -8, 7)``; ``byte[j] = (q[2j] & 0xF) | (q[2j+1] & 0xF) << 4``.
    """
    _validate_dims(w)
    if group_size <= 0 or group_size % 2 != 0:
        raise QuantizationError(f"group_size must be a positive even integer, got {group_size}")
    _lib.require_device(w, "weight")
    lib = _lib.load()
    wv, code, ld = _weight_view(w)
    n, k = wv.shape
    num_groups = (k + group_size - 1) // group_size
    kp = num_groups * group_size
    payload = torch.empty((n, kp // 2), dtype=torch.uint8, device=w.device)
    scales = torch.empty((n, num_groups), dtype=torch.float16, device=w.device)
    flag = torch.empty(1, dtype=torch.int32, device=w.device)
    _lib.check(lib.kq_quantize_int4(wv.data_ptr(), code, n, k, ld, group_size,
                                    payload.data_ptr(), scales.data_ptr(), flag.data_ptr(),
                                    _lib.stream_of(wv)))
    _raise_if_nonfinite(flag)
    return QuantizedWeight(payload=payload, scales=scales, scheme="int4_per_group",
                           original_shape=(int(n), int(k)), group_size=int(group_size),
                           in_features_padded=int(kp))


def _dequantize_int4_per_group(qw: QuantizedWeight,
                               dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """engine/quantization.py:321-344: unpack, sign-restore, scale, slice to ``in``."""
    assert qw.group_size is not None and qw.in_features_padded is not None
    _lib.require_device(qw.payload, "payload")
    lib = _lib.load()
    n, k = qw.original_shape
    od = _out_dtype(dtype)
    out = torch.empty((n, k), dtype=od, device=qw.payload.device)
    p, s = qw.payload.contiguous(), _fp16_scales(qw.scales)
    _lib.check(lib.kq_dequantize_int4(p.data_ptr(), s.data_ptr(), n, k, qw.group_size,
                                      qw.in_features_padded, out.data_ptr(),
                                      _lib.DTYPE_CODE[od], _lib.stream_of(p)))
    return out if od == dtype else out.to(dtype)


# ---------------------------------------------------------------------- #
# Fused dequant-matmul (engine/quantization.py:394-396)
# ---------------------------------------------------------------------- #


class _Operands:
    """Device operands of one dequant-matmul call, checked before any launch."""

    __slots__ = ("x2", "ldx", "m", "payload", "scales", "bias", "stream", "lib")


def _fp16_scales(scales: torch.Tensor) -> torch.Tensor:
    """The kernels read fp16 scales (what the quantizers store).  Scales of
    another float dtype are accepted when fp16 holds them exactly -- the
    reference's ``scales.to(torch.float32)`` (engine/quantization.py:228, :339)
    then sees the same values -- and refused otherwise."""
    if scales.dtype == torch.float16:
        return scales.contiguous()
    if not scales.dtype.is_floating_point:
        raise QuantizationError(f"scales must be a float tensor, got {scales.dtype}")
    s16 = scales.to(torch.float16)
    if not torch.equal(s16.to(scales.dtype), scales):
        raise QuantizationError(
            f"scales of dtype {scales.dtype} are not exactly representable in float16")
    return s16.contiguous()


def _operands(x: torch.Tensor, qw: QuantizedWeight, bias: Optional[torch.Tensor],
              out_features: int) -> _Operands:
    """Shape, device and dtype checks shared by every dequant-matmul entry.

    As ``F.linear`` would: a mismatched inner dimension and operands on
    different devices raise ``RuntimeError`` (the reference's payload is a
    plain attribute that ``module.to()`` leaves behind, engine/quantization.py:
    383-392, while its bias buffer moves).  The payload and fp16 scales are
    made contiguous, the bias fp32 and contiguous; ``x`` is viewed as a
    ``[M, in_features]`` fp32 matrix with unit column stride.
    """
    _lib.require_device(x, "input")
    in_features = qw.original_shape[1]
    if x.shape[-1] != in_features:
        raise RuntimeError(
            f"mat1 and mat2 shapes cannot be multiplied "
            f"({x.numel() // max(x.shape[-1], 1)}x{x.shape[-1]} and {in_features}x{out_features})")
    for name, t in (("weight payload", qw.payload), ("weight scales", qw.scales),
                    ("bias", bias)):
        if t is not None and t.device != x.device:
            raise RuntimeError(f"input on {x.device} but {name} on {t.device}")
    if bias is not None and tuple(bias.shape) != (out_features,):
        raise RuntimeError(f"bias shape {tuple(bias.shape)} != ({out_features},)")
    op = _Operands()
    op.lib = _lib.load()
    x2 = x.reshape(-1, in_features)
    if x2.dtype != torch.float32:
        x2 = x2.to(torch.float32)
    if x2.stride(1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < in_features):
        x2 = x2.contiguous()
    op.x2, op.m = x2, x2.shape[0]
    op.ldx = x2.stride(0) if op.m > 1 else in_features
    op.payload = qw.payload.contiguous()
    op.scales = _fp16_scales(qw.scales)
    op.bias = None
    if bias is not None:
        b = bias.detach()
        if b.dtype != torch.float32 or not b.is_contiguous():
            b = b.to(torch.float32).contiguous()
        op.bias = b
    op.stream = _lib.stream_of(x2)
    return op


def quantized_linear(x: torch.Tensor, qw: QuantizedWeight,
                     bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``F.linear(x, qw.dequantize(x.dtype), bias)`` without materialising the
    weight: one fused HIP dequant-matmul over the packed payload."""
    out_features, in_features = qw.original_shape
    op = _operands(x, qw, bias, out_features)
    lib, m = op.lib, op.m
    y = torch.empty((m, out_features), dtype=torch.float32, device=x.device)
    if m > 0:
        args = (op.x2.data_ptr(), m, op.ldx, op.payload.data_ptr(), op.scales.data_ptr())
        if qw.scheme == "int8_per_channel":
            nbytes = lib.kq_linear_workspace_bytes(8, m, out_features, in_features, 0)
            ws = _lib.workspace(x.device, op.stream, nbytes)
            _lib.check(lib.kq_linear_int8(
                *args, _lib.ptr(op.bias), y.data_ptr(), out_features, out_features, in_features,
                _lib.ptr(ws), nbytes, op.stream))
        else:
            g = qw.group_size
            nbytes = lib.kq_linear_workspace_bytes(4, m, out_features, in_features, g)
            ws = _lib.workspace(x.device, op.stream, nbytes)
            _lib.check(lib.kq_linear_int4(
                *args, g, qw.in_features_padded, _lib.ptr(op.bias), y.data_ptr(), out_features,
                out_features, in_features, _lib.ptr(ws), nbytes, op.stream))
    y = y.reshape(*x.shape[:-1], out_features)
    return y if x.dtype == torch.float32 else y.to(x.dtype)


def quantized_linear_argmax(x: torch.Tensor, qw: QuantizedWeight,
                            bias: Optional[torch.Tensor] = None, return_logits: bool = False):
    """Greedy token per row of ``F.linear(x, qw.dequantize(), bias)``: the
    lm_head projection (engine/model.py:151) and ``logits.argmax()``
    (:187, :200; first index of the maximum, a NaN counts as the maximum)
    in one call.  The skinny kernel reduces each tile's logits to a partial
    argmax in its epilogue; the logits are written only when
    ``return_logits`` is set.  Returns int64 tokens of shape ``x.shape[:-1]``
    (and the fp32 logits)."""
    out_features, in_features = qw.original_shape
    op = _operands(x, qw, bias, out_features)
    lib, m = op.lib, op.m
    tokens = torch.empty((m,), dtype=torch.int64, device=x.device)
    logits = (torch.empty((m, out_features), dtype=torch.float32, device=x.device)
              if return_logits else None)
    if m > 0:
        args = (op.x2.data_ptr(), m, op.ldx, op.payload.data_ptr(), op.scales.data_ptr())
        lp = _lib.ptr(logits)
        if qw.scheme == "int8_per_channel":
            nbytes = lib.kq_linear_argmax_workspace_bytes(8, m, out_features, in_features, 0)
            ws = _lib.workspace(x.device, op.stream, nbytes)
            _lib.check(lib.kq_linear_argmax_int8(
                *args, _lib.ptr(op.bias), lp, out_features, out_features, in_features,
                tokens.data_ptr(), _lib.ptr(ws), nbytes, op.stream))
        else:
            g = qw.group_size
            nbytes = lib.kq_linear_argmax_workspace_bytes(4, m, out_features, in_features, g)
            ws = _lib.workspace(x.device, op.stream, nbytes)
            _lib.check(lib.kq_linear_argmax_int4(
                *args, g, qw.in_features_padded, _lib.ptr(op.bias), lp, out_features, out_features,
                in_features, tokens.data_ptr(), _lib.ptr(ws), nbytes, op.stream))
    tokens = tokens.reshape(x.shape[:-1])
    if return_logits:
        return tokens, logits.reshape(*x.shape[:-1], out_features)
    return tokens


# ---------------------------------------------------------------------- #
# Module wrapper (engine/quantization.py:352-403)
# ---------------------------------------------------------------------- #


class QuantizedLinear(nn.Module):
    """A drop-in replacement for ``nn.Linear`` with quantized weights.

    ``forward(x) = x @ (q * s)^T + bias`` computed by the fused HIP
    dequant-matmul; the bias stays a registered buffer in its original dtype.
    """

    def __init__(self, linear: nn.Linear, scheme: str = "int8", group_size: int = 128) -> None:
        super().__init__()
        if not isinstance(linear, nn.Linear):
            raise QuantizationError(f"expected nn.Linear, got {type(linear).__name__}")
        if scheme not in ("int8", "int4"):
            raise QuantizationError(f"scheme must be 'int8' or 'int4', got {scheme!r}")
        self.in_features = linear.in_features
        self.out_features = linear.out_features
        self.scheme = scheme
        w = linear.weight.detach()
        if scheme == "int8":
            self.weight = quantize_int8_per_channel(w)
        else:
            self.weight = quantize_int4_per_group(w, group_size)
        if linear.bias is not None:
            self.register_buffer("bias", linear.bias.detach().clone())
        else:
            self.bias = None

    @classmethod
    def from_quantized(cls, qw: QuantizedWeight, bias: Optional[torch.Tensor] = None) -> "QuantizedLinear":
        """A module around an already quantized weight (e.g. loaded from disk:
        kshipra_amd.checkpoint), without the float original."""
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.out_features, self.in_features = qw.original_shape
        self.scheme = "int8" if qw.scheme == "int8_per_channel" else "int4"
        self.weight = qw
        if bias is not None:
            if bias.shape != (self.out_features,):
                raise QuantizationError(f"bias shape {tuple(bias.shape)} != ({self.out_features},)")
            self.register_buffer("bias", bias.detach().clone())
        else:
            self.bias = None
        return self

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return quantized_linear(x, self.weight, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"scheme={self.scheme}, storage_bytes={self.weight.storage_bytes()}")


# ---------------------------------------------------------------------- #
# Fused projections of one input (q/k/v, gate/up)
# ---------------------------------------------------------------------- #


def concat_quantized(parts) -> QuantizedWeight:
    """Row-stack quantized weights that share ``in_features`` and scheme.

    Every row (INT8) or row x group (INT4) is quantized on its own
    (engine/quantization.py:206-208, :293-295), so stacking the payloads and
    scales equals quantizing the row-stacked fp32 weight -- bit for bit.  One
    dequant-GEMV over the stacked weight then replaces one launch per part
    (the adjacent q/k/v calls of engine/model.py:115-117, gate/up of the MLP).
    """
    parts = list(parts)
    if not parts:
        raise QuantizationError("nothing to concatenate")
    first = parts[0]
    for p in parts[1:]:
        if (p.scheme != first.scheme or p.original_shape[1] != first.original_shape[1]
                or p.group_size != first.group_size
                or p.in_features_padded != first.in_features_padded):
            raise QuantizationError("parts differ in scheme, in_features or group size")
        if p.payload.device != first.payload.device:
            raise QuantizationError("parts live on different devices")
    out = sum(p.original_shape[0] for p in parts)
    return QuantizedWeight(
        payload=torch.cat([p.payload for p in parts], dim=0),
        scales=torch.cat([p.scales for p in parts], dim=0),
        scheme=first.scheme,
        original_shape=(out, first.original_shape[1]),
        group_size=first.group_size,
        in_features_padded=first.in_features_padded,
    )


class FusedQuantizedLinear(nn.Module):
    """Several ``QuantizedLinear`` of the same input run as one launch.

    ``forward(x)`` returns one output per part, as views of the single
    ``[..., sum(out_features)]`` result (same values the parts would give,
    up to fp32 summation order).  Parts without a bias contribute zeros to the
    stacked bias when any part has one.
    """

    def __init__(self, parts) -> None:
        super().__init__()
        parts = list(parts)
        for p in parts:
            if not isinstance(p, QuantizedLinear):
                raise QuantizationError(f"expected QuantizedLinear, got {type(p).__name__}")
        self.in_features = parts[0].in_features
        self.splits = [p.out_features for p in parts]
        self.out_features = sum(self.splits)
        self.scheme = parts[0].scheme
        self.weight = concat_quantized([p.weight for p in parts])
        if any(p.bias is not None for p in parts):
            dev = self.weight.payload.device
            self.register_buffer("bias", torch.cat([
                p.bias.detach().to(torch.float32) if p.bias is not None
                else torch.zeros(p.out_features, dtype=torch.float32, device=dev) for p in parts]))
        else:
            self.bias = None

    def forward(self, x: torch.Tensor):
        return quantized_linear(x, self.weight, self.bias).split(self.splits, dim=-1)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.splits}, "
                f"scheme={self.scheme}, storage_bytes={self.weight.storage_bytes()}")


# ---------------------------------------------------------------------- #
# Gate / up projection with the SiLU gate (the MLP input)
# ---------------------------------------------------------------------- #

_PAIR = 16  # rows per tile of the gate / up interleave


def _interleave_rows(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    n = g.shape[0]
    rest = g.shape[1:]
    return torch.stack([g.reshape(n // _PAIR, _PAIR, *rest), u.reshape(n // _PAIR, _PAIR, *rest)],
                       dim=1).reshape(2 * n, *rest)


def interleave_gate_up(gate: QuantizedWeight, up: QuantizedWeight) -> QuantizedWeight:
    """Gate and up weights interleaved by 16-row tiles (rows 32 b .. 32 b + 15
    are gate rows 16 b .., the next 16 the same up rows), the layout the fused
    SiLU-gated projection reads.  Rows are quantized independently
    (engine/quantization.py:206-208, :293-295), so this is a permutation of
    the row-stacked quantization, bit for bit."""
    if (gate.scheme != up.scheme or gate.original_shape != up.original_shape
            or gate.group_size != up.group_size
            or gate.in_features_padded != up.in_features_padded):
        raise QuantizationError("gate and up differ in scheme, shape or group size")
    if gate.payload.device != up.payload.device:
        raise QuantizationError("gate and up live on different devices")
    n, k = gate.original_shape
    if n % _PAIR != 0:
        raise QuantizationError(f"out_features {n} is not a multiple of {_PAIR}")
    return QuantizedWeight(
        payload=_interleave_rows(gate.payload, up.payload),
        scales=_interleave_rows(gate.scales, up.scales),
        scheme=gate.scheme, original_shape=(2 * n, k), group_size=gate.group_size,
        in_features_padded=gate.in_features_padded)


def quantized_gate_up_silu(x: torch.Tensor, qw: QuantizedWeight,
                           bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``silu(x Wg^T + bg) * (x Wu^T + bu)`` -- the input of the MLP's down
    projection (engine/model.py:147 runs ``layer.mlp``, whose gate_proj and
    up_proj are ``QuantizedLinear`` after engine/model.py:80-91) -- from the
    interleaved weight of ``interleave_gate_up`` (and bias interleaved the
    same way), in one dequant-matmul launch whose epilogue applies the gate
    (M <= 16), or the matmul plus one pairing kernel."""
    rows, in_features = qw.original_shape
    nh = rows // 2
    op = _operands(x, qw, bias, rows)
    lib, m = op.lib, op.m
    act = torch.empty((m, nh), dtype=torch.float32, device=x.device)
    if m > 0:
        args = (op.x2.data_ptr(), m, op.ldx, op.payload.data_ptr(), op.scales.data_ptr())
        if qw.scheme == "int8_per_channel":
            nbytes = lib.kq_linear_silu_mul_workspace_bytes(8, m, nh, in_features, 0)
            ws = _lib.workspace(x.device, op.stream, nbytes)
            _lib.check(lib.kq_linear_silu_mul_int8(
                *args, _lib.ptr(op.bias), act.data_ptr(), nh, nh, in_features, _lib.ptr(ws),
                nbytes, op.stream))
        else:
            g = qw.group_size
            nbytes = lib.kq_linear_silu_mul_workspace_bytes(4, m, nh, in_features, g)
            ws = _lib.workspace(x.device, op.stream, nbytes)
            _lib.check(lib.kq_linear_silu_mul_int4(
                *args, g, qw.in_features_padded, _lib.ptr(op.bias), act.data_ptr(), nh, nh,
                in_features, _lib.ptr(ws), nbytes, op.stream))
    act = act.reshape(*x.shape[:-1], nh)
    return act if x.dtype == torch.float32 else act.to(x.dtype)


class FusedGateUpSiLU(nn.Module):
    """``silu(gate(x)) * up(x)`` for two ``QuantizedLinear`` of one input (the
    Llama / Qwen2 MLP's gate_proj and up_proj) as one launch over their
    16-row-tile interleaved weight.  Same values as the two projections
    followed by ``F.silu(g) * u``, up to fp32 summation order and the
    exponential's rounding."""

    def __init__(self, gate: "QuantizedLinear", up: "QuantizedLinear") -> None:
        super().__init__()
        for p in (gate, up):
            if not isinstance(p, QuantizedLinear):
                raise QuantizationError(f"expected QuantizedLinear, got {type(p).__name__}")
        self.in_features = gate.in_features
        self.out_features = gate.out_features
        self.scheme = gate.scheme
        self.weight = interleave_gate_up(gate.weight, up.weight)
        if gate.bias is not None or up.bias is not None:
            dev = self.weight.payload.device

            def _b(p):
                return (p.bias.detach().to(torch.float32) if p.bias is not None
                        else torch.zeros(p.out_features, dtype=torch.float32, device=dev))
            self.register_buffer("bias", _interleave_rows(_b(gate), _b(up)))
        else:
            self.bias = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return quantized_gate_up_silu(x, self.weight, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"scheme={self.scheme}, storage_bytes={self.weight.storage_bytes()}")
