"""Quantize / pack / dequantize / linear restatements (test infrastructure only).

Two independent restatements of Kshipra ``engine/quantization.py``:

* ``c_*``  -- ctypes wrappers over ``kq_oracle.c`` (scalar C, binary32);
* ``np_*`` -- vectorised numpy (binary32 arithmetic, numpy's own fp16 cast).

Linear (``engine/quantization.py:394-396``): the reference materialises the
exact fp32 weight ``q * s`` and calls ``F.linear``.  ``linear_f64`` evaluates
the same sum in float64 (the value every fp32 implementation approximates);
``linear_f32`` is the reference's own fp32 "materialise, then BLAS" order and
is what the CPU baseline times.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkq_oracle.so")
_lib = None


def lib() -> ctypes.CDLL:
    """Load the compiled C restatement (built by ``make -C oracle``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library not built: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        i64, vp = ctypes.c_int64, ctypes.c_void_p
        L.kqo_f32_to_f16.argtypes = [ctypes.c_float]
        L.kqo_f32_to_f16.restype = ctypes.c_uint16
        L.kqo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.kqo_f16_to_f32.restype = ctypes.c_float
        L.kqo_quantize_int8.argtypes = [vp, i64, i64, i64, vp, vp]
        L.kqo_quantize_int4.argtypes = [vp, i64, i64, i64, i64, vp, vp]
        L.kqo_dequantize_int8.argtypes = [vp, vp, i64, i64, vp]
        L.kqo_dequantize_int4.argtypes = [vp, vp, i64, i64, i64, i64, vp]
        L.kqo_count_nonfinite.argtypes = [vp, i64, i64, i64]
        L.kqo_count_nonfinite.restype = i64
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _as_f32_rows(w: np.ndarray) -> np.ndarray:
    """``w.detach().to(torch.float32)`` (engine/quantization.py:205, :282):
    fp16/bf16/fp32 -> fp32 is exact; a row-major contiguous copy."""
    return np.ascontiguousarray(np.asarray(w, dtype=np.float32))


# ---------------------------------------------------------------------- #
# C restatement
# ---------------------------------------------------------------------- #


def c_f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    L = lib()
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([L.kqo_f32_to_f16(float(v)) for v in flat], dtype=np.uint16).reshape(np.shape(x))


def c_quantize_int8(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """engine/quantization.py:196-223.  Returns (payload int8 [N,K], scales fp16 [N])."""
    w = _as_f32_rows(w)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty((n,), np.uint16)
    lib().kqo_quantize_int8(_ptr(w), n, k, k, _ptr(q), _ptr(s))
    return q, s.view(np.float16)


def c_quantize_int4(w: np.ndarray, group_size: int = 128) -> Tuple[np.ndarray, np.ndarray, int]:
    """engine/quantization.py:238-318.  Returns (payload uint8 [N,Kp/2], scales fp16 [N,ng], Kp)."""
    w = _as_f32_rows(w)
    n, k = w.shape
    ng = (k + group_size - 1) // group_size
    kp = ng * group_size
    q = np.empty((n, kp // 2), np.uint8)
    s = np.empty((n, ng), np.uint16)
    lib().kqo_quantize_int4(_ptr(w), n, k, k, group_size, _ptr(q), _ptr(s))
    return q, s.view(np.float16), kp


def c_dequantize_int8(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """engine/quantization.py:226-230."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    s = np.ascontiguousarray(s, dtype=np.float16).view(np.uint16)
    n, k = q.shape
    out = np.empty((n, k), np.float32)
    lib().kqo_dequantize_int8(_ptr(q), _ptr(s), n, k, _ptr(out))
    return out


def c_dequantize_int4(q: np.ndarray, s: np.ndarray, k: int, group_size: int) -> np.ndarray:
    """engine/quantization.py:321-344."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.float16).view(np.uint16)
    n = q.shape[0]
    kp = q.shape[1] * 2
    out = np.empty((n, k), np.float32)
    lib().kqo_dequantize_int4(_ptr(q), _ptr(s), n, k, group_size, kp, _ptr(out))
    return out


def c_count_nonfinite(w: np.ndarray) -> int:
    w = _as_f32_rows(w)
    return int(lib().kqo_count_nonfinite(_ptr(w), w.shape[0], w.shape[1], w.shape[1]))


# ---------------------------------------------------------------------- #
# numpy restatement (independent of the C one)
# ---------------------------------------------------------------------- #


def _round_clamp_i8(t: np.ndarray, lo: int, hi: int) -> np.ndarray:
    """``torch.round(t).clamp(lo, hi).to(int8)``: half-to-even, NaN -> 0."""
    r = np.rint(t)
    r = np.where(np.isnan(r), np.float32(0), np.clip(r, lo, hi))
    return r.astype(np.int8)


def np_quantize_int8(w: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """engine/quantization.py:196-223 in numpy binary32."""
    w32 = _as_f32_rows(w)
    m = np.abs(w32).max(axis=1)
    s32 = np.maximum(m / np.float32(127.0), np.float32(1e-8))
    s16 = s32.astype(np.float16)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = w32 / s16.astype(np.float32)[:, None]
    return _round_clamp_i8(t, -127, 127), s16


def np_quantize_int4(w: np.ndarray, group_size: int = 128) -> Tuple[np.ndarray, np.ndarray, int]:
    """engine/quantization.py:238-318 in numpy binary32."""
    w32 = _as_f32_rows(w)
    n, k = w32.shape
    ng = (k + group_size - 1) // group_size
    kp = ng * group_size
    wp = np.zeros((n, kp), np.float32)
    wp[:, :k] = w32
    wg = wp.reshape(n, ng, group_size)
    m = np.abs(wg).max(axis=-1)
    s32 = np.maximum(m / np.float32(7.0), np.float32(1e-8))
    s16 = s32.astype(np.float16)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = wg / s16.astype(np.float32)[..., None]
    q = _round_clamp_i8(t, -8, 7).reshape(n, kp)
    u = q.view(np.uint8) & np.uint8(0x0F)
    packed = (u[:, 0::2] | (u[:, 1::2] << np.uint8(4))).astype(np.uint8)
    return packed, s16, kp


def np_unpack_int4(q: np.ndarray) -> np.ndarray:
    """Packed uint8 [N, Kp/2] -> signed int8 [N, Kp] (engine/quantization.py:327-335)."""
    lo = (q & 0x0F).astype(np.int16)
    hi = ((q >> 4) & 0x0F).astype(np.int16)
    u = np.stack([lo, hi], axis=-1).reshape(q.shape[0], q.shape[1] * 2)
    return np.where(u >= 8, u - 16, u).astype(np.int8)


def np_dequantize_int8(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    return q.astype(np.float32) * np.asarray(s, np.float16).astype(np.float32)[:, None]


def np_dequantize_int4(q: np.ndarray, s: np.ndarray, k: int, group_size: int) -> np.ndarray:
    v = np_unpack_int4(q).astype(np.float32)
    sc = np.repeat(np.asarray(s, np.float16).astype(np.float32), group_size, axis=1)
    return (v * sc)[:, :k]


# ---------------------------------------------------------------------- #
# Linear (engine/quantization.py:394-396)
# ---------------------------------------------------------------------- #


def linear_f64(x: np.ndarray, w_hat: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """``x @ w_hat.T + b`` accumulated in float64.  ``w_hat`` is the exact fp32
    dequantized weight, so the only rounding is float64's."""
    y = np.asarray(x, np.float64) @ np.asarray(w_hat, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


def linear_f32(x: np.ndarray, w_hat: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """The reference's fp32 order: materialised weight, then one fp32 BLAS
    GEMM (``F.linear``), then the bias."""
    y = np.asarray(x, np.float32) @ np.asarray(w_hat, np.float32).T
    if bias is not None:
        y = y + np.asarray(bias, np.float32)
    return y


def dequantize(qw: dict) -> np.ndarray:
    """Dispatch on a dict ``{"scheme", "payload", "scales", "k", "group_size"}``."""
    if qw["scheme"] == "int8_per_channel":
        return c_dequantize_int8(qw["payload"], qw["scales"])
    return c_dequantize_int4(qw["payload"], qw["scales"], qw["k"], qw["group_size"])


def quantize(w: np.ndarray, scheme: str, group_size: int = 128) -> dict:
    if scheme in ("int8", "int8_per_channel"):
        q, s = c_quantize_int8(w)
        return {"scheme": "int8_per_channel", "payload": q, "scales": s, "k": w.shape[1], "group_size": None}
    q, s, kp = c_quantize_int4(w, group_size)
    return {"scheme": "int4_per_group", "payload": q, "scales": s, "k": w.shape[1],
            "group_size": group_size, "k_padded": kp}


def algorithmic_bytes(m: int, n: int, k: int, scheme: str, group_size: int = 128,
                      bias: bool = False) -> int:
    """payload + scales + x (fp32) + y (fp32) + bias, each counted once."""
    if scheme.startswith("int8"):
        w = n * k + 2 * n
    else:
        ng = (k + group_size - 1) // group_size
        w = n * ng * group_size // 2 + 2 * n * ng
    return w + 4 * m * k + 4 * m * n + (4 * n if bias else 0)
