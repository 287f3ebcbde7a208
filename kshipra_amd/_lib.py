"""ctypes binding of ``libkshipra_quant.so`` (declared in ``include/kshipra_quant.h``).

The library is built in-tree by ``python -m kshipra_amd.build``.  Nothing here
falls back to another implementation: a missing library, a tensor that is not
on a ROCm device or a non-OK status raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Dict, Tuple

import torch

from ._errors import QuantizationError

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libkshipra_quant.so")
ABI_VERSION = 103

KQ_OK, KQ_ERR_ARG, KQ_ERR_HIP, KQ_ERR_WORKSPACE = 0, 1, 2, 3
DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

# (name, restype, argtypes) of every symbol the header declares.
_i64, _vp, _int, _sz = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
SIGNATURES = [
    ("kq_version", _int, []),
    ("kq_last_error", ctypes.c_char_p, []),
    ("kq_check_finite", _int, [_vp, _int, _i64, _i64, _i64, _vp, _vp]),
    ("kq_quantize_int8", _int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    ("kq_quantize_int4", _int, [_vp, _int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    ("kq_dequantize_int8", _int, [_vp, _vp, _i64, _i64, _vp, _int, _vp]),
    ("kq_dequantize_int4", _int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _int, _vp]),
    ("kq_linear_workspace_bytes", _sz, [_int, _i64, _i64, _i64, _i64]),
    ("kq_linear_int8", _int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    ("kq_linear_int4", _int,
     [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    ("kq_linear_argmax_workspace_bytes", _sz, [_int, _i64, _i64, _i64, _i64]),
    ("kq_linear_argmax_int8", _int,
     [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    ("kq_linear_argmax_int4", _int,
     [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _sz, _vp]),
    ("kq_linear_silu_mul_workspace_bytes", _sz, [_int, _i64, _i64, _i64, _i64]),
    ("kq_linear_silu_mul_int8", _int,
     [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    ("kq_linear_silu_mul_int4", _int,
     [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _sz, _vp]),
    ("kq_paged_kv_write_f32", _int,
     [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    ("kq_chunked_attention_workspace_bytes", _sz, [_i64, _i64, _i64, _i64, _i64]),
    ("kq_chunked_attention_f32", _int,
     [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64,
      _i64, _vp, _i64, _i64, _vp, _sz, _vp]),
]

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load and type the library once; raise if it is absent or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"kshipra_amd: native library not built ({LIB_PATH}); "
                    "run `python -m kshipra_amd.build`")
            lib = ctypes.CDLL(LIB_PATH)
            for name, res, args in SIGNATURES:
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.kq_version() != ABI_VERSION:
                raise RuntimeError(
                    f"kshipra_amd: ABI version {lib.kq_version()} != expected {ABI_VERSION}")
            _lib = lib
    return _lib


def check(status: int) -> None:
    """Map a C status to the Python exception the reference would raise."""
    if status == KQ_OK:
        return
    msg = (load().kq_last_error() or b"").decode(errors="replace")
    if status == KQ_ERR_ARG:
        raise QuantizationError(msg)
    raise RuntimeError(f"kshipra_amd: {msg} (status {status})")


def require_device(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"kshipra_amd: {what} must be on a ROCm GPU (HIP device); got {t.device}. "
            "Move the model / weight to the GPU before quantizing.")


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


# Workspace buffers, one per (device, stream).  Calls on one stream are
# ordered, so reusing the buffer across them is safe.
_ws: Dict[Tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    if nbytes == 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    buf = _ws.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _ws[key] = buf
    return buf
