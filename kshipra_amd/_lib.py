"""ctypes binding of ``libkshipra_quant.so`` (declared in ``include/kshipra_quant.h``).

The library is built in-tree by ``python -m kshipra_amd.build``.  Nothing here
falls back to another implementation: a missing library, a tensor that is not
on a ROCm device or a non-OK status raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Dict, List, Optional, Tuple

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
    ("kq_linear_int4_noalloc", _int,
     [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _i64, _i64, _i64, _vp]),
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


# Workspace buffers.
#
# Eager calls: one buffer per (device, stream).  Calls on one stream are
# ordered, so they can share it; when a call needs more, the buffer is
# replaced and the old one returns to torch's caching allocator, whose reuse
# of it is ordered on the same stream.
#
# Calls recorded into a HIP graph bake the buffer's address into the graph's
# kernel nodes, and a replay writes there long after the call returned.  Such
# calls therefore get buffers of their own, keyed by (device, stream, capture
# id): shared only by calls of the same capture (ordered on its stream), never
# by eager calls or other graphs, and never freed -- a buffer superseded
# inside a capture is retired, not released -- until
# ``release_graph_workspaces()`` is called once those graphs are gone.
_ws: Dict[Tuple[int, int], torch.Tensor] = {}
_graph_ws: Dict[Tuple[int, int, int], torch.Tensor] = {}
_graph_retired: List[torch.Tensor] = []
_MIN_WS = 1 << 20


def _alloc(device: torch.device, nbytes: int) -> torch.Tensor:
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


_hip = None


def _capture_id(stream: int) -> Optional[int]:
    """The id of the HIP graph capture ``stream`` is recording, or None."""
    global _hip
    if not torch.cuda.is_current_stream_capturing():
        return None
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipStreamGetCaptureInfo.restype = ctypes.c_int
        _hip.hipStreamGetCaptureInfo.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int),
                                                 ctypes.POINTER(ctypes.c_ulonglong)]
    status, cid = ctypes.c_int(0), ctypes.c_ulonglong(0)
    err = _hip.hipStreamGetCaptureInfo(ctypes.c_void_p(stream), ctypes.byref(status),
                                       ctypes.byref(cid))
    if err != 0:
        raise RuntimeError(f"kshipra_amd: hipStreamGetCaptureInfo failed ({err})")
    return int(cid.value)


def workspace(device: torch.device, stream: int, nbytes: int) -> Optional[torch.Tensor]:
    if nbytes == 0:
        return None
    dev = device.index if device.index is not None else torch.cuda.current_device()
    cid = _capture_id(stream)
    if cid is None:
        key = (dev, stream)
        buf = _ws.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = _alloc(device, max(nbytes, _MIN_WS))
            _ws[key] = buf
        return buf
    gkey = (dev, stream, cid)
    buf = _graph_ws.get(gkey)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _graph_retired.append(buf)        # captured kernels still point into it
        buf = _alloc(device, max(nbytes, _MIN_WS))
        _graph_ws[gkey] = buf
    return buf


def release_graph_workspaces() -> None:
    """Free every workspace handed to calls made under HIP graph capture.
    Only safe once no graph that captured a call of this library will be
    replayed again."""
    _graph_ws.clear()
    _graph_retired.clear()
