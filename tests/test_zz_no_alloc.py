"""kq_linear_int4_noalloc (the entry point without a workspace argument, for
callers that cannot allocate) against kq_linear_int4 with a torch-allocated
workspace, both called through the C ABI: the same kernels and plans, so the
outputs must agree bit for bit.  Two calls in a row, the second smaller
(the scratch keeps the first call's contents), then a call with no scratch
at all and a shape beyond the scratch, which must be refused before launch.
"""

from __future__ import annotations

import pytest
import torch

from cases import gaussian
from kshipra_amd import _lib
from kshipra_amd.quantization import quantize_int4_per_group

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20


def _with_workspace(lib, x, qw, b, y, n, k):
    m = x.shape[0]
    nbytes = lib.kq_linear_workspace_bytes(4, m, n, k, 128)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    _lib.check(lib.kq_linear_int4(x.data_ptr(), m, k, qw.payload.data_ptr(), qw.scales.data_ptr(),
                                  128, qw.in_features_padded, _lib.ptr(b), y.data_ptr(), n, n, k,
                                  ws.data_ptr(), nbytes, torch.cuda.current_stream().cuda_stream))
    return nbytes


def _no_alloc(lib, x, qw, b, y, n, k):
    m = x.shape[0]
    return lib.kq_linear_int4_noalloc(x.data_ptr(), m, k, qw.payload.data_ptr(), qw.scales.data_ptr(),
                                      128, qw.in_features_padded, _lib.ptr(b), y.data_ptr(), n, n, k,
                                      torch.cuda.current_stream().cuda_stream)


def test_no_alloc_matches_workspace_entry(gpu):
    lib = _lib.load()
    n, k = 4096, 14336                                   # down_proj of Llama-3-8B
    qw = quantize_int4_per_group(torch.from_numpy(gaussian((n, k), seed=91)).to(gpu), 128)
    b = torch.from_numpy(gaussian((n,), seed=92)).to(gpu)
    # M = 64: staged operand planes + split-K partials (~19.5 MiB of scratch);
    # then M = 8: a K-split skinny launch over the first call's leftovers;
    # then M = 1: no scratch used.
    for m in (64, 8, 1):
        x = torch.from_numpy(gaussian((m, k), seed=93 + m, std=1.0)).to(gpu)
        y_ref = torch.full((m, n), float("nan"), device=gpu)
        y = torch.full((m, n), float("nan"), device=gpu)
        need = _with_workspace(lib, x, qw, b, y_ref, n, k)
        assert need <= SCRATCH
        _lib.check(_no_alloc(lib, x, qw, b, y, n, k))
        torch.cuda.synchronize()
        print(f"[no-alloc m={m}] scratch {need} bytes", flush=True)
        assert torch.equal(y, y_ref), m
    # beyond the scratch: refused on the host, output untouched
    m = 512
    assert lib.kq_linear_workspace_bytes(4, m, n, k, 128) > SCRATCH
    x = torch.randn(m, k, device=gpu)
    y = torch.full((m, n), 7.0, device=gpu)
    status = _no_alloc(lib, x, qw, b, y, n, k)
    assert status == _lib.KQ_ERR_WORKSPACE
    assert b"scratch" in lib.kq_last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
