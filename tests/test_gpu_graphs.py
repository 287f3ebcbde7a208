"""HIP-graph capture of the library's launches, replayed several times.

One graph holds a K-split skinny launch (partials + ordered reduction in the
workspace), a tiled GEMM launch (operand staging + split-K reduction), the
paged K/V write, a split-key decode attention (+ combine) and a shared-tile
prefill attention.  The graph is replayed three times with eager work on the
same stream in between (which reuses the workspace and rewrites the inputs),
and every replay must reproduce the eager results bit for bit: the kernels
are deterministic (fixed reduction orders) and record no memset.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import gaussian
from kshipra_amd.attention import chunked_attention, paged_kv_write
from kshipra_amd.quantization import (quantize_int4_per_group, quantize_int8_per_channel,
                                      quantized_linear)

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(gpu):
    torch.manual_seed(0)
    w_down = torch.from_numpy(gaussian((4096, 14336), seed=1)).to(gpu)
    w_gate = torch.from_numpy(gaussian((1024, 4096), seed=2)).to(gpu)
    q_down = quantize_int8_per_channel(w_down)          # M = 8, K = 14336: K-split skinny
    q_gate = quantize_int4_per_group(w_gate, 128)        # M = 24: tiled GEMM
    del w_down, w_gate
    x8 = torch.randn(8, 14336, device=gpu)
    x24 = torch.randn(24, 4096, device=gpu)
    b8 = torch.randn(4096, device=gpu)

    hq, hkv, d, blk = 32, 8, 128, 64
    nb = 40
    pool = torch.randn((nb, 1, 2, hkv, blk, d), device=gpu)
    table = torch.randperm(nb, device=gpu)[:36].to(torch.int32).contiguous()
    k_new = torch.randn((hkv, 1, d), device=gpu)
    v_new = torch.randn((hkv, 1, d), device=gpu)
    pos = 2000                                           # decode position: 2000 keys before it
    slot = torch.tensor([int(table[pos // blk]) * blk + pos % blk], dtype=torch.int64, device=gpu)
    q_dec = torch.randn((hq, 1, d), device=gpu)
    q_pre = torch.randn((hq, 512, d), device=gpu)        # 512-token chunk after 1000 keys

    outs = {}

    def step():
        outs["down"] = quantized_linear(x8, q_down, b8)
        outs["gate"] = quantized_linear(x24, q_gate)
        paged_kv_write(pool, 0, k_new, v_new, slot)
        outs["dec"] = chunked_attention(q_dec, pool[:, 0, 0], pool[:, 0, 1], table, pos, 1, blk)
        outs["pre"] = chunked_attention(q_pre, pool[:, 0, 0], pool[:, 0, 1], table, 1000, 512, blk)

    with torch.inference_mode():
        step()
        torch.cuda.synchronize()
        eager = {k: v.clone() for k, v in outs.items()}
        pool_eager = pool.clone()

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            step()                                       # warm the workspace on this stream
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=s):
                step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()

        for rep in range(3):
            # eager work between replays: other shapes through the same library
            # (its workspace is reused), then the inputs are restored
            quantized_linear(torch.randn(3, 14336, device=gpu), q_down)
            chunked_attention(torch.randn((hq, 1, d), device=gpu), pool[:, 0, 0], pool[:, 0, 1], table,
                              100, 1, blk)
            for v in outs.values():
                v.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            print(f"[graph replay {rep}]", flush=True)
            for name, ref in eager.items():
                assert torch.equal(outs[name], ref), (rep, name)
            assert torch.equal(pool, pool_eager), rep


def test_captured_workspace_survives_eager_growth(gpu):
    """A graph keeps the workspace address its launches were recorded with.
    After capture, an eager call on the same stream that needs a larger
    workspace and a fresh allocation filled with a pattern must neither
    change the replayed result nor be overwritten by the replay."""
    w = torch.from_numpy(gaussian((4096, 14336), seed=3)).to(gpu)
    q = quantize_int8_per_channel(w)                     # M = 8: K-split skinny (partials)
    del w
    x8 = torch.randn(8, 14336, device=gpu)
    x16 = torch.randn(16, 14336, device=gpu)             # 16 slices of 16 rows: larger workspace
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.stream(s):
        ref = quantized_linear(x8, q).clone()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            out = quantized_linear(x8, q)
        torch.cuda.synchronize()
        for rep in range(3):
            big = quantized_linear(x16, q)               # same stream, larger workspace
            filler = torch.full((8 << 20,), 7.0, device=gpu)
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            print(f"[graph workspace replay {rep}]", flush=True)
            assert torch.equal(out, ref), rep
            assert bool((filler == 7.0).all()), rep
            assert torch.isfinite(big).all()
            del big, filler
