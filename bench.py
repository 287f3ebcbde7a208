"""Benchmark of the weight-only quantized linear path on one MI355X.

Headline workload: one Llama-3-8B decode step at M = 1 through all 32 layers x
7 projections (q, k, v, o, gate, up, down) with INT4 G=128 weights, fp32
activations -- every projection a distinct weight (3.6 GB INT4 / 7.0 GB INT8
resident in HBM, far beyond the 256 MB MALL, so no repeat read is a cache hit).
As the decoder runs it, q/k/v and gate/up are each one dequant-GEMV launch over
their row-stacked weights (4 launches per layer, 128 per step); the step is
captured once in a HIP graph and replayed.  ``value`` is algorithmic bytes
(payload + scales + x + y) per step over the measured step time.

Also reported (same JSON line):
  * the same step with 7 separate launches per layer (224 per step);
  * INT8 per-channel M = 1 sweeps (same shapes);
  * per-projection GB/s (events around graphs of 32 same-shape launches);
  * skinny / tiled M = 4 / 8 / 32 / 64 sweeps (continuous-batching decode);
  * INT4 prefill-chunk GEMM TFLOP/s (X [512 x 4096] through gate/up
    [14336 x 4096], then [512 x 14336] through down);
  * lm_head [128256 x 4096] INT8 / INT4 at M = 1 and 32: the GEMV alone,
    followed by torch.argmax, and with the greedy argmax fused into it;
  * paged K/V chunked attention with Llama-3-8B heads over a 32-layer block
    pool: decode at 4096 / 16384 context (GB/s) and prefill chunks (TFLOP/s);
  * ``roofline``: the kernel that dominates the headline step (the fused
    gate/up dequant-GEMV, [28672 x 4096]) vs the 8 TB/s HBM peak, with its
    HBM traffic from the rocprofv3 counter summary under profiles/;
  * ``cpu_baseline``: the reference's CPU forward (torch materialises the
    fp32 weight, then F.linear; oracle/torch_ref.py) on this host with all
    available physical cores and with one thread, one row per config (large
    ones on a stated sample); ``value`` is the INT4 M = 1 Llama-3-8B layer.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--eager] [--quick]
                       [--only all|prefill|lm_head|attention|batch|cpu|m1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from kshipra_amd import _lib  # noqa: E402
from kshipra_amd.quantization import (concat_quantized, quantize_int4_per_group,  # noqa: E402
                                      quantize_int8_per_channel)

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE counter passes
# (calibrated against a 1 GiB device copy), written next to the profile summary.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "skinny_gemv_int4_llama3_8b_m1.json")
FP16_MFMA_PEAK_TFLOPS = 2500.0
LAYERS = 32
SHAPES = [("q_proj", 4096, 4096), ("k_proj", 1024, 4096), ("v_proj", 1024, 4096),
          ("o_proj", 4096, 4096), ("gate_proj", 14336, 4096), ("up_proj", 14336, 4096),
          ("down_proj", 4096, 14336)]
# q/k/v and gate/up row-stacked into one weight each: one launch per group.
FUSED = [("qkv", 6144, 4096), ("o_proj", 4096, 4096), ("gate_up", 28672, 4096),
         ("down_proj", 4096, 14336)]
# Qwen2.5-0.5B decoder (24 layers, hidden 896, intermediate 4864, 14 / 2 heads
# of 64): the small-model INT4 decode step, launch-bound by construction.
QWEN_LAYERS = 24
QWEN_SHAPES = [("q_proj", 896, 896), ("k_proj", 128, 896), ("v_proj", 128, 896),
               ("o_proj", 896, 896), ("gate_proj", 4864, 896), ("up_proj", 4864, 896),
               ("down_proj", 896, 4864)]
QWEN_FUSED = [("qkv", 1152, 896), ("o_proj", 896, 896), ("gate_up", 9728, 896),
              ("down_proj", 896, 4864)]


def algorithmic_bytes(m, n, k, scheme):
    """payload + scales + x (fp32) + y (fp32), each counted once."""
    w = n * k + 2 * n if scheme == "int8" else n * k // 2 + 2 * n * (k // 128)
    return w + 4 * m * k + 4 * m * n


class Proj:
    """One quantized projection with direct C-ABI launches (no Python per call
    beyond the ctypes call, so it can be captured into a graph)."""

    def __init__(self, qw, n, k, scheme):
        self.qw, self.n, self.k, self.scheme = qw, n, k, scheme
        self.lib = _lib.load()

    def launch(self, x, y, ws, ws_bytes, stream):
        m = x.shape[0]
        if self.scheme == "int8":
            st = self.lib.kq_linear_int8(x.data_ptr(), m, self.k, self.qw.payload.data_ptr(),
                                         self.qw.scales.data_ptr(), None, y.data_ptr(), self.n,
                                         self.n, self.k, ws, ws_bytes, stream)
        else:
            st = self.lib.kq_linear_int4(x.data_ptr(), m, self.k, self.qw.payload.data_ptr(),
                                         self.qw.scales.data_ptr(), 128, self.k, None,
                                         y.data_ptr(), self.n, self.n, self.k, ws, ws_bytes, stream)
        _lib.check(st)


def build_layers(scheme, dev, seed, nlayers=LAYERS, shapes=None):
    """``nlayers`` layers x 7 projections, N(0, 0.02) weights drawn on the GPU
    and quantized by the HIP kernel."""
    g = torch.Generator(device=dev).manual_seed(seed)
    layers = []
    for _ in range(nlayers):
        layer = {}
        for name, n, k in shapes or SHAPES:
            w = torch.randn(n, k, device=dev, generator=g) * 0.02
            qw = quantize_int8_per_channel(w) if scheme == "int8" else quantize_int4_per_group(w, 128)
            del w
            layer[name] = Proj(qw, n, k, scheme)
        for fname, parts in (("qkv", ("q_proj", "k_proj", "v_proj")), ("gate_up", ("gate_proj", "up_proj"))):
            fq = concat_quantized([layer[p].qw for p in parts])
            layer[fname] = Proj(fq, fq.original_shape[0], fq.original_shape[1], scheme)
        layers.append(layer)
    torch.cuda.synchronize()
    return layers


class Sweep:
    """All launches of one decode step at batch M, with preallocated buffers."""

    def __init__(self, layers, m, dev, names=None, shapes=None):
        self.names = names or [s[0] for s in SHAPES]
        shapes = {s[0]: s for s in (shapes or SHAPES + FUSED)}
        self.calls = []
        lib = _lib.load()
        ws_bytes = 0
        self.bytes = 0
        self.flops = 0
        for layer in layers:
            for name in self.names:
                _, n, k = shapes[name]
                p = layer[name]
                x = torch.randn(m, k, device=dev)
                y = torch.empty(m, n, device=dev)
                ws_bytes = max(ws_bytes, lib.kq_linear_workspace_bytes(
                    8 if p.scheme == "int8" else 4, m, n, k, 128))
                self.calls.append((p, x, y))
                self.bytes += algorithmic_bytes(m, n, k, p.scheme)
                self.flops += 2 * m * n * k
        self.ws_bytes = ws_bytes
        self.ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
        self.graph = None

    def run(self):
        stream = torch.cuda.current_stream().cuda_stream
        wsp = self.ws.data_ptr() if self.ws_bytes else None
        for p, x, y in self.calls:
            p.launch(x, y, wsp, self.ws_bytes, stream)

    def capture(self):
        self.run()                                   # warm the launch path outside capture
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self.run()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = g

    def step(self):
        if self.graph is not None:
            self.graph.replay()
        else:
            self.run()


def time_steps(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps            # ms per step


def measure(layers, m, dev, steps, warmup, eager, names=None, shapes=None):
    sw = Sweep(layers, m, dev, names, shapes)
    if not eager:
        sw.capture()
    ms = time_steps(sw.step, steps, warmup)
    return {"ms": ms, "bytes": sw.bytes, "flops": sw.flops,
            "gbs": sw.bytes / (ms * 1e-3) / 1e9, "tflops": sw.flops / (ms * 1e-3) / 1e12}


def batch_steps(int8, int4, dev, steps, warmup, eager, ms):
    """Continuous-batching decode steps at batch M: the 7 projections as
    separate launches (``int8_m{M}``), and as the decoder runs them with
    q/k/v and gate/up row-stacked (4 launches per layer, ``*_fused``)."""
    out = {}
    for m in ms:
        for scheme, layers in (("int8", int8), ("int4", int4)):
            r = measure(layers, m, dev, steps, warmup, eager)
            out[f"{scheme}_m{m}"] = {"gbs": round(r["gbs"], 1), "tflops": round(r["tflops"], 1),
                                     "us_per_step": round(r["ms"] * 1e3, 1)}
            r = measure(layers, m, dev, steps, warmup, eager, names=[f[0] for f in FUSED])
            out[f"{scheme}_m{m}_fused"] = {"gbs": round(r["gbs"], 1), "tflops": round(r["tflops"], 1),
                                           "us_per_step": round(r["ms"] * 1e3, 1)}
    return out


def prefill_tflops(dev, steps, warmup, eager, scheme="int4"):
    """Config: INT4 G=128 (or INT8) prefill chunk through one Llama-3-8B MLP."""
    g = torch.Generator(device=dev).manual_seed(7)
    qf = (lambda w: quantize_int4_per_group(w, 128)) if scheme == "int4" else quantize_int8_per_channel
    mk = lambda n, k: Proj(qf(torch.randn(n, k, device=dev, generator=g) * 0.02), n, k, scheme)
    gate, up, down = mk(14336, 4096), mk(14336, 4096), mk(4096, 14336)
    lib = _lib.load()
    x = torch.randn(512, 4096, device=dev)
    a = torch.randn(512, 14336, device=dev)
    yg, yu, yd = (torch.empty(512, 14336, device=dev), torch.empty(512, 14336, device=dev),
                  torch.empty(512, 4096, device=dev))
    bits = 4 if scheme == "int4" else 8
    wsb = max(lib.kq_linear_workspace_bytes(bits, 512, 14336, 4096, 128),
              lib.kq_linear_workspace_bytes(bits, 512, 4096, 14336, 128))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)

    def run():
        st = torch.cuda.current_stream().cuda_stream
        gate.launch(x, yg, ws.data_ptr(), wsb, st)
        up.launch(x, yu, ws.data_ptr(), wsb, st)
        down.launch(a, yd, ws.data_ptr(), wsb, st)

    fn = run
    if not eager:
        run()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                run()
        torch.cuda.current_stream().wait_stream(s)
        fn = graph.replay
    ms = time_steps(fn, steps, warmup)
    flops = 3 * 2 * 512 * 14336 * 4096
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "gflop": flops / 1e9}


def graph_or_eager(run, eager):
    if eager:
        return run
    run()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            run()
    torch.cuda.current_stream().wait_stream(s)
    return graph.replay


def lm_head(dev, steps, warmup, eager):
    """Vocab projection [128256 x 4096] (INT8 and INT4 G=128) at M = 1 and 32,
    then the greedy argmax over each row's logits."""
    vocab, hidden = 128256, 4096
    lib = _lib.load()
    g = torch.Generator(device=dev).manual_seed(11)
    w = torch.randn(vocab, hidden, device=dev, generator=g) * 0.02
    out = {}
    for scheme in ("int8", "int4"):
        qw = quantize_int8_per_channel(w) if scheme == "int8" else quantize_int4_per_group(w, 128)
        p = Proj(qw, vocab, hidden, scheme)
        for m in (1, 32):
            x = torch.randn(m, hidden, device=dev)
            y = torch.empty(m, vocab, device=dev)
            wsb = lib.kq_linear_workspace_bytes(8 if scheme == "int8" else 4, m, vocab, hidden, 128)
            ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)
            tok = torch.empty(m, dtype=torch.int64, device=dev)
            awsb = lib.kq_linear_argmax_workspace_bytes(8 if scheme == "int8" else 4, m, vocab, hidden, 128)
            aws = torch.empty(awsb, dtype=torch.uint8, device=dev)

            def fused_argmax():
                st = torch.cuda.current_stream().cuda_stream
                if scheme == "int8":
                    r = lib.kq_linear_argmax_int8(x.data_ptr(), m, hidden, qw.payload.data_ptr(),
                                                  qw.scales.data_ptr(), None, None, 0, vocab, hidden,
                                                  tok.data_ptr(), aws.data_ptr(), awsb, st)
                else:
                    r = lib.kq_linear_argmax_int4(x.data_ptr(), m, hidden, qw.payload.data_ptr(),
                                                  qw.scales.data_ptr(), 128, hidden, None, None, 0,
                                                  vocab, hidden, tok.data_ptr(), aws.data_ptr(), awsb, st)
                _lib.check(r)

            def gemv():
                p.launch(x, y, ws.data_ptr() if wsb else None, wsb,
                         torch.cuda.current_stream().cuda_stream)

            def gemv_argmax():
                gemv()
                torch.argmax(y, dim=-1, out=tok)

            # Per call as the decoder issues it: LM_HEAD_REPS back-to-back calls
            # per HIP graph (like the per-projection sweep's 32), each
            # streaming the whole 263-525 MB weight from HBM (beyond the
            # 256 MB MALL); one call per graph replay is reported beside it
            # (it adds the gap between graph launches).
            def reps(fn):
                def run():
                    for _ in range(LM_HEAD_REPS):
                        fn()
                return run
            ms = time_steps(graph_or_eager(reps(gemv), eager), steps, warmup) / LM_HEAD_REPS
            ms_tok = time_steps(graph_or_eager(reps(gemv_argmax), eager), steps, warmup) / LM_HEAD_REPS
            ms_fused = time_steps(graph_or_eager(reps(fused_argmax), eager), steps, warmup) / LM_HEAD_REPS
            ms_one = time_steps(graph_or_eager(gemv, eager), steps, warmup)
            nbytes = algorithmic_bytes(m, vocab, hidden, scheme)
            out[f"{scheme}_m{m}"] = {"gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                     "us_gemv": round(ms * 1e3, 2),
                                     "us_gemv_then_torch_argmax": round(ms_tok * 1e3, 2),
                                     "us_fused_argmax": round(ms_fused * 1e3, 2),
                                     "us_gemv_one_call_per_graph": round(ms_one * 1e3, 2),
                                     "bytes": nbytes}
        del qw, p
    del w
    torch.cuda.synchronize()
    return out


FP32_MFMA_PEAK_TFLOPS = 157.3
LM_HEAD_REPS = 8


def attention(dev, steps, warmup, eager):
    """Paged K/V attention with Llama-3-8B heads (32 query / 8 KV heads, D = 128)
    over a 32-layer block pool [blocks, 32, 2, 8, 64, 128] fp32: one
    chunked_attention call per layer (graph of 32), each layer's K / V distinct
    in HBM.  Decode (1 query) reports K/V GB/s; prefill chunks report TFLOP/s
    (4 * H_q * D * visible (query, key) pairs)."""
    from kshipra_amd.attention import chunked_attention
    hq, hkv, d, b, layers = 32, 8, 128, 64, 32
    out = {}
    for name, c, p in (("decode_ctx4096", 1, 4095), ("decode_ctx16384", 1, 16383),
                       ("prefill_chunk512_after3584", 512, 3584), ("prefill_chunk2048", 2048, 0)):
        nb = (p + c + b - 1) // b
        pool = torch.randn((nb, layers, 2, hkv, b, d), device=dev)
        q = torch.randn((layers, hq, c, d), device=dev)
        o = torch.empty((layers, hq, c, d), device=dev)
        table = torch.arange(nb, dtype=torch.int32, device=dev)

        def run():
            for li in range(layers):
                chunked_attention(q[li], pool[:, li, 0], pool[:, li, 1], table, p, c, b, out=o[li])

        ms = time_steps(graph_or_eager(run, eager), steps, warmup) / layers
        kv_bytes = 2 * hkv * (p + c) * d * 4 + 2 * hq * c * d * 4
        flops = 4 * hq * d * (c * p + c * (c + 1) // 2)
        r = {"us_per_layer": round(ms * 1e3, 2), "gbs": round(kv_bytes / (ms * 1e-3) / 1e9, 1),
             "tflops": round(flops / (ms * 1e-3) / 1e12, 2)}
        if c == 1:
            r["frac_of_hbm_peak"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
        else:
            r["frac_of_fp32_mfma_peak"] = round(r["tflops"] / FP32_MFMA_PEAK_TFLOPS, 4)
        out[name] = r
        del pool, q, o
        torch.cuda.empty_cache()
    return out


def _host_info():
    """CPU model, logical CPUs, the CPUs this process may run on and how many
    distinct physical cores those are (from the sysfs topology)."""
    info = {"os_cpu_count": os.cpu_count()}
    try:
        cpus = sorted(os.sched_getaffinity(0))
    except AttributeError:
        cpus = list(range(os.cpu_count() or 1))
    info["affinity_cpus"] = len(cpus)
    cores = set()
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            pkg = open(base + "physical_package_id").read().strip()
            core = open(base + "core_id").read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", str(c)))
    info["physical_cores"] = len(cores)
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                info["model"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return info


def _time_cpu(fn, budget_s, max_iter=5, warmup=1):
    """Median wall time (s) of fn() after warm-up, at most max_iter runs and
    roughly budget_s seconds."""
    for _ in range(warmup):
        fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < max_iter and (not times or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline(dev, budget_s=40.0):
    """The reference's CPU forward (oracle/torch_ref.py: torch materialises the
    fp32 weight, then F.linear; engine/quantization.py:226-230, 321-344,
    394-396) on this host, for each BASELINE config, with all available
    physical cores and with one thread (the reference harness's setting,
    benchmarks/run_benchmarks.py:63,123).  Weights are quantized on the GPU
    (bit-identical to the reference quantizer) and copied to host memory.
    Large configs are timed on a stated sample (a number of layers or a row
    slice of the weight) and reported as rates of that sample."""
    import torch.nn.functional as F

    from oracle import torch_ref
    host = _host_info()
    threads_all = max(1, host["physical_cores"])
    g = torch.Generator(device=dev).manual_seed(21)

    def q_host(n, k, scheme):
        w = torch.randn(n, k, device=dev, generator=g) * 0.02
        qw = quantize_int8_per_channel(w) if scheme == "int8" else quantize_int4_per_group(w, 128)
        return qw.payload.cpu(), qw.scales.cpu()

    rows = []
    per_row_budget = budget_s / 12

    def run(config, sample, projs, m, scheme, scale_rows=1.0, gflop=None):
        """projs: [(payload, scales, n, k)] on the host; times one pass over them."""
        xs = {k: torch.randn(m, k) for (_, _, _, k) in projs}
        nbytes = sum(algorithmic_bytes(m, n, k, scheme) for (_, _, n, k) in projs)

        def one():
            for payload, scales, n, k in projs:
                torch_ref.linear(xs[k], payload, scales, scheme, k)
        for threads in (threads_all, 1):
            torch.set_num_threads(threads)
            t, it = _time_cpu(one, per_row_budget, max_iter=5 if threads > 1 else 3)
            # rates over the sample (a row slice or a few layers runs at the
            # rate of the whole); ms_full scales the sample's time up
            r = {"config": config, "sample": sample, "threads": threads, "ms": round(t * 1e3, 2),
                 "ms_full": round(t * 1e3 * scale_rows, 2), "iters": it,
                 "gbs": round(nbytes / t / 1e9, 3)}
            if gflop is not None:
                r["tflops"] = round(gflop / t / 1e3, 4)
            rows.append(r)
            print(f"# cpu {config} {threads} threads: {t * 1e3:.1f} ms", file=sys.stderr, flush=True)

    # 1. INT8 [4864 x 896] dequant-matvec
    p, sc = q_host(4864, 896, "int8")
    run("int8_4864x896_m1", "the whole config", [(p, sc, 4864, 896)], 1, "int8")
    # 2. INT4 Qwen2.5-0.5B decode step: 2 of 24 layers (7 projections each)
    qw = [q_host(n, k, "int4") + (n, k) for _ in range(2) for _, n, k in QWEN_SHAPES]
    run("int4_qwen2.5_0.5b_step_m1", "2 of 24 layers", qw, 1, "int4", scale_rows=12.0)
    # headline workload: INT4 Llama-3-8B decode step at M = 1, one layer
    l4 = [q_host(n, k, "int4") + (n, k) for _, n, k in SHAPES]
    run("int4_llama3_8b_step_m1", "1 of 32 layers (7 projections)", l4, 1, "int4", scale_rows=32.0)
    del l4
    # 3. INT8 Llama-3-8B layer at M = 1 / 8 / 32 / 64
    l8 = [q_host(n, k, "int8") + (n, k) for _, n, k in SHAPES]
    for m in (1, 8, 32, 64):
        run(f"int8_llama3_8b_layer_m{m}", "one layer (7 projections)", l8, m, "int8",
            gflop=2 * m * sum(n * k for _, _, n, k in l8) / 1e9)
    del l8
    # 4. INT4 prefill MLP, M = 512: gate and up [14336 x 4096], down [4096 x
    #    14336] -- a quarter of each weight's rows (the work is row-separable)
    mlp = []
    for n, k in ((14336, 4096), (14336, 4096), (4096, 14336)):
        pp, ss = q_host(n, k, "int4")
        mlp.append((pp[: n // 4].contiguous(), ss[: n // 4].contiguous(), n // 4, k))
    run("int4_prefill_mlp_m512", "a quarter of each weight's rows",
        mlp, 512, "int4", scale_rows=4.0, gflop=2 * 512 * sum(n * k for _, _, n, k in mlp) / 1e9)
    del mlp
    # 5. lm_head [128256 x 4096] INT8 / INT4 at M = 1: an eighth of the vocab
    for scheme in ("int8", "int4"):
        pp, ss = q_host(128256, 4096, scheme)
        part = [(pp[:16032].contiguous(), ss[:16032].contiguous(), 16032, 4096)]
        del pp, ss
        run(f"lm_head_{scheme}_m1", "an eighth of the vocabulary rows", part, 1, scheme,
            scale_rows=8.0)
    torch.set_num_threads(threads_all)
    head = next(r for r in rows if r["config"] == "int4_llama3_8b_step_m1" and r["threads"] == threads_all)
    head1 = next(r for r in rows if r["config"] == "int4_llama3_8b_step_m1" and r["threads"] == 1)
    return {"value": head["gbs"], "unit": "GB/s", "cores": threads_all, "kind": "port",
            "sample": (f"the reference's CPU forward (torch dequantize + F.linear, oracle/torch_ref.py) "
                       f"over one Llama-3-8B layer (7 INT4 G=128 projections, M=1), {head['ms']} ms "
                       f"with {threads_all} threads ({head1['ms']} ms with 1); every BASELINE config "
                       f"is in rows"),
            "host": host, "rows": rows}


def hbm_copy_reference(dev):
    """A plain 1 GiB device-to-device copy: the reference dispatch that scales
    the FETCH_SIZE / WRITE_SIZE counters of the same run to HBM bytes."""
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--eager", action="store_true", help="launch without HIP graphs (for counters)")
    ap.add_argument("--quick", action="store_true", help="headline only (no extras, no CPU baseline)")
    ap.add_argument("--layers", type=int, default=LAYERS,
                    help="layers in the sweep (fewer only for counter runs; the headline uses 32)")
    ap.add_argument("--only", choices=("all", "prefill", "lm_head", "attention", "batch", "cpu", "m1"), default="all",
                    help="profiling aid: run one section and print its figures only")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: the quantized-linear path runs on a single GPU "
              f"here (--gpus {args.gpus} requested); no multi-GPU figure is produced",
              file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    t_all = time.time()
    if args.only != "all":
        if args.only == "prefill":
            for scheme in ("int4", "int8"):
                pf = prefill_tflops(dev, args.steps, args.warmup, args.eager, scheme)
                print(json.dumps({"section": f"{scheme}_prefill_m512_mlp", "tflops": round(pf["tflops"], 1),
                                  "ms": round(pf["ms"], 4), "gflop": round(pf["gflop"], 1),
                                  "frac_of_fp16_mfma_peak": round(pf["tflops"] / FP16_MFMA_PEAK_TFLOPS, 4)}))
        elif args.only == "m1":
            # M = 1 per projection, INT4 and INT8 (counter runs)
            res = {}
            for scheme, seed in (("int4", 1), ("int8", 2)):
                layers = build_layers(scheme, dev, seed=seed, nlayers=args.layers)
                for name, n, k in SHAPES + [f for f in FUSED if f[0] in ("qkv", "gate_up")]:
                    r = measure(layers, 1, dev, args.steps, args.warmup, args.eager, names=[name])
                    res[f"{scheme}_{name}"] = {"gbs": round(r["gbs"], 1),
                                               "us_per_launch": round(r["ms"] * 1e3 / args.layers, 2)}
                del layers
                torch.cuda.empty_cache()
            hbm_copy_reference(dev)
            print(json.dumps({"section": "m1_per_projection", "results": res}))
        elif args.only == "cpu":
            print(json.dumps({"section": "cpu_baseline", "results": cpu_baseline(dev)}))
        elif args.only == "attention":
            print(json.dumps({"section": "attention_llama3_8b_heads",
                              "results": attention(dev, args.steps, args.warmup, args.eager)}))
        elif args.only == "batch":
            # decode batches: the 7-projection and the fused 4-launch step at M = 8, 32, 64
            int8 = build_layers("int8", dev, seed=2, nlayers=args.layers)
            int4 = build_layers("int4", dev, seed=1, nlayers=args.layers)
            res = batch_steps(int8, int4, dev, args.steps, args.warmup, args.eager, (8, 32, 64))
            print(json.dumps({"section": "decode_batches_llama3_8b", "results": res}))
        else:
            print(json.dumps({"section": "lm_head_128256x4096",
                              "results": lm_head(dev, args.steps, args.warmup, args.eager)}))
        return

    nl = args.layers
    int4 = build_layers("int4", dev, seed=1, nlayers=nl)
    # Headline: the decode step as the framework runs it, q/k/v and gate/up
    # each one launch over their row-stacked weights (same bytes and outputs
    # as the 7 separate projections, 4 launches per layer instead of 7).
    head = measure(int4, 1, dev, args.steps, args.warmup, args.eager, names=[f[0] for f in FUSED])
    print(f"# int4 M=1 fused sweep: {head['ms'] * 1e3:.1f} us/step, {head['gbs']:.0f} GB/s",
          file=sys.stderr, flush=True)
    sep = measure(int4, 1, dev, args.steps, args.warmup, args.eager)
    breakdown = {"int4_m1_fused_qkv_gateup": {"gbs": round(head["gbs"], 1), "us_per_step": round(head["ms"] * 1e3, 1)},
                 "int4_m1_separate_projections": {"gbs": round(sep["gbs"], 1), "us_per_step": round(sep["ms"] * 1e3, 1)}}
    per_proj = {}
    for name, n, k in SHAPES + [f for f in FUSED if f[0] in ("qkv", "gate_up")]:   # 32 same-shape launches per graph
        r = measure(int4, 1, dev, args.steps, args.warmup, args.eager, names=[name])
        per_proj[name] = {"gbs": round(r["gbs"], 1), "us_per_launch": round(r["ms"] * 1e3 / nl, 2),
                          "bytes_per_launch": r["bytes"] // nl}
    breakdown["int4_m1_per_projection"] = per_proj
    # Roofline: the kernel that dominates the headline step's time.
    dom = "gate_up"
    dom_bytes = per_proj[dom]["bytes_per_launch"]
    dom_us = per_proj[dom]["us_per_launch"]
    achieved = dom_bytes / (dom_us * 1e-6) / 1e9
    traffic, traffic_src = None, None
    if os.path.exists(TRAFFIC_FILE):
        tf = json.load(open(TRAFFIC_FILE))
        traffic = tf.get("hbm_bytes_per_launch", {}).get(dom)
        traffic_src = tf.get("source") if traffic is not None else None

    cpu = None
    if not args.quick:
        int8 = build_layers("int8", dev, seed=2, nlayers=nl)
        fz8 = measure(int8, 1, dev, args.steps, args.warmup, args.eager, names=[f[0] for f in FUSED])
        breakdown["int8_m1_fused_qkv_gateup"] = {"gbs": round(fz8["gbs"], 1),
                                                 "us_per_step": round(fz8["ms"] * 1e3, 1)}
        r8 = measure(int8, 1, dev, args.steps, args.warmup, args.eager)
        breakdown["int8_m1_separate_projections"] = {"gbs": round(r8["gbs"], 1), "us_per_step": round(r8["ms"] * 1e3, 1)}
        per8 = {}
        for name, n, k in SHAPES + [f for f in FUSED if f[0] in ("qkv", "gate_up")]:
            r = measure(int8, 1, dev, args.steps, args.warmup, args.eager, names=[name])
            per8[name] = {"gbs": round(r["gbs"], 1), "us_per_launch": round(r["ms"] * 1e3 / nl, 2)}
        breakdown["int8_m1_per_projection"] = per8
        qwen = build_layers("int4", dev, seed=5, nlayers=QWEN_LAYERS, shapes=QWEN_SHAPES)
        rq = measure(qwen, 1, dev, args.steps, args.warmup, args.eager,
                     names=[f[0] for f in QWEN_FUSED], shapes=QWEN_SHAPES + QWEN_FUSED)
        breakdown["int4_m1_qwen2.5_0.5b_fused_step"] = {
            "gbs": round(rq["gbs"], 1), "us_per_step": round(rq["ms"] * 1e3, 1),
            "bytes_per_step": rq["bytes"], "launches": 4 * QWEN_LAYERS}
        del qwen
        breakdown.update(batch_steps(int8, int4, dev, max(args.steps // 2, 3), 1, args.eager, (4, 8, 32, 64)))
        del int8
        torch.cuda.empty_cache()
        pf = prefill_tflops(dev, max(args.steps // 2, 3), 1, args.eager)
        breakdown["int4_prefill_m512_mlp"] = {"tflops": round(pf["tflops"], 1), "ms": round(pf["ms"], 3),
                                              "gflop": round(pf["gflop"], 1),
                                              "frac_of_fp16_mfma_peak": round(pf["tflops"] / FP16_MFMA_PEAK_TFLOPS, 4)}
        pf8 = prefill_tflops(dev, max(args.steps // 2, 3), 1, args.eager, "int8")
        breakdown["int8_prefill_m512_mlp"] = {"tflops": round(pf8["tflops"], 1), "ms": round(pf8["ms"], 3),
                                              "gflop": round(pf8["gflop"], 1),
                                              "frac_of_fp16_mfma_peak": round(pf8["tflops"] / FP16_MFMA_PEAK_TFLOPS, 4)}
        breakdown["lm_head_128256x4096"] = lm_head(dev, args.steps, args.warmup, args.eager)
        breakdown["attention_llama3_8b_heads"] = attention(dev, max(args.steps // 2, 3), 1, args.eager)
        cpu = cpu_baseline(dev)

    hbm_copy_reference(dev)

    out = {
        "metric": "dequant-GEMV HBM GB/s (% of peak) at M=1 INT4/INT8; prefill GEMM TFLOPS",
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xf32",
        "data": "synthetic: N(0, 0.02) weights drawn on the GPU and quantized by the HIP kernel; x ~ N(0, 1)",
        "config": {"workload": "Llama-3-8B decode step at M=1: 32 layers x (q,k,v,o,gate,up,down) "
                               "INT4 G=128 dequant-GEMV, fp32 activations, q/k/v and gate/up each "
                               "one launch over row-stacked weights (4 launches per layer), one "
                               "HIP graph per step",
                   "layers": nl, "batch_m": 1, "scheme": "int4_per_group_g128",
                   "launch": "eager" if args.eager else "hip_graph",
                   "bytes_per_step": head["bytes"], "parallelism": "single_gpu"},
        "frac_of_hbm_peak": round(head["gbs"] / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": f"skinny dequant-GEMV INT4 ({dom} [28672x4096], M=1)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "bytes_per_launch": dom_bytes, "us_per_launch": dom_us},
        "cpu_baseline": cpu,
        "breakdown": breakdown,
        "wall_s": round(time.time() - t_all, 1),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
