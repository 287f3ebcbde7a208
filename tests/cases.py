"""Seeded inputs shared by the CPU and GPU tests (generated on the CPU, so the
oracle and the HIP path see identical bytes)."""

from __future__ import annotations

from typing import Dict

import numpy as np
import torch


def adversarial_rows(rng: np.random.Generator, k: int) -> np.ndarray:
    """Rows that exercise every branch of the quantizer's arithmetic: exact .5
    ties (INT8 and INT4 scales that are powers of two), an all-zero row, a row
    whose fp16 scale underflows to 0 (w / 0 = +-inf -> clamp), subnormal fp16
    scales, the configs' N(0, 0.02), large values, a row whose fp16 scale
    overflows to inf, Student-t tails, and random fp32 bit patterns."""
    rows = []
    t8 = np.zeros(k, np.float32)
    t8[0] = 127 * 2.0 ** -7
    vals = (np.arange(1, k) % 127 + 0.5) * 2.0 ** -7
    t8[1:] = np.where(np.arange(1, k) % 2 == 0, vals, -vals)
    rows.append(t8)
    t4 = np.zeros(k, np.float32)
    t4[0] = 7 * 2.0 ** -5
    v4 = (np.arange(1, k) % 7 + 0.5) * 2.0 ** -5
    t4[1:] = np.where(np.arange(1, k) % 3 == 0, -v4, v4)
    rows.append(t4)
    rows.append(np.zeros(k, np.float32))
    rows.append((rng.standard_normal(k) * 1e-9).astype(np.float32))
    rows.append((rng.standard_normal(k) * 3e-6).astype(np.float32))
    rows.append((rng.standard_normal(k) * 1e-3).astype(np.float32))
    rows.append((rng.standard_normal(k) * 0.02).astype(np.float32))
    rows.append((rng.standard_normal(k) * 1e3).astype(np.float32))
    rows.append((rng.standard_normal(k) * 2e7).astype(np.float32))
    rows.append((rng.standard_t(3, k) * 0.2).astype(np.float32))
    bits = rng.integers(0, 2 ** 23, k, dtype=np.uint32) | (rng.integers(100, 140, k, dtype=np.uint32) << 23)
    bits |= rng.integers(0, 2, k, dtype=np.uint32) << 31
    rows.append(bits.view(np.float32))
    w = np.stack(rows)
    w[5, min(3, k - 1)] = -0.0
    return w


def gaussian(shape, seed: int, std: float = 0.02) -> np.ndarray:
    """``torch.manual_seed(seed); torch.randn(shape) * std`` as numpy fp32."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).numpy()


def with_outliers(w: np.ndarray, seed: int, frac: float = 1e-3, scale: float = 0.2) -> np.ndarray:
    """Replace round(frac * numel) uniformly chosen entries by Student-t(3) * scale."""
    rng = np.random.default_rng(seed)
    w = w.copy()
    n = int(round(frac * w.size))
    idx = rng.choice(w.size, size=n, replace=False)
    w.reshape(-1)[idx] = (rng.standard_t(3, n) * scale).astype(np.float32)
    return w


QWEN05B = dict(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_layers=24,
               num_heads=14, num_kv_heads=2, head_dim=64, rope_theta=1000000.0,
               rms_norm_eps=1e-6, qkv_bias=True)
LLAMA3_8B_SHAPES = {
    "q_proj": (4096, 4096), "k_proj": (1024, 4096), "v_proj": (1024, 4096), "o_proj": (4096, 4096),
    "gate_proj": (14336, 4096), "up_proj": (14336, 4096), "down_proj": (4096, 14336),
}


def decoder_weights(cfg: Dict, seed: int = 0) -> Dict[str, np.ndarray]:
    """Random-init decoder: every linear N(0, 0.02), biases N(0, 0.02) on q/k/v
    when ``qkv_bias``, RMSNorm weights 1, embeddings N(0, 0.02), lm_head tied to
    the embedding (as Qwen2.5-0.5B ties them)."""
    g = torch.Generator().manual_seed(seed)
    h, i, d = cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"]
    hq, hk = cfg["num_heads"], cfg["num_kv_heads"]
    shapes = {"q_proj": (hq * d, h), "k_proj": (hk * d, h), "v_proj": (hk * d, h),
              "o_proj": (h, hq * d), "gate_proj": (i, h), "up_proj": (i, h), "down_proj": (h, i)}
    w: Dict[str, np.ndarray] = {}
    w["embed_tokens.weight"] = (torch.randn(cfg["vocab_size"], h, generator=g) * 0.02).numpy()
    w["lm_head.weight"] = w["embed_tokens.weight"]
    w["norm.weight"] = np.ones(h, np.float32)
    for li in range(cfg["num_layers"]):
        w[f"layers.{li}.input_layernorm.weight"] = np.ones(h, np.float32)
        w[f"layers.{li}.post_attention_layernorm.weight"] = np.ones(h, np.float32)
        for p, shp in shapes.items():
            w[f"layers.{li}.{p}.weight"] = (torch.randn(*shp, generator=g) * 0.02).numpy()
        if cfg.get("qkv_bias", False):
            for p in ("q_proj", "k_proj", "v_proj"):
                w[f"layers.{li}.{p}.bias"] = (torch.randn(shapes[p][0], generator=g) * 0.02).numpy()
    return w
