"""numpy fp32 decoder step for greedy-token parity (test infrastructure only).

Restates the op order of Kshipra ``engine/model.py:93-151`` (``KshipraModel.
forward``) and ``:153-205`` (``generate``: one prefill forward, then M=1
decode steps, first-index argmax each step):

    embed -> per layer [ RMSNorm -> q/k/v -> RoPE -> append K,V ->
    causal GQA attention -> o -> residual -> RMSNorm -> down(SiLU(gate)*up)
    -> residual ] -> final RMSNorm -> lm_head -> argmax

* RMSNorm is HF's LlamaRMSNorm (fp32 variance, ``x * rsqrt(var + eps) * w``).
* RoPE follows ``engine/model.py:35-55`` (``inv_freq = 1/theta^(2i/D)``,
  ``emb = cat(freqs, freqs)``, ``rotate_half``).
* Attention is softmax(q k^T / sqrt(D)) v over all cached positions <= the
  query's, kv head ``h // (H_q / H_kv)`` (``engine/chunked_prefill.py:104-140``
  computes the same with an online softmax over paged blocks).
* Projections use the oracle's exact dequantized fp32 weights and an fp32
  GEMM, as ``QuantizedLinear.forward`` does (``engine/quantization.py:394-396``).
  The lm_head is an unquantized fp32 linear (``engine/model.py:151``);
  ``lm_head_scheme`` quantizes it the same way for the quantized-lm_head
  extension (no counterpart in the reference, which keeps it fp32).

Weights are a plain dict (see ``DecoderConfig`` and ``layer_keys``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List

import numpy as np

from . import quant

PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass(frozen=True)
class DecoderConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rope_theta: float = 1000000.0
    rms_norm_eps: float = 1e-6
    qkv_bias: bool = True

    def proj_shape(self, name: str):
        h, i, d = self.hidden_size, self.intermediate_size, self.head_dim
        return {
            "q_proj": (self.num_heads * d, h),
            "k_proj": (self.num_kv_heads * d, h),
            "v_proj": (self.num_kv_heads * d, h),
            "o_proj": (h, self.num_heads * d),
            "gate_proj": (i, h),
            "up_proj": (i, h),
            "down_proj": (h, i),
        }[name]


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(np.float32)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    return (w * (x / np.sqrt(var + np.float32(eps)))).astype(np.float32)


def rope_cos_sin(head_dim: int, positions: np.ndarray, theta: float):
    """engine/model.py:35-44."""
    exps = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    inv_freq = (np.float32(1.0) / (np.float32(theta) ** exps)).astype(np.float32)
    freqs = positions.astype(np.float32)[:, None] * inv_freq[None, :]
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def expand_kv(kv: np.ndarray, g: int) -> np.ndarray:
    """GQA: query head h reads KV head h // g (engine/chunked_prefill.py:104-105)."""
    return np.repeat(kv, g, axis=0)


def future_mask(qpos: np.ndarray, s: int) -> np.ndarray:
    """True where key position > query position (causal, engine/chunked_prefill.py:122-126)."""
    return np.arange(s)[None, :] > qpos[:, None]


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """engine/model.py:30-32, 47-55.  x: [H, L, D]; cos/sin: [L, D]."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return (x * cos[None] + rot * sin[None]).astype(np.float32)


class OracleDecoder:
    """fp32 CPU restatement of the decoder, with its own KV cache."""

    def __init__(self, cfg: DecoderConfig, weights: Dict[str, np.ndarray], scheme: str,
                 group_size: int = 128, lm_head_scheme=None) -> None:
        self.cfg = cfg
        self.w = weights
        self.lm_head = weights["lm_head.weight"]
        if lm_head_scheme is not None:
            self.lm_head = quant.dequantize(quant.quantize(self.lm_head, lm_head_scheme, group_size))
        self.w_hat: List[Dict[str, np.ndarray]] = []
        for li in range(cfg.num_layers):
            d = {}
            for p in PROJ:
                qw = quant.quantize(weights[f"layers.{li}.{p}.weight"], scheme, group_size)
                d[p] = quant.dequantize(qw)
            self.w_hat.append(d)
        self.reset()

    def reset(self) -> None:
        self.k_cache = [None] * self.cfg.num_layers
        self.v_cache = [None] * self.cfg.num_layers
        self.pos = 0

    def _lin(self, li: int, name: str, x: np.ndarray) -> np.ndarray:
        b = self.w.get(f"layers.{li}.{name}.bias")
        return quant.linear_f32(x, self.w_hat[li][name], b).astype(np.float32)

    def forward(self, ids: List[int]) -> np.ndarray:
        """Logits [L, vocab] for the next L tokens; appends their K/V."""
        c = self.cfg
        L = len(ids)
        pos = np.arange(self.pos, self.pos + L)
        cos, sin = rope_cos_sin(c.head_dim, pos, c.rope_theta)
        h = self.w["embed_tokens.weight"][np.asarray(ids)].astype(np.float32)
        g = c.num_heads // c.num_kv_heads
        scale = np.float32(1.0 / np.sqrt(c.head_dim))
        for li in range(c.num_layers):
            res = h
            x = rms_norm(h, self.w[f"layers.{li}.input_layernorm.weight"], c.rms_norm_eps)
            q = self._lin(li, "q_proj", x).reshape(L, c.num_heads, c.head_dim).transpose(1, 0, 2)
            k = self._lin(li, "k_proj", x).reshape(L, c.num_kv_heads, c.head_dim).transpose(1, 0, 2)
            v = self._lin(li, "v_proj", x).reshape(L, c.num_kv_heads, c.head_dim).transpose(1, 0, 2)
            q = apply_rope(q, cos, sin)
            k = apply_rope(k, cos, sin)
            kc = k if self.k_cache[li] is None else np.concatenate([self.k_cache[li], k], axis=1)
            vc = v if self.v_cache[li] is None else np.concatenate([self.v_cache[li], v], axis=1)
            self.k_cache[li], self.v_cache[li] = kc, vc
            S = kc.shape[1]
            kq = expand_kv(kc, g)
            vq = expand_kv(vc, g)
            s = np.matmul(q, kq.transpose(0, 2, 1)) * scale                # [H, L, S]
            s = np.where(future_mask(pos, S), np.float32(-np.inf), s)
            s = s - s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p = p / p.sum(axis=-1, keepdims=True)
            a = np.matmul(p.astype(np.float32), vq).transpose(1, 0, 2).reshape(L, c.num_heads * c.head_dim)
            h = res + self._lin(li, "o_proj", a.astype(np.float32))
            res = h
            x = rms_norm(h, self.w[f"layers.{li}.post_attention_layernorm.weight"], c.rms_norm_eps)
            gt = self._lin(li, "gate_proj", x)
            up = self._lin(li, "up_proj", x)
            act = (gt / (np.float32(1.0) + np.exp(-gt))).astype(np.float32) * up
            h = res + self._lin(li, "down_proj", act.astype(np.float32))
        self.pos += L
        h = rms_norm(h, self.w["norm.weight"], c.rms_norm_eps)
        return quant.linear_f32(h, self.lm_head).astype(np.float32)

    def generate(self, prompt: List[int], max_new_tokens: int):
        """engine/model.py:153-205 greedy loop.  Returns (tokens, per-step logits)."""
        self.reset()
        logits = self.forward(prompt)[-1]
        toks, all_logits = [int(np.argmax(logits))], [logits]
        for _ in range(1, max_new_tokens):
            logits = self.forward([toks[-1]])[-1]
            toks.append(int(np.argmax(logits)))
            all_logits.append(logits)
        return toks, all_logits
