"""Caller side of the quantized-linear path: the projection swap and a greedy
decoder that runs every projection through ``QuantizedLinear`` on the GPU.

* ``quantize_all_linears(hf_model, scheme)`` -- Kshipra ``engine/model.py:80-91``:
  swaps q/k/v/o and gate/up/down of every decoder layer of a HuggingFace
  Llama / Qwen2 model for ``QuantizedLinear`` (always ``group_size=128``);
  embeddings and lm_head stay unquantized.  Move the model to the GPU first
  (``engine/model.py:67``): the quantized payload is created on the weight's
  device.
* ``DecoderLM`` -- a decoder-only LM over a plain weight dict with the op order
  of ``KshipraModel.forward`` (``engine/model.py:93-151``) and the greedy loop
  of ``generate`` (``:153-205``): one prefill forward over the prompt (M = prompt
  length), then M = 1 decode steps, first-index argmax.  The seven projections
  of each layer are ``QuantizedLinear`` modules (the hot path).  K / V live in
  the reference's block pool [num_blocks, layers, 2, H_kv, B, D] (B =
  ``block_size``, 64 as in ``generate``; block table = identity, slot of
  position p = table[p // B] * B + p % B, ``engine/model.py:163-197``) and
  each layer stores its chunk with ``paged_kv_write`` and attends with the
  HIP ``chunked_attention`` (``engine/model.py:124-140``);
  ``attention="dense"`` keeps a contiguous cache and plain torch attention
  instead (for comparisons).  RMSNorm, RoPE and the fp32 lm_head are plain
  torch ops on the same device and stream.  With ``fuse=True`` q/k/v run as one
  ``FusedQuantizedLinear`` launch (same weights, row-stacked) and gate/up with
  the SiLU gate as one ``FusedGateUpSiLU`` launch (intermediate size a
  multiple of 16; else a ``FusedQuantizedLinear`` and torch's silu * up).
  ``lm_head_scheme="int8"|"int4"`` quantizes the vocab projection too (the
  reference keeps it fp32) and takes each greedy token from the argmax fused
  into that projection.

Weight dict keys (HF naming): ``embed_tokens.weight``, ``norm.weight``,
``lm_head.weight``, ``layers.{i}.{q,k,v,o,gate,up,down}_proj.weight``,
``layers.{i}.{q,k,v}_proj.bias`` (Qwen2), ``layers.{i}.input_layernorm.weight``,
``layers.{i}.post_attention_layernorm.weight``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import chunked_attention, paged_kv_write
from .quantization import (FusedGateUpSiLU, FusedQuantizedLinear, QuantizedLinear, QuantizedWeight,
                           quantize_int4_per_group, quantize_int8_per_channel, quantized_linear,
                           quantized_linear_argmax)

PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def quantize_all_linears(model: nn.Module, scheme: str, group_size: int = 128) -> nn.Module:
    """engine/model.py:80-91: swap the 7 projections of every layer in place."""
    for layer in model.model.layers:
        attn, mlp = layer.self_attn, layer.mlp
        attn.q_proj = QuantizedLinear(attn.q_proj, scheme=scheme, group_size=group_size)
        attn.k_proj = QuantizedLinear(attn.k_proj, scheme=scheme, group_size=group_size)
        attn.v_proj = QuantizedLinear(attn.v_proj, scheme=scheme, group_size=group_size)
        attn.o_proj = QuantizedLinear(attn.o_proj, scheme=scheme, group_size=group_size)
        mlp.gate_proj = QuantizedLinear(mlp.gate_proj, scheme=scheme, group_size=group_size)
        mlp.up_proj = QuantizedLinear(mlp.up_proj, scheme=scheme, group_size=group_size)
        mlp.down_proj = QuantizedLinear(mlp.down_proj, scheme=scheme, group_size=group_size)
    return model


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

    def proj_shape(self, name: str) -> Tuple[int, int]:
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


def _rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    var = x.pow(2).mean(-1, keepdim=True)
    return w * (x * torch.rsqrt(var + eps))


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([-x2, x1], dim=-1)


class DecoderLM:
    """Greedy decoder whose projections are ``QuantizedLinear`` (INT8 / INT4)."""

    def __init__(self, cfg: DecoderConfig, weights: Dict[str, torch.Tensor], scheme: str,
                 device: torch.device, group_size: int = 128, max_seq: int = 256,
                 fuse: bool = False, lm_head_scheme: Optional[str] = None,
                 quantized: Optional[Dict[str, "QuantizedWeight"]] = None,
                 block_size: int = 64, attention: str = "paged") -> None:
        """``quantized``: name (``layers.{i}.{proj}``) -> QuantizedWeight already
        on ``device`` (e.g. from kshipra_amd.checkpoint.load_quantized_weights);
        those projections are used as they are and their float weights are not
        needed in ``weights``."""
        if attention not in ("paged", "dense"):
            raise ValueError(f"attention must be 'paged' or 'dense', got {attention!r}")
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        self.cfg = cfg
        self.device = device
        self.attention = attention
        self.block_size = block_size
        dev = lambda t: torch.as_tensor(t).to(device=device, dtype=torch.float32)
        self.embed = dev(weights["embed_tokens.weight"])
        self.norm = dev(weights["norm.weight"])
        self.lm_head = dev(weights["lm_head.weight"])
        self.lm_head_q = None
        if lm_head_scheme == "int8":
            self.lm_head_q = quantize_int8_per_channel(self.lm_head)
        elif lm_head_scheme == "int4":
            self.lm_head_q = quantize_int4_per_group(self.lm_head, group_size)
        elif lm_head_scheme is not None:
            raise ValueError(f"lm_head_scheme must be None, 'int8' or 'int4', got {lm_head_scheme!r}")
        self.layers: List[Dict[str, object]] = []
        for li in range(cfg.num_layers):
            layer: Dict[str, object] = {
                "in_norm": dev(weights[f"layers.{li}.input_layernorm.weight"]),
                "post_norm": dev(weights[f"layers.{li}.post_attention_layernorm.weight"]),
            }
            for p in PROJ:
                out_f, in_f = cfg.proj_shape(p)
                bias_key = f"layers.{li}.{p}.bias"
                if quantized is not None and f"layers.{li}.{p}" in quantized:
                    qw = quantized[f"layers.{li}.{p}"]
                    if tuple(qw.original_shape) != (out_f, in_f):
                        raise ValueError(f"layers.{li}.{p}: shape {qw.original_shape} != {(out_f, in_f)}")
                    layer[p] = QuantizedLinear.from_quantized(
                        qw, dev(weights[bias_key]) if bias_key in weights else None)
                    continue
                lin = nn.Linear(in_f, out_f, bias=bias_key in weights, device=device)
                with torch.no_grad():
                    lin.weight.copy_(dev(weights[f"layers.{li}.{p}.weight"]))
                    if bias_key in weights:
                        lin.bias.copy_(dev(weights[bias_key]))
                layer[p] = QuantizedLinear(lin, scheme=scheme, group_size=group_size)
                del lin
            if fuse:
                layer["qkv"] = FusedQuantizedLinear([layer.pop(p) for p in ("q_proj", "k_proj", "v_proj")])
                gate, up = layer.pop("gate_proj"), layer.pop("up_proj")
                if gate.out_features % 16 == 0:
                    layer["gate_up_act"] = FusedGateUpSiLU(gate, up)
                else:
                    layer["gate_up"] = FusedQuantizedLinear([gate, up])
            self.layers.append(layer)
        exps = torch.arange(0, cfg.head_dim, 2, dtype=torch.float32) / cfg.head_dim
        self.inv_freq = (1.0 / (cfg.rope_theta ** exps)).to(device)
        self.max_seq = max_seq
        self.reset()

    def quantized_weights(self) -> Dict[str, "QuantizedWeight"]:
        """name (``layers.{i}.{proj}``) -> QuantizedWeight of every projection
        (per projection: build with ``fuse=False`` to export)."""
        out = {}
        for li, layer in enumerate(self.layers):
            for p in PROJ:
                if p not in layer:
                    raise ValueError("fused projections: build with fuse=False to export")
                out[f"layers.{li}.{p}"] = layer[p].weight
        return out

    def reset(self) -> None:
        c = self.cfg
        self.pos = 0
        if self.attention == "dense":
            shape = (c.num_layers, c.num_kv_heads, self.max_seq, c.head_dim)
            self.k_cache = torch.zeros(shape, dtype=torch.float32, device=self.device)
            self.v_cache = torch.zeros(shape, dtype=torch.float32, device=self.device)
            return
        # engine/model.py:165-177: pool sized for the whole sequence, identity table
        B = self.block_size
        nb = (self.max_seq + B - 1) // B
        self.pool = torch.zeros((nb, c.num_layers, 2, c.num_kv_heads, B, c.head_dim),
                                dtype=torch.float32, device=self.device)
        self.block_table = list(range(nb))
        self.table_dev = torch.tensor(self.block_table, dtype=torch.int32, device=self.device)

    @torch.inference_mode()
    def forward(self, ids: List[int]) -> torch.Tensor:
        """Logits [L, vocab] for the next L tokens (engine/model.py:93-151)."""
        h = self.hidden(ids)
        if self.lm_head_q is not None:
            return quantized_linear(h, self.lm_head_q)
        return F.linear(h, self.lm_head)

    @torch.inference_mode()
    def hidden(self, ids: List[int]) -> torch.Tensor:
        """Final-normed hidden states [L, hidden] (engine/model.py:93-150),
        advancing the KV cache."""
        c = self.cfg
        L = len(ids)
        if self.pos + L > self.max_seq:
            raise RuntimeError("KV cache capacity exceeded")
        pos = torch.arange(self.pos, self.pos + L, device=self.device, dtype=torch.float32)
        freqs = pos[:, None] * self.inv_freq[None, :]
        emb = torch.cat([freqs, freqs], dim=-1)
        cos, sin = emb.cos(), emb.sin()
        h = self.embed[torch.as_tensor(ids, device=self.device)]
        g = c.num_heads // c.num_kv_heads
        scale = 1.0 / math.sqrt(c.head_dim)
        S = self.pos + L
        if self.attention == "dense":
            qpos = torch.arange(self.pos, S, device=self.device)
            kpos = torch.arange(S, device=self.device)
            mask = kpos[None, :] > qpos[:, None]
        else:
            B = self.block_size
            slots = torch.tensor([self.block_table[p // B] * B + p % B for p in range(self.pos, S)],
                                 dtype=torch.int64, device=self.device)
            attn_buf = torch.empty((L, c.num_heads, c.head_dim), dtype=torch.float32,
                                   device=self.device)
        for li, layer in enumerate(self.layers):
            res = h
            x = _rms_norm(h, layer["in_norm"], c.rms_norm_eps)
            if "qkv" in layer:
                q, k, v = layer["qkv"](x)
            else:
                q, k, v = layer["q_proj"](x), layer["k_proj"](x), layer["v_proj"](x)
            q = q.reshape(L, c.num_heads, c.head_dim).transpose(0, 1)
            k = k.reshape(L, c.num_kv_heads, c.head_dim).transpose(0, 1)
            v = v.reshape(L, c.num_kv_heads, c.head_dim).transpose(0, 1)
            q = q * cos[None] + _rotate_half(q) * sin[None]
            k = k * cos[None] + _rotate_half(k) * sin[None]
            if self.attention == "dense":
                self.k_cache[li, :, self.pos:S] = k
                self.v_cache[li, :, self.pos:S] = v
                kc = self.k_cache[li, :, :S].repeat_interleave(g, dim=0).contiguous()
                vc = self.v_cache[li, :, :S].repeat_interleave(g, dim=0).contiguous()
                s = torch.matmul(q.contiguous(), kc.transpose(1, 2).contiguous()) * scale
                s = s.masked_fill(mask[None], float("-inf"))
                p = torch.softmax(s, dim=-1)
                a = torch.matmul(p, vc).transpose(0, 1).reshape(L, c.num_heads * c.head_dim)
            else:
                paged_kv_write(self.pool, li, k, v, slots)
                chunked_attention(q, self.pool[:, li, 0], self.pool[:, li, 1], self.table_dev,
                                  self.pos, L, self.block_size, out=attn_buf.transpose(0, 1))
                a = attn_buf.view(L, c.num_heads * c.head_dim)
            h = res + layer["o_proj"](a.contiguous())
            res = h
            x = _rms_norm(h, layer["post_norm"], c.rms_norm_eps)
            if "gate_up_act" in layer:
                act = layer["gate_up_act"](x)
            else:
                if "gate_up" in layer:
                    gate, up = layer["gate_up"](x)
                else:
                    gate, up = layer["gate_proj"](x), layer["up_proj"](x)
                act = F.silu(gate) * up
            h = res + layer["down_proj"](act)
        self.pos = S
        return _rms_norm(h, self.norm, c.rms_norm_eps)

    @torch.inference_mode()
    def _next(self, ids: List[int]) -> Tuple[int, torch.Tensor]:
        """Greedy token after ``ids`` and its logits row (engine/model.py:187,200)."""
        h = self.hidden(ids)[-1:]
        if self.lm_head_q is not None:
            tok, logits = quantized_linear_argmax(h, self.lm_head_q, return_logits=True)
            return int(tok[0].item()), logits[0]
        logits = F.linear(h, self.lm_head)[0]
        return int(torch.argmax(logits).item()), logits

    @torch.inference_mode()
    def generate(self, prompt: List[int], max_new_tokens: int,
                 eos_token_id: Optional[int] = None) -> Tuple[List[int], List[torch.Tensor]]:
        """engine/model.py:153-205 greedy loop; returns (tokens, per-step logits)."""
        self.reset()
        tok, logits = self._next(prompt)
        toks, all_logits = [tok], [logits]
        for _ in range(1, max_new_tokens):
            if eos_token_id is not None and toks[-1] == eos_token_id:
                break
            tok, logits = self._next([toks[-1]])
            toks.append(tok)
            all_logits.append(logits)
        return toks, all_logits
