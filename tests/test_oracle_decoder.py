"""Pins the decoder oracle (oracle/decoder.py) to the model semantics the
reference runs, without importing the reference.

Kshipra computes RMSNorm and the MLP through HF modules (engine/model.py:113,
146-147) and RoPE through its own helpers (:30-55), and proves its pipeline
token-identical to HF ``generate`` on a random-init model (demo.py:17-56,
README.md:75-76).  Here HF ``Qwen2ForCausalLM`` / ``LlamaForCausalLM`` (the
installed transformers, run on the CPU in fp32) are built from the same
weight dict, with the oracle's exact dequantized projection weights loaded
into their ``nn.Linear`` layers, and must agree with ``OracleDecoder``:

* per-step logits within 1e-5 of the largest logit (fp32 summation order is
  the only difference), over a prompt and >= 8 greedy steps;
* identical greedy tokens (HF ``generate(do_sample=False)``);

on configurations with GQA, q/k/v biases (Qwen2), none (Llama), non-unit
RMSNorm weights, a large eps (so its placement matters) and two RoPE bases.
Planted slips in the oracle -- the other ``rotate_half`` sign convention,
eps outside the square root, ``theta^(i/D)`` instead of ``theta^(2i/D)``, a
non-causal mask, the ``h % H_kv`` head map -- must each break the agreement.

Closed forms on the oracle's RoPE and RMSNorm: position 0 is the identity,
rotations preserve norms, <RoPE(q, m), RoPE(k, n)> depends only on m - n,
and RMSNorm of a constant row with unit weight is +-1/sqrt(1 + eps/c^2).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import decoder_weights
from oracle import decoder as od
from oracle import quant

transformers = pytest.importorskip("transformers")

TOL = 1e-5
STEPS = 10
PROMPT = [3, 14, 15, 92, 65, 35]

CONFIGS = {
    # Qwen2-style: q/k/v biases, GQA 4:2 (g = 2), RoPE base 1e6
    "qwen2": dict(vocab_size=101, hidden_size=128, intermediate_size=256, num_layers=3,
                  num_heads=4, num_kv_heads=2, head_dim=32, rope_theta=1000000.0,
                  rms_norm_eps=1e-6, qkv_bias=True),
    # Llama-style: no biases, GQA 8:2 (g = 4), RoPE base 1e4, eps large enough
    # that x / sqrt(var + eps) and x / (sqrt(var) + eps) differ visibly
    "llama": dict(vocab_size=97, hidden_size=128, intermediate_size=192, num_layers=2,
                  num_heads=8, num_kv_heads=2, head_dim=16, rope_theta=10000.0,
                  rms_norm_eps=0.05, qkv_bias=False),
}


# Random-init N(0, 0.02) projections leave attention scores near zero (the
# softmax is almost uniform and position barely matters), which would hide
# RoPE and masking slips; these gains make the scores and the attention
# output O(1) while keeping the network the same function of its weights.
GAINS = {"q_proj": 10.0, "k_proj": 10.0, "v_proj": 5.0, "o_proj": 5.0,
         "gate_proj": 3.0, "up_proj": 3.0, "down_proj": 3.0}


def _weights(cfg: dict, seed: int):
    w = decoder_weights(cfg, seed=seed)
    for k in list(w):
        for p, gain in GAINS.items():
            if k.endswith(f"{p}.weight"):
                w[k] = (w[k] * np.float32(gain)).astype(np.float32)
    rng = np.random.default_rng(seed + 100)
    for k in list(w):
        if k.endswith("layernorm.weight") or k == "norm.weight":
            w[k] = (1.0 + 0.2 * rng.standard_normal(w[k].shape)).astype(np.float32)
    # untie the lm_head so a swapped tensor would show
    w["lm_head.weight"] = (w["embed_tokens.weight"] + 0.01 * rng.standard_normal(
        w["embed_tokens.weight"].shape)).astype(np.float32)
    return w


def _hf_model(cfg: dict, w: dict, scheme: str):
    common = dict(vocab_size=cfg["vocab_size"], hidden_size=cfg["hidden_size"],
                  intermediate_size=cfg["intermediate_size"], num_hidden_layers=cfg["num_layers"],
                  num_attention_heads=cfg["num_heads"], num_key_value_heads=cfg["num_kv_heads"],
                  max_position_embeddings=256, rope_theta=cfg["rope_theta"],
                  rms_norm_eps=cfg["rms_norm_eps"], tie_word_embeddings=False)
    if cfg["qkv_bias"]:
        hf_cfg = transformers.Qwen2Config(**common)
        model = transformers.Qwen2ForCausalLM(hf_cfg)
    else:
        hf_cfg = transformers.LlamaConfig(**common, head_dim=cfg["head_dim"], attention_bias=False,
                                          mlp_bias=False)
        model = transformers.LlamaForCausalLM(hf_cfg)
    assert cfg["hidden_size"] // cfg["num_heads"] == cfg["head_dim"] or not cfg["qkv_bias"]
    sd = {"model.embed_tokens.weight": w["embed_tokens.weight"], "lm_head.weight": w["lm_head.weight"],
          "model.norm.weight": w["norm.weight"]}
    for li in range(cfg["num_layers"]):
        pre = f"model.layers.{li}."
        sd[pre + "input_layernorm.weight"] = w[f"layers.{li}.input_layernorm.weight"]
        sd[pre + "post_attention_layernorm.weight"] = w[f"layers.{li}.post_attention_layernorm.weight"]
        for p in od.PROJ:
            mod = "self_attn." if p in ("q_proj", "k_proj", "v_proj", "o_proj") else "mlp."
            w_hat = quant.dequantize(quant.quantize(w[f"layers.{li}.{p}.weight"], scheme, 128))
            sd[pre + mod + p + ".weight"] = w_hat
            if f"layers.{li}.{p}.bias" in w:
                sd[pre + mod + p + ".bias"] = w[f"layers.{li}.{p}.bias"]
    state = {k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)) for k, v in sd.items()}
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return model.eval().float()


def _compare(cfg_name: str, scheme: str, seed: int = 0):
    """(max per-step logit error / max |logit|, HF tokens, oracle tokens, min top-2 gap)."""
    cfg = CONFIGS[cfg_name]
    w = _weights(cfg, seed)
    model = _hf_model(cfg, w, scheme)
    with torch.no_grad():
        hf = model.generate(torch.tensor([PROMPT]), max_new_tokens=STEPS, do_sample=False, num_beams=1,
                            pad_token_id=0, eos_token_id=None)
        hf_tokens = hf[0, len(PROMPT):].tolist()
        seq = torch.tensor([PROMPT + hf_tokens[:-1]])
        hf_logits = model(seq).logits[0, len(PROMPT) - 1:].numpy().astype(np.float64)
    dec = od.OracleDecoder(od.DecoderConfig(**cfg), w, scheme)
    toks, logits = dec.generate(PROMPT, STEPS)
    ol = np.stack(logits).astype(np.float64)
    n = min(len(ol), len(hf_logits))
    err = np.abs(ol[:n] - hf_logits[:n]).max() / np.abs(hf_logits[:n]).max()
    top2 = np.sort(hf_logits, axis=-1)[:, -2:]
    gap = float((top2[:, 1] - top2[:, 0]).min() / np.abs(hf_logits).max())
    return err, hf_tokens, toks, gap


@pytest.mark.parametrize("cfg_name", sorted(CONFIGS))
@pytest.mark.parametrize("scheme", ["int8", "int4"])
def test_oracle_decoder_matches_hf(cfg_name, scheme):
    err, hf_tokens, toks, gap = _compare(cfg_name, scheme)
    print(f"[oracle vs HF {cfg_name} {scheme}] logits rel {err:.2e}, min top-2 gap {gap:.2e}, "
          f"tokens {toks}", flush=True)
    assert err <= TOL
    assert toks == hf_tokens


def _slip_rope_sign(x, cos, sin):
    half = x.shape[-1] // 2
    rot = np.concatenate([x[..., half:], -x[..., :half]], axis=-1)     # rotate the other way
    return (x * cos[None] + rot * sin[None]).astype(np.float32)


def _slip_eps(x, w, eps):
    x = x.astype(np.float32)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    return (w * (x / (np.sqrt(var) + np.float32(eps)))).astype(np.float32)


def _slip_theta(head_dim, positions, theta):
    exps = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(2 * head_dim)   # i/D
    inv_freq = (np.float32(1.0) / (np.float32(theta) ** exps)).astype(np.float32)
    freqs = positions.astype(np.float32)[:, None] * inv_freq[None, :]
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def _slip_head_map(kv, g):
    return np.tile(kv, (g, 1, 1))                     # query head h reads KV head h % H_kv


def _slip_no_mask(qpos, s):
    return np.zeros((len(qpos), s), dtype=bool)       # every cached key visible


@pytest.mark.parametrize("slip", ["rope_sign", "eps", "theta", "causal", "head_map"])
def test_planted_slips_break_agreement(monkeypatch, slip):
    cfg_name = "llama"
    if slip == "rope_sign":
        monkeypatch.setattr(od, "apply_rope", _slip_rope_sign)
    elif slip == "eps":
        monkeypatch.setattr(od, "rms_norm", _slip_eps)
    elif slip == "theta":
        monkeypatch.setattr(od, "rope_cos_sin", _slip_theta)
    elif slip == "causal":
        monkeypatch.setattr(od, "future_mask", _slip_no_mask)
    else:
        monkeypatch.setattr(od, "expand_kv", _slip_head_map)
    err, hf_tokens, toks, _ = _compare(cfg_name, "int8")
    print(f"[planted {slip}] logits rel {err:.2e}, tokens {toks} vs {hf_tokens}", flush=True)
    assert err > 100 * TOL


def test_rope_closed_forms():
    rng = np.random.default_rng(0)
    d, theta = 64, 10000.0
    q = rng.standard_normal((3, 1, d)).astype(np.float32)
    k = rng.standard_normal((3, 1, d)).astype(np.float32)
    cos0, sin0 = od.rope_cos_sin(d, np.array([0]), theta)
    np.testing.assert_array_equal(od.apply_rope(q, cos0, sin0), q)              # position 0
    for pos in (1, 17, 1000):
        c, s = od.rope_cos_sin(d, np.array([pos]), theta)
        r = od.apply_rope(q, c, s)
        np.testing.assert_allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(q, axis=-1), rtol=1e-5)
    dots = []
    for m, n in ((5, 2), (13, 10), (103, 100)):                                  # m - n = 3
        cm, sm = od.rope_cos_sin(d, np.array([m]), theta)
        cn, sn = od.rope_cos_sin(d, np.array([n]), theta)
        dots.append(np.sum(od.apply_rope(q, cm, sm) * od.apply_rope(k, cn, sn), axis=-1))
    np.testing.assert_allclose(dots[0], dots[1], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(dots[0], dots[2], rtol=1e-4, atol=1e-4)
    # frequency i of the first half rotates by pos * theta^(-2i/d)
    c, s = od.rope_cos_sin(d, np.array([1]), theta)
    i = np.arange(d // 2)
    np.testing.assert_allclose(np.arccos(np.clip(c[0, :d // 2], -1, 1)),
                               np.abs(np.angle(np.exp(1j * theta ** (-2.0 * i / d)))), atol=1e-3)


def test_rms_norm_closed_forms():
    for cval, eps in ((3.0, 1e-6), (-0.5, 1e-6), (0.01, 0.05)):
        x = np.full((2, 64), cval, np.float32)
        y = od.rms_norm(x, np.ones(64, np.float32), eps)
        np.testing.assert_allclose(y, np.sign(cval) / np.sqrt(1.0 + eps / cval ** 2), rtol=1e-6)
    x = np.random.default_rng(1).standard_normal((4, 32)).astype(np.float32)
    w = np.linspace(0.5, 2.0, 32).astype(np.float32)
    y = od.rms_norm(x, w, 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean((y / w) ** 2, axis=-1)), 1.0, rtol=1e-5)
