"""GPU parity at the decoder level: greedy tokens of the random-init model.

The GPU decoder (kshipra_amd.model.DecoderLM: every projection a HIP
QuantizedLinear) and the oracle decoder (oracle.decoder: exact dequantized
fp32 weights + fp32 BLAS, the op order of engine/model.py:93-205) run the
same seeded weights.  Bar: identical greedy tokens at every step; the logits'
worst relative deviation and the smallest top-2 gap over the steps are printed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import QWEN05B, decoder_weights
from kshipra_amd.model import DecoderConfig, DecoderLM, quantize_all_linears
from kshipra_amd.quantization import QuantizedLinear
from oracle import decoder as odec

pytestmark = pytest.mark.gpu


def _greedy_parity(gpu, cfg_dict, scheme, prompt, new_tokens, seed, fuse=False, lm_head_scheme=None,
                   **attn):
    w = decoder_weights(cfg_dict, seed=seed)
    ocfg = odec.DecoderConfig(**cfg_dict)
    gcfg = DecoderConfig(**cfg_dict)
    gpu_lm = DecoderLM(gcfg, {k: torch.from_numpy(v) for k, v in w.items()}, scheme, gpu,
                       max_seq=len(prompt) + new_tokens + 1, fuse=fuse, lm_head_scheme=lm_head_scheme,
                       **attn)
    toks_g, logits_g = gpu_lm.generate(prompt, new_tokens)
    oracle_lm = odec.OracleDecoder(ocfg, w, scheme, lm_head_scheme=lm_head_scheme)
    toks_o, logits_o = oracle_lm.generate(prompt, new_tokens)
    worst, min_gap = 0.0, np.inf
    for lg, lo in zip(logits_g, logits_o):
        lg = lg.float().cpu().numpy()
        worst = max(worst, float(np.abs(lg - lo).max() / np.abs(lo).max()))
        top2 = np.sort(lo)[-2:]
        min_gap = min(min_gap, float(top2[1] - top2[0]))
    print(f"[{scheme} L={cfg_dict['num_layers']} prompt={len(prompt)} fuse={fuse} "
          f"lm_head={lm_head_scheme} {attn}] tokens {toks_g} "
          f"logit rel dev {worst:.3e} min top-2 gap {min_gap:.3e}", flush=True)
    assert toks_g == toks_o
    assert worst < 1e-3


@pytest.mark.parametrize("scheme", ["int4", "int8"])
def test_qwen05b_shaped_greedy_tokens(gpu, scheme):
    """Random-init Qwen2.5-0.5B-shaped decoder (24 layers, 896/4864, 14/2 heads,
    head_dim 64, vocab 151936, q/k/v bias): prefill of 6 tokens then M = 1 decode."""
    _greedy_parity(gpu, QWEN05B, scheme, [1, 42, 100, 201, 7, 999], 8, seed=0)


@pytest.mark.parametrize("scheme", ["int4", "int8"])
def test_qwen05b_shaped_fused_projections(gpu, scheme):
    """Same model with q/k/v and gate/up each run as one fused launch."""
    _greedy_parity(gpu, QWEN05B, scheme, [1, 42, 100, 201, 7, 999], 8, seed=0, fuse=True)


@pytest.mark.parametrize("scheme", ["int4", "int8"])
def test_qwen05b_shaped_quantized_lm_head(gpu, scheme):
    """Fused projections plus a quantized lm_head whose greedy token comes from
    the argmax fused into the projection; the oracle quantizes its lm_head the
    same way."""
    _greedy_parity(gpu, QWEN05B, scheme, [1, 42, 100, 201, 7, 999], 8, seed=0, fuse=True,
                   lm_head_scheme=scheme)


@pytest.mark.parametrize("scheme", ["int4", "int8"])
def test_long_prompt_uses_gemm_prefill(gpu, scheme):
    """A 48-token prompt sends the prefill projections through the tiled GEMM."""
    cfg = dict(QWEN05B, num_layers=4, vocab_size=32000)
    prompt = [int(t) for t in np.random.default_rng(1).integers(0, 32000, 48)]
    _greedy_parity(gpu, cfg, scheme, prompt, 6, seed=1)


@pytest.mark.parametrize("scheme", ["int4", "int8"])
def test_paged_pool_small_blocks(gpu, scheme):
    """K / V in a block pool of 16-token blocks: the 40-token prefill spans
    three blocks (several 16-row attention tiles) and decode crosses the next
    block boundary (engine/model.py:124-140 with the generate loop's slots)."""
    cfg = dict(QWEN05B, num_layers=4, vocab_size=32000)
    prompt = [int(t) for t in np.random.default_rng(2).integers(0, 32000, 40)]
    _greedy_parity(gpu, cfg, scheme, prompt, 12, seed=2, fuse=True, block_size=16)


def test_long_prompt_shared_tile_attention(gpu):
    """A 600-token prompt: the prefill's attention runs as workgroups of 4 row
    tiles sharing K / V tiles (7 x 600 rows per KV head), the decode steps
    after it split their ~600 keys; INT4 projections through the GEMM path."""
    cfg = dict(QWEN05B, num_layers=3, vocab_size=32000)
    prompt = [int(t) for t in np.random.default_rng(4).integers(0, 32000, 600)]
    _greedy_parity(gpu, cfg, "int4", prompt, 4, seed=4, fuse=True)


def test_dense_attention_option(gpu):
    """attention="dense" (contiguous cache, torch attention) gives the same tokens."""
    cfg = dict(QWEN05B, num_layers=4, vocab_size=32000)
    _greedy_parity(gpu, cfg, "int4", [1, 42, 100, 201, 7, 999], 6, seed=3, attention="dense")


def test_hf_projection_swap(gpu):
    """engine/model.py:80-91 on a tiny HF Llama: 7 swaps per layer, lm_head and
    embeddings untouched, logits close to the same model with the exact
    dequantized weights put back into nn.Linear."""
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(0)
    cfg = transformers.LlamaConfig(vocab_size=256, hidden_size=128, intermediate_size=256,
                                   num_hidden_layers=2, num_attention_heads=4,
                                   num_key_value_heads=2, max_position_embeddings=64)
    hf = transformers.LlamaForCausalLM(cfg).to(gpu).eval()
    ids = torch.tensor([[1, 42, 100, 201, 7]], device=gpu)
    quantize_all_linears(hf, "int4")
    for layer in hf.model.layers:
        for mod in (layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj,
                    layer.self_attn.o_proj, layer.mlp.gate_proj, layer.mlp.up_proj,
                    layer.mlp.down_proj):
            assert isinstance(mod, QuantizedLinear)
    assert isinstance(hf.lm_head, torch.nn.Linear)
    with torch.no_grad():
        logits_q = hf(ids).logits.float()
        for layer in hf.model.layers:                 # exact dequantized weights, plain Linear
            for parent, name in ((layer.self_attn, "q_proj"), (layer.self_attn, "k_proj"),
                                 (layer.self_attn, "v_proj"), (layer.self_attn, "o_proj"),
                                 (layer.mlp, "gate_proj"), (layer.mlp, "up_proj"),
                                 (layer.mlp, "down_proj")):
                q = getattr(parent, name)
                lin = torch.nn.Linear(q.in_features, q.out_features, bias=q.bias is not None,
                                      device=gpu)
                lin.weight.copy_(q.weight.dequantize(torch.float32))
                if q.bias is not None:
                    lin.bias.copy_(q.bias)
                setattr(parent, name, lin)
        logits_d = hf(ids).logits.float()
    rel = ((logits_q - logits_d).abs().max() / logits_d.abs().max()).item()
    print(f"[hf swap] logits rel dev {rel:.3e}", flush=True)
    assert rel < 1e-4
