"""Pinning the attention oracle (oracle/attention.py) on the CPU.

* the reference's golden relation: chunked online softmax == monolithic
  masked softmax (tests/test_chunked_prefill.py:22-80 use rel-L2 < 1e-5 in
  fp32; float64 here, so 1e-12), on its own configurations and on GQA,
  shuffled block tables and ragged last blocks;
* closed forms: a single key returns its value; equal keys return the mean
  of the values; a dominant key returns its value; a query that sees only
  key 0 (position 0, no prefix) returns v[0];
* GQA: query head h attends with KV head h // g (repeat_interleave);
* the KV write against an explicit read-back at the mapped slots.
A planted error (a dropped causal mask, a wrong GQA head map) fails these.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import attention as att


def _rel(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(a), 1e-300))


def _case(h, hkv, c, p, d, b, seed, shuffle=False):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((h, c, d))
    k = rng.standard_normal((hkv, p + c, d))
    v = rng.standard_normal((hkv, p + c, d))
    nb = (p + c + b - 1) // b
    table = list(range(nb))
    if shuffle:
        table = list(rng.permutation(nb + 3)[:nb])
    kp, vp = att.fill_pool(k, v, b, table, nb + 3)
    return q, k, v, kp, vp, table


@pytest.mark.parametrize("h,hkv,c,p,d,b,shuffle", [
    (4, 4, 128, 256, 64, 16, False),    # tests/test_chunked_prefill.py:22
    (4, 4, 1, 1024, 64, 16, False),     # :55 (prefix only, one query)
    (8, 2, 33, 37, 64, 16, True),       # GQA, ragged blocks, shuffled table
    (14, 2, 5, 0, 64, 32, True),        # no prefix (pure causal chunk)
    (32, 8, 1, 300, 128, 16, True),     # Llama-3-8B heads, one decode step
])
def test_chunked_equals_monolithic(h, hkv, c, p, d, b, shuffle):
    q, k, v, kp, vp, table = _case(h, hkv, c, p, d, b, seed=h + c + p, shuffle=shuffle)
    out = att.chunked_attention(q, kp, vp, table, p, c, b)
    g = h // hkv
    ref = att.monolithic_attention(q, np.repeat(k, g, axis=0), np.repeat(v, g, axis=0), p, c)
    assert _rel(ref, out) < 1e-12


def test_closed_forms():
    rng = np.random.default_rng(1)
    d = 64
    v = rng.standard_normal((1, 1, d))
    k = rng.standard_normal((1, 1, d))
    q = rng.standard_normal((1, 1, d))
    kp, vp = att.fill_pool(k, v, 16, [0], 1)
    assert np.allclose(att.chunked_attention(q, kp, vp, [0], 0, 1, 16), v, rtol=0, atol=1e-15)
    # equal keys: uniform weights -> mean of the values
    s = 40
    k = np.repeat(rng.standard_normal((1, 1, d)), s, axis=1)
    v = rng.standard_normal((1, s, d))
    q = rng.standard_normal((1, 1, d))
    kp, vp = att.fill_pool(k, v, 16, [2, 0, 1], 3)
    out = att.chunked_attention(q, kp, vp, [2, 0, 1], s - 1, 1, 16)
    assert np.allclose(out[0, 0], v[0].mean(axis=0), rtol=0, atol=1e-12)
    # a dominant key wins
    k = rng.standard_normal((1, s, d)) * 0.01
    k[0, 17] = 50.0
    q = np.full((1, 1, d), 1.0)
    kp, vp = att.fill_pool(k, v, 16, [0, 1, 2], 3)
    out = att.chunked_attention(q, kp, vp, [0, 1, 2], s - 1, 1, 16)
    assert np.allclose(out[0, 0], v[0, 17], rtol=0, atol=1e-9)
    # first chunk query (position 0) sees only key 0
    k = rng.standard_normal((1, 5, d))
    v = rng.standard_normal((1, 5, d))
    q = rng.standard_normal((1, 5, d))
    kp, vp = att.fill_pool(k, v, 16, [0], 1)
    out = att.chunked_attention(q, kp, vp, [0], 0, 5, 16)
    assert np.allclose(out[0, 0], v[0, 0], rtol=0, atol=1e-15)


def test_gqa_head_map():
    """Query head h uses KV head h // g (not h % hkv)."""
    q, k, v, kp, vp, table = _case(4, 2, 3, 10, 64, 16, seed=3)
    out = att.chunked_attention(q, kp, vp, table, 10, 3, 16)
    for h in range(4):
        ref = att.monolithic_attention(q[h:h + 1], k[h // 2:h // 2 + 1], v[h // 2:h // 2 + 1], 10, 3)
        assert _rel(ref, out[h:h + 1]) < 1e-12
    wrong = att.monolithic_attention(q[1:2], k[1:2], v[1:2], 10, 3)  # the h % hkv map
    assert _rel(wrong, out[1:2]) > 1e-3


def test_causal_mask_matters():
    q, k, v, kp, vp, table = _case(2, 2, 8, 4, 64, 16, seed=5)
    out = att.chunked_attention(q, kp, vp, table, 4, 8, 16)
    s = np.einsum("hcd,hnd->hcn", q, k) / 8.0      # every query sees all 12 keys
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    no_mask = np.einsum("hcn,hnd->hcd", p, v)
    assert _rel(no_mask, out) > 1e-3
    # the last query (position 11) sees every key: unmasked there
    assert _rel(no_mask[:, -1], out[:, -1]) < 1e-12


def test_kv_write_places_tokens_at_their_slots():
    rng = np.random.default_rng(7)
    hkv, L, d, b = 2, 9, 8, 4
    pool = np.zeros((5, 3, 2, hkv, b, d))
    k, v = rng.standard_normal((hkv, L, d)), rng.standard_normal((hkv, L, d))
    slots = [17, 3, 4, 5, 6, 12, 0, 19, 8]
    att.kv_write(pool, 1, k, v, slots)
    for t, s in enumerate(slots):
        assert np.array_equal(pool[s // b, 1, 0, :, s % b], k[:, t])
        assert np.array_equal(pool[s // b, 1, 1, :, s % b], v[:, t])
    assert not pool[:, 0].any() and not pool[:, 2].any()
