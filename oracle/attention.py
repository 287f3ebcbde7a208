"""CPU restatement of the paged KV write and chunked attention.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker for the
HIP kernels of ``kshipra_amd/csrc/kq_attention.hip``.

* ``kv_write``             -- ``engine/model.py:124-128``: token t's K / V of
  every KV head go to ``pool[slot // B, layer, 0 / 1, :, slot % B, :]`` with
  ``slot = slot_mapping[t]``.
* ``chunked_attention``    -- ``engine/chunked_prefill.py:93-140``: online
  softmax over the blocks of ``block_table`` (prefix and chunk keys), GQA by
  ``repeat_interleave`` (query head h reads KV head h // g), the causal mask
  ``key position > query position`` for query i at position prefix_len + i,
  scale 1 / sqrt(D); float64 here.
* ``monolithic_attention`` -- ``engine/chunked_prefill.py:47-90``: the same
  attention as one masked softmax over the concatenated keys (the
  reference's own oracle for the chunked path), float64.

Pinned in ``tests/test_oracle_attention.py``: chunked == monolithic on the
reference tests' configurations (``tests/test_chunked_prefill.py:22-80``)
and on GQA / ragged-block cases; closed forms (one key -> its value, equal
keys -> the mean of the values, a dominant key -> its value); the KV write
against an explicit gather.
"""

from __future__ import annotations

import math
from typing import Sequence

import numpy as np


def kv_write(pool: np.ndarray, layer: int, k: np.ndarray, v: np.ndarray,
             slot_mapping: Sequence[int]) -> None:
    """pool: [num_blocks, layers, 2, H_kv, B, D]; k, v: [H_kv, L, D]."""
    block_size = pool.shape[4]
    for t, slot in enumerate(slot_mapping):
        blk, off = slot // block_size, slot % block_size
        pool[blk, layer, 0, :, off, :] = k[:, t, :]
        pool[blk, layer, 1, :, off, :] = v[:, t, :]


def chunked_attention(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray,
                      block_table: Sequence[int], prefix_len: int, chunk_len: int,
                      block_size: int) -> np.ndarray:
    """q: [H_q, C, D]; k_pool, v_pool: [num_blocks, H_kv, B, D] -> [H_q, C, D]."""
    hq, c, d = q.shape
    hkv = k_pool.shape[1]
    assert hq % hkv == 0
    g = hq // hkv
    q = q.astype(np.float64)
    scale = 1.0 / math.sqrt(d)
    total = prefix_len + chunk_len
    m = np.full((hq, c), -np.inf)
    l = np.zeros((hq, c))
    acc = np.zeros((hq, c, d))
    qpos = prefix_len + np.arange(c)
    for j in range((total + block_size - 1) // block_size):
        blk = block_table[j]
        start = j * block_size
        n = min(start + block_size, total) - start
        kt = np.repeat(k_pool[blk, :, :n, :].astype(np.float64), g, axis=0)   # [H_q, n, D]
        vt = np.repeat(v_pool[blk, :, :n, :].astype(np.float64), g, axis=0)
        s = np.einsum("hcd,hnd->hcn", q, kt) * scale
        if start + n > prefix_len:
            kpos = start + np.arange(n)
            s = np.where((kpos[None, :] > qpos[:, None])[None], -np.inf, s)
        m_new = np.maximum(m, s.max(axis=-1))
        m_safe = np.where(np.isinf(m_new), 0.0, m_new)
        p = np.exp(s - m_safe[..., None])
        corr = np.exp(m - m_safe)
        l = l * corr + p.sum(axis=-1)
        acc = acc * corr[..., None] + np.einsum("hcn,hnd->hcd", p, vt)
        m = m_new
    return acc / l[..., None]


def monolithic_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, prefix_len: int,
                         chunk_len: int) -> np.ndarray:
    """q: [H, C, D]; k, v: [H, P + C, D] (same head count) -> [H, C, D]."""
    h, c, d = q.shape
    s = np.einsum("hcd,hnd->hcn", q.astype(np.float64), k.astype(np.float64)) / math.sqrt(d)
    kpos = np.arange(prefix_len + chunk_len)
    qpos = prefix_len + np.arange(c)
    s = np.where((kpos[None, :] > qpos[:, None])[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("hcn,hnd->hcd", p, v.astype(np.float64))


def fill_pool(k: np.ndarray, v: np.ndarray, block_size: int, block_table: Sequence[int],
              num_blocks: int) -> tuple:
    """Pools [num_blocks, H_kv, B, D] holding k, v ([H_kv, S, D]) at the
    blocks of block_table (token i -> block_table[i // B], offset i % B)."""
    hkv, s, d = k.shape
    kp = np.zeros((num_blocks, hkv, block_size, d), dtype=k.dtype)
    vp = np.zeros_like(kp)
    for i in range(s):
        kp[block_table[i // block_size], :, i % block_size, :] = k[:, i, :]
        vp[block_table[i // block_size], :, i % block_size, :] = v[:, i, :]
    return kp, vp
