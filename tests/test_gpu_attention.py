"""GPU parity of the paged K/V write and chunked attention
(kshipra_amd/attention.py, csrc/kq_attention.hip).

* ``paged_kv_write`` is bit-exact with the oracle's store loop
  (engine/model.py:124-129), including a repeated slot (last token wins),
  negative slots (Python indexing from the end) and the untouched layers.
* ``chunked_attention`` against the float64 oracle (engine/chunked_prefill.py:
  93-140, itself pinned against monolithic masked softmax): the reference's
  own bar for chunked vs monolithic, relative L2 < 1e-5
  (tests/test_chunked_prefill.py:22-52), plus an element-wise bar
  max|out - ref| <= 1e-5 * max|v| (fp32 rounding of the D-term dot products
  and of the softmax; measured values are printed).  Cases: the reference
  tests' configurations, GQA g = 1 / 4 / 7, D = 64 / 128, block sizes that
  are and are not multiples of 16, shuffled block tables, prefix-only decode
  over long contexts (the split-key path), long prefill chunks, strided q /
  out views, device block tables, and 30 seeded random configurations
  (decode-like contexts up to 8k keys, chunks up to 96 queries).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kshipra_amd.attention import chunked_attention, paged_kv_write
from oracle import attention as att

pytestmark = pytest.mark.gpu

REL_L2 = 1e-5
ELEM = 1e-5


def _case(h, hkv, c, p, d, b, seed, shuffle):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((h, c, d)).astype(np.float32)
    k = rng.standard_normal((hkv, p + c, d)).astype(np.float32)
    v = rng.standard_normal((hkv, p + c, d)).astype(np.float32)
    nb = (p + c + b - 1) // b
    extra = 3
    table = list(range(nb))
    if shuffle:
        table = [int(x) for x in rng.permutation(nb + extra)[:nb]]
    kp, vp = att.fill_pool(k, v, b, table, nb + extra)
    return q, kp, vp, table


def _check(name, out, ref, vmax):
    out = out.astype(np.float64)
    rel = float(np.linalg.norm(out - ref) / np.linalg.norm(ref))
    elem = float(np.abs(out - ref).max() / vmax)
    print(f"[attention {name}] rel-L2 {rel:.3e} max-err/max|v| {elem:.3e}", flush=True)
    assert rel < REL_L2 and elem < ELEM, (name, rel, elem)


CASES = [
    # h, hkv, c, p, d, b, shuffle
    (4, 4, 128, 256, 64, 16, False),     # tests/test_chunked_prefill.py:22
    (4, 4, 1, 1024, 64, 16, False),      # :55 prefix only, one query
    (32, 8, 1, 4095, 128, 64, True),     # Llama-3-8B decode step, 4k context
    (32, 8, 1, 17, 128, 64, False),      # decode, short context (one split)
    (32, 8, 512, 0, 128, 64, True),      # prefill chunk, no prefix
    (32, 8, 100, 300, 128, 16, True),    # chunk after a prefix, B = 16
    (28, 4, 37, 50, 128, 32, True),      # g = 7, ragged tiles
    (14, 2, 9, 70, 64, 12, True),        # g = 7, B not a multiple of 16
    (8, 8, 33, 40, 128, 5, True),        # g = 1, B = 5
    (2, 1, 3, 0, 64, 16, False),         # 3 queries, no prefix (pure causal)
    # unsplit chunks: workgroups of 4 row tiles sharing K / V tiles in LDS
    (28, 4, 300, 40, 128, 48, True),     # g = 7, B not a multiple of 16
    (16, 16, 520, 20, 64, 20, True),     # g = 1, 33 row tiles (a partial workgroup)
    (32, 8, 600, 1000, 128, 64, True),   # chunk after a long prefix, B = 64
]


@pytest.mark.parametrize("h,hkv,c,p,d,b,shuffle", CASES)
def test_chunked_attention_matches_oracle(gpu, h, hkv, c, p, d, b, shuffle):
    q, kp, vp, table = _case(h, hkv, c, p, d, b, seed=h * 1000 + c + p, shuffle=shuffle)
    ref = att.chunked_attention(q, kp, vp, table, p, c, b)
    name = f"h={h} hkv={hkv} c={c} p={p} d={d} b={b}"
    print(f"[attention {name}] launching", flush=True)
    out = chunked_attention(torch.from_numpy(q).to(gpu), torch.from_numpy(kp).to(gpu),
                            torch.from_numpy(vp).to(gpu), table, p, c, b)
    torch.cuda.synchronize()
    assert out.shape == (h, c, d)
    _check(name, out.cpu().numpy(), ref, float(np.abs(vp).max()))


def test_strided_views_and_device_table(gpu):
    """q as the transposed projection output [C, H*D] -> [H, C, D], out into a
    [C, H, D] buffer through its transposed view, the pool halves as views of a
    6-D pool, a device int32 block table."""
    h, hkv, c, p, d, b, layers = 32, 8, 7, 90, 128, 16, 3
    rng = np.random.default_rng(5)
    nb = (p + c + b - 1) // b + 2
    table = [int(x) for x in rng.permutation(nb)[: (p + c + b - 1) // b]]
    k = rng.standard_normal((hkv, p + c, d)).astype(np.float32)
    v = rng.standard_normal((hkv, p + c, d)).astype(np.float32)
    kp, vp = att.fill_pool(k, v, b, table, nb)
    pool = np.zeros((nb, layers, 2, hkv, b, d), dtype=np.float32)
    pool[:, 1, 0], pool[:, 1, 1] = kp, vp
    pool_g = torch.from_numpy(pool).to(gpu)
    qflat = rng.standard_normal((c, h * d)).astype(np.float32)
    q = torch.from_numpy(qflat).to(gpu).view(c, h, d).transpose(0, 1)
    buf = torch.full((c, h, d), float("nan"), device=gpu)
    dtab = torch.tensor(table, dtype=torch.int32, device=gpu)
    out = chunked_attention(q, pool_g[:, 1, 0], pool_g[:, 1, 1], dtab, p, c, b,
                            out=buf.transpose(0, 1))
    torch.cuda.synchronize()
    ref = att.chunked_attention(qflat.reshape(c, h, d).transpose(1, 0, 2), kp, vp, table, p, c, b)
    _check("strided views", out.cpu().numpy(), ref, float(np.abs(vp).max()))
    assert not torch.isnan(buf).any()


def test_decode_sequence_matches_oracle(gpu):
    """Write-then-attend over successive decode steps (the reference generate
    loop, engine/model.py:190-203): each step writes one token's K/V and
    attends with prefix_len = its position, across block boundaries."""
    h, hkv, d, b, nb = 8, 2, 64, 16, 6
    rng = np.random.default_rng(9)
    pool = torch.zeros((nb, 1, 2, hkv, b, d), device=gpu)
    pool_np = np.zeros((nb, 1, 2, hkv, b, d), dtype=np.float32)
    table = [4, 1, 5, 0, 2, 3]
    for pos in range(0, 70, 3):
        k = rng.standard_normal((hkv, 1, d)).astype(np.float32)
        v = rng.standard_normal((hkv, 1, d)).astype(np.float32)
        q = rng.standard_normal((h, 1, d)).astype(np.float32)
        slot = table[pos // b] * b + pos % b
        att.kv_write(pool_np, 0, k, v, [slot])
        paged_kv_write(pool, 0, torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu), [slot])
        out = chunked_attention(torch.from_numpy(q).to(gpu), pool[:, 0, 0], pool[:, 0, 1], table,
                                pos, 1, b)
        ref = att.chunked_attention(q, pool_np[:, 0, 0], pool_np[:, 0, 1], table, pos, 1, b)
        torch.cuda.synchronize()
        _check(f"decode pos={pos}", out.cpu().numpy(), ref, float(np.abs(pool_np).max()))
    assert np.array_equal(pool.cpu().numpy(), pool_np)


def test_paged_kv_write_bit_exact(gpu):
    rng = np.random.default_rng(3)
    nb, layers, hkv, b, d, L = 7, 3, 4, 16, 128, 40
    pool_np = rng.standard_normal((nb, layers, 2, hkv, b, d)).astype(np.float32)
    pool = torch.from_numpy(pool_np).to(gpu)
    kflat = rng.standard_normal((L, hkv * d)).astype(np.float32)
    vflat = rng.standard_normal((L, hkv * d)).astype(np.float32)
    slots = [int(s) for s in rng.permutation(nb * b)[:L]]
    slots[5] = slots[30]            # repeated slot: token 30 wins
    slots[7] = -1                   # the pool's last slot
    slots[8] = -(nb * b)            # the pool's first slot
    # the transposed projection outputs, [1, H_kv, L, D] views
    k = torch.from_numpy(kflat).to(gpu).view(1, L, hkv, d).transpose(1, 2)
    v = torch.from_numpy(vflat).to(gpu).view(1, L, hkv, d).transpose(1, 2)
    paged_kv_write(pool, 2, k, v, slots)
    att.kv_write(pool_np, 2, kflat.reshape(L, hkv, d).transpose(1, 0, 2),
                 vflat.reshape(L, hkv, d).transpose(1, 0, 2), slots)
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy(), pool_np)


@pytest.mark.parametrize("i", range(12))
def test_paged_kv_write_random_bit_exact(gpu, i):
    """Seeded random pool shapes, layers and slot mappings -- negative slots
    and repeated slots (the later token wins) included -- bit-exact with the
    oracle's store loop."""
    rng = np.random.default_rng(500 + i)
    nb, layers, hkv = int(rng.integers(1, 9)), int(rng.integers(1, 4)), int(rng.choice([1, 2, 4, 8]))
    b, d = int(rng.choice([5, 12, 16, 64])), int(rng.choice([64, 128]))
    layer = int(rng.integers(layers))
    cap = nb * b
    L = int(rng.integers(1, 2 * cap + 1))
    slots = [int(s) for s in rng.integers(-cap, cap, size=L)]
    pool_np = rng.standard_normal((nb, layers, 2, hkv, b, d)).astype(np.float32)
    pool = torch.from_numpy(pool_np).to(gpu)
    kflat = rng.standard_normal((L, hkv * d)).astype(np.float32)
    vflat = rng.standard_normal((L, hkv * d)).astype(np.float32)
    k = torch.from_numpy(kflat).to(gpu).view(1, L, hkv, d).transpose(1, 2)
    v = torch.from_numpy(vflat).to(gpu).view(1, L, hkv, d).transpose(1, 2)
    paged_kv_write(pool, layer, k, v, slots)
    att.kv_write(pool_np, layer, kflat.reshape(L, hkv, d).transpose(1, 0, 2),
                 vflat.reshape(L, hkv, d).transpose(1, 0, 2), slots)
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy(), pool_np), (nb, layers, hkv, b, d, L)


def test_errors_mirror_the_reference(gpu):
    q = torch.zeros((6, 2, 64), device=gpu)
    kp = torch.zeros((4, 4, 16, 64), device=gpu)
    with pytest.raises(AssertionError, match="GQA requires"):
        chunked_attention(q, kp, kp, [0, 1], 0, 2, 16)
    q = torch.zeros((8, 2, 64), device=gpu)
    with pytest.raises(IndexError):
        chunked_attention(q, kp, kp, [0], 20, 2, 16)          # table too short
    with pytest.raises(IndexError):
        chunked_attention(q, kp, kp, [0, 9], 20, 2, 16)       # block outside the pool
    with pytest.raises(ValueError):
        chunked_attention(q.half(), kp, kp, [0, 1], 20, 2, 16)
    with pytest.raises(ValueError):
        chunked_attention(torch.zeros((8, 2, 80), device=gpu), torch.zeros((4, 4, 16, 80), device=gpu),
                          torch.zeros((4, 4, 16, 80), device=gpu), [0, 1], 20, 2, 16)
    pool = torch.zeros((2, 1, 2, 4, 16, 64), device=gpu)
    with pytest.raises(IndexError):
        paged_kv_write(pool, 0, torch.zeros((4, 1, 64), device=gpu),
                       torch.zeros((4, 1, 64), device=gpu), [32])
    out = chunked_attention(torch.zeros((8, 0, 64), device=gpu), kp, kp, [0], 5, 0, 16)
    assert out.shape == (8, 0, 64)


def _random_case(i: int):
    rng = np.random.default_rng(4242 + i)
    h, hkv = [(4, 4), (8, 2), (32, 8), (28, 4), (14, 2), (16, 16), (2, 1), (12, 3)][int(rng.integers(8))]
    d = int(rng.choice([64, 128]))
    b = int(rng.choice([5, 12, 16, 20, 32, 48, 64]))
    if i % 2 == 0:                                   # decode-like: few queries, long context
        c, p = int(rng.integers(1, 5)), int(rng.integers(1, 8000))
    else:                                            # chunk after a prefix
        c, p = int(rng.integers(5, 97)), int(rng.integers(0, 800))
    return h, hkv, c, p, d, b, bool(rng.random() < 0.7)


@pytest.mark.parametrize("i", range(30))
def test_random_attention_shapes(gpu, i):
    """Seeded random heads / GQA group / head dim / block size / chunk / prefix /
    block-table order against the float64 oracle, at the same bars."""
    h, hkv, c, p, d, b, shuffle = _random_case(i)
    q, kp, vp, table = _case(h, hkv, c, p, d, b, seed=7000 + i, shuffle=shuffle)
    ref = att.chunked_attention(q, kp, vp, table, p, c, b)
    name = f"random {i}: h={h} hkv={hkv} c={c} p={p} d={d} b={b} shuffle={shuffle}"
    print(f"[attention {name}] launching", flush=True)
    out = chunked_attention(torch.from_numpy(q).to(gpu), torch.from_numpy(kp).to(gpu),
                            torch.from_numpy(vp).to(gpu), table, p, c, b)
    torch.cuda.synchronize()
    assert out.shape == (h, c, d)
    _check(name, out.cpu().numpy(), ref, float(np.abs(vp).max()))
