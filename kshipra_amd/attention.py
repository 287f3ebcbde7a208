"""Paged K/V pool write and chunked attention on the GPU (fp32).

Drop-in mirrors of Kshipra's attention half of the layer loop, both running
the HIP kernels of ``csrc/kq_attention.hip`` through the C-ABI:

* ``chunked_attention(q, k_pool, v_pool, block_table, prefix_len, chunk_len,
  block_size)`` -- ``engine/chunked_prefill.py:93-140``: same arguments, same
  result ([H_q, C, D]; query i at position prefix_len + i attends causally to
  the prefix and the chunk, read in place through the block table; GQA by
  h -> h // g), same ``AssertionError`` for H_q % H_kv != 0 and ``IndexError``
  for a block table that is too short or names a block outside the pool.
* ``paged_kv_write(pool, layer, k, v, slot_mapping)`` -- the store loop of
  ``KshipraModel.forward`` (``engine/model.py:124-129``): token t's K / V of
  every KV head go to ``pool[slot // B, layer, 0 / 1, :, slot % B, :]``; a
  repeated slot keeps the last token, as the loop does; negative slots index
  from the end as Python indexing does there.

Tensors live on the GPU in float32 (the pool dtype of an fp32 model,
``engine/model.py:167-175``); the pool is [num_blocks, layers, 2, H_kv, B, D]
with D contiguous.  ``block_table`` / ``slot_mapping`` may be Python
sequences (validated on the host, then copied to the device) or device
tensors (int32 / int64) taken as they are: entries outside the pool are then
not reported (the kernels clamp or skip them to stay in bounds).
"""

from __future__ import annotations

from typing import Optional, Sequence, Union

import torch

from . import _lib

__all__ = ["chunked_attention", "paged_kv_write", "device_block_table"]

IndexLike = Union[Sequence[int], torch.Tensor]


def _require_f32(t: torch.Tensor, what: str, dims: int) -> None:
    _lib.require_device(t, what)
    if t.dtype != torch.float32:
        raise ValueError(f"{what}: float32 required, got {t.dtype}")
    if t.dim() != dims:
        raise ValueError(f"{what}: {dims}-D tensor required, got shape {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError(f"{what}: the last dimension must be contiguous")


def device_block_table(block_table: Sequence[int], num_blocks: int, needed: int,
                       device: torch.device) -> torch.Tensor:
    """int32 device copy of ``block_table[:needed]`` with the reference's
    indexing rules: an entry j < needed must exist (IndexError otherwise, as
    ``block_table[j]`` raises) and name a block of the pool, negative ids
    counting from the end (``k_pool[blk_id]``)."""
    if len(block_table) < needed:
        raise IndexError(f"block_table has {len(block_table)} entries; {needed} needed")
    ids = []
    for j in range(needed):
        b = int(block_table[j])
        if not -num_blocks <= b < num_blocks:
            raise IndexError(f"index {b} is out of bounds for dimension 0 with size {num_blocks}")
        ids.append(b + num_blocks if b < 0 else b)
    return torch.tensor(ids, dtype=torch.int32, device=device)


def chunked_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                      block_table: IndexLike, prefix_len: int, chunk_len: int, block_size: int,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """engine/chunked_prefill.py:93-140 on the GPU.

    q: [H_q, C, D]; k_pool, v_pool: [num_blocks, H_kv, B, D] (e.g. the views
    ``pool[:, i, 0]`` / ``pool[:, i, 1]``), same strides.  Returns [H_q, C, D]
    float32, written into ``out`` when given (any strides with D contiguous,
    e.g. a transposed view of a [C, H_q, D] buffer)."""
    H_q = q.shape[0]
    H_kv = k_pool.shape[1]
    assert H_q % H_kv == 0, f"GQA requires H_q ({H_q}) % H_kv ({H_kv}) == 0"
    _require_f32(q, "q", 3)
    _require_f32(k_pool, "k_pool", 4)
    _require_f32(v_pool, "v_pool", 4)
    _, C, D = q.shape
    if k_pool.shape != v_pool.shape or k_pool.stride() != v_pool.stride():
        raise ValueError("k_pool and v_pool must have the same shape and strides")
    if k_pool.shape[3] != D:
        raise ValueError(f"pool head_dim {k_pool.shape[3]} != q head_dim {D}")
    if C != chunk_len:
        raise ValueError(f"q holds {C} queries but chunk_len is {chunk_len}")
    if prefix_len < 0:
        raise ValueError("prefix_len must be >= 0")
    if not 0 < block_size <= k_pool.shape[2]:
        raise ValueError(f"block_size {block_size} must be in [1, {k_pool.shape[2]}]")
    if q.device != k_pool.device or q.device != v_pool.device:
        raise ValueError("q and the pools must be on one device")
    if out is None:
        out = torch.empty((H_q, C, D), dtype=torch.float32, device=q.device)
    else:
        _require_f32(out, "out", 3)
        if tuple(out.shape) != (H_q, C, D) or out.device != q.device:
            raise ValueError(f"out must be [{H_q}, {C}, {D}] on {q.device}")
    num_blocks = k_pool.shape[0]
    needed = (prefix_len + chunk_len + block_size - 1) // block_size
    if isinstance(block_table, torch.Tensor) and block_table.device.type == "cuda":
        if block_table.dtype != torch.int32 or block_table.dim() != 1:
            raise ValueError("a device block_table must be a 1-D int32 tensor")
        if block_table.numel() < needed:
            raise IndexError(f"block_table has {block_table.numel()} entries; {needed} needed")
        table = block_table
    else:
        table = device_block_table(block_table, num_blocks, needed, q.device)
    if C == 0:
        return out
    lib = _lib.load()
    stream = _lib.stream_of(q)
    nbytes = lib.kq_chunked_attention_workspace_bytes(H_q, H_kv, C, D, prefix_len)
    ws = _lib.workspace(q.device, stream, nbytes)
    _lib.check(lib.kq_chunked_attention_f32(
        q.data_ptr(), H_q, C, D, q.stride(0), q.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(), H_kv, num_blocks, block_size,
        k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        table.data_ptr(), table.numel(), prefix_len,
        out.data_ptr(), out.stride(0), out.stride(1), _lib.ptr(ws), nbytes, stream))
    return out


def _device_slots(slot_mapping: IndexLike, tokens: int, nslots: int,
                  device: torch.device) -> torch.Tensor:
    if isinstance(slot_mapping, torch.Tensor) and slot_mapping.device.type == "cuda":
        if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1:
            raise ValueError("a device slot_mapping must be a 1-D int64 tensor")
        if slot_mapping.numel() < tokens:
            raise IndexError(f"slot_mapping has {slot_mapping.numel()} entries; {tokens} needed")
        return slot_mapping
    if len(slot_mapping) < tokens:
        raise IndexError(f"slot_mapping has {len(slot_mapping)} entries; {tokens} needed")
    slots = []
    last = {}
    for t in range(tokens):
        s = int(slot_mapping[t])
        if not -nslots <= s < nslots:
            raise IndexError(f"slot {s} is outside the pool's {nslots} slots")
        s = s + nslots if s < 0 else s
        if s in last:
            slots[last[s]] = -1          # the reference loop's later store wins
        last[s] = t
        slots.append(s)
    return torch.tensor(slots, dtype=torch.int64, device=device)


def paged_kv_write(pool: torch.Tensor, layer: int, k: torch.Tensor, v: torch.Tensor,
                   slot_mapping: IndexLike) -> None:
    """engine/model.py:124-129: ``pool[slot // B, layer, 0, :, slot % B, :] =
    k[:, t, :]`` (and V into half 1) for each token t.

    pool: [num_blocks, layers, 2, H_kv, B, D] float32; k, v: [H_kv, L, D] or
    [1, H_kv, L, D] (any strides with D contiguous, e.g. the transposed
    projection output)."""
    _require_f32(pool, "pool", 6)
    if k.dim() == 4:
        k, v = k[0], v[0]
    _require_f32(k, "k", 3)
    _require_f32(v, "v", 3)
    nb, layers, two, H_kv, B, D = pool.shape
    if two != 2:
        raise ValueError("pool dimension 2 must hold K and V (size 2)")
    if k.shape != v.shape or k.shape[0] != H_kv or k.shape[2] != D:
        raise ValueError(f"k, v must be [{H_kv}, L, {D}], got {tuple(k.shape)}, {tuple(v.shape)}")
    if k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    if not -layers <= layer < layers:
        raise IndexError(f"layer {layer} is out of bounds for {layers} layers")
    layer = layer + layers if layer < 0 else layer
    if k.device != pool.device or v.device != pool.device:
        raise ValueError("k, v and the pool must be on one device")
    L = k.shape[1]
    if L == 0:
        return
    slots = _device_slots(slot_mapping, L, nb * B, pool.device)
    kp, vp = pool[:, layer, 0], pool[:, layer, 1]
    lib = _lib.load()
    _lib.check(lib.kq_paged_kv_write_f32(
        k.data_ptr(), v.data_ptr(), L, H_kv, D, k.stride(1), k.stride(0), slots.data_ptr(),
        kp.data_ptr(), vp.data_ptr(), nb, B, kp.stride(0), kp.stride(1), kp.stride(2),
        _lib.stream_of(pool)))
