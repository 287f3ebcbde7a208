"""CPU-only checks of the attention entry points' host side: the workspace
plan, argument validation before any launch, the reference-style index
handling of block tables and slot mappings, and the header's citations.
No GPU is touched (every C-ABI call here fails validation on the host)."""

from __future__ import annotations

import os

import pytest
import torch

from kshipra_amd import _lib
from kshipra_amd.attention import _device_slots, chunked_attention, device_block_table, paged_kv_write

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kshipra_quant.h")
CPU = torch.device("cpu")


def test_workspace_plan():
    lib = _lib.load()
    ws = lib.kq_chunked_attention_workspace_bytes
    # Llama-3-8B decode at 4096 keys: 8 KV heads x one row tile -> 256 key
    # splits of one 16-key tile, each keeping (acc[128], m, l) per query row
    assert ws(32, 8, 1, 128, 4095) == 256 * 32 * 1 * 130 * 4
    # 16384 keys: still 256 splits (the cap), of 4 tiles each
    assert ws(32, 8, 1, 128, 16383) == 256 * 32 * 1 * 130 * 4
    # 1024 keys: 64 one-tile splits
    assert ws(32, 8, 1, 128, 1023) == 64 * 32 * 1 * 130 * 4
    # short context: a single split, no workspace
    assert ws(32, 8, 1, 128, 10) == 0
    # prefill chunks: >= 512 row-tile waves run unsplit (8 x 128 at 512 tokens)
    assert ws(32, 8, 4096, 128, 0) == 0
    assert ws(32, 8, 512, 128, 3584) == 0
    # a 64-token chunk (8 x 16 row tiles) still splits its keys
    assert ws(32, 8, 64, 128, 1000) > 0
    # invalid shapes report 0 (the entry point rejects them)
    assert ws(6, 4, 1, 128, 100) == 0
    assert ws(32, 8, 0, 128, 100) == 0


A16 = 1 << 12     # an aligned dummy address, never dereferenced


@pytest.mark.parametrize("args", [
    # head_dim 80
    (A16, 32, 1, 80, 80, 80, A16, A16, 8, 4, 16, 1024, 128, 80, A16, 2, 10, A16, 80, 80, None, 0, None),
    # q_heads % kv_heads
    (A16, 30, 1, 128, 128, 128, A16, A16, 8, 4, 16, 1024, 128, 128, A16, 2, 10, A16, 128, 128, None, 0, None),
    # table too short for prefix 40 + chunk 1 at B = 16
    (A16, 32, 1, 128, 128, 128, A16, A16, 8, 4, 16, 1024, 128, 128, A16, 2, 40, A16, 128, 128, None, 0, None),
    # misaligned q
    (A16 + 4, 32, 1, 128, 128, 128, A16, A16, 8, 4, 16, 1024, 128, 128, A16, 2, 10, A16, 128, 128, None, 0,
     None),
    # stride not a multiple of 4
    (A16, 32, 1, 128, 130, 128, A16, A16, 8, 4, 16, 1024, 128, 128, A16, 2, 10, A16, 128, 128, None, 0, None),
    # negative prefix
    (A16, 32, 1, 128, 128, 128, A16, A16, 8, 4, 16, 1024, 128, 128, A16, 2, -1, A16, 128, 128, None, 0, None),
])
def test_attention_argument_errors(args):
    lib = _lib.load()
    assert lib.kq_chunked_attention_f32(*args) == _lib.KQ_ERR_ARG
    assert lib.kq_last_error() not in (None, b"")


def test_attention_missing_workspace():
    lib = _lib.load()
    st = lib.kq_chunked_attention_f32(A16, 32, 1, 128, 128, 128, A16, A16, 8, 100, 64, 1 << 20, 8192,
                                      128, A16, 64, 4095, A16, 128, 128, None, 0, None)
    assert st == _lib.KQ_ERR_WORKSPACE


def test_kv_write_argument_errors():
    lib = _lib.load()
    f = lib.kq_paged_kv_write_f32
    assert f(A16, A16, 4, 8, 126, 1008, 126, A16, A16, A16, 4, 16, 1 << 16, 2048, 128, None) == _lib.KQ_ERR_ARG
    assert f(None, A16, 4, 8, 128, 1024, 128, A16, A16, A16, 4, 16, 1 << 16, 2048, 128, None) == _lib.KQ_ERR_ARG
    assert f(A16, A16, 4, 8, 128, 1024, 128, A16, A16, A16, 0, 16, 1 << 16, 2048, 128, None) == _lib.KQ_ERR_ARG
    assert f(A16 + 8, A16, 4, 8, 128, 1024, 128, A16, A16, A16, 4, 16, 1 << 16, 2048, 128,
             None) == _lib.KQ_ERR_ARG


def test_block_table_follows_python_indexing():
    t = device_block_table([3, -1, 0, 7], num_blocks=5, needed=3, device=CPU)
    assert t.dtype == torch.int32 and t.tolist() == [3, 4, 0]      # -1 -> the last block
    with pytest.raises(IndexError):
        device_block_table([0, 1], num_blocks=5, needed=3, device=CPU)
    with pytest.raises(IndexError):
        device_block_table([0, 5], num_blocks=5, needed=2, device=CPU)
    with pytest.raises(IndexError):
        device_block_table([0, -6], num_blocks=5, needed=2, device=CPU)


def test_slot_mapping_last_store_wins_and_wraps():
    s = _device_slots([5, 9, 5, -1, 79], tokens=5, nslots=80, device=CPU)
    # token 0's slot 5 is stored again by token 2; -1 is slot 79, stored again by token 4
    assert s.tolist() == [-1, 9, 5, -1, 79]
    with pytest.raises(IndexError):
        _device_slots([80], tokens=1, nslots=80, device=CPU)
    with pytest.raises(IndexError):
        _device_slots([-81], tokens=1, nslots=80, device=CPU)
    with pytest.raises(IndexError):
        _device_slots([1, 2], tokens=3, nslots=80, device=CPU)


def test_python_api_errors_on_the_host():
    kp = torch.zeros((4, 4, 16, 64))
    with pytest.raises(AssertionError, match="GQA requires"):
        chunked_attention(torch.zeros((6, 1, 64)), kp, kp, [0], 0, 1, 16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        chunked_attention(torch.zeros((8, 1, 64)), kp, kp, [0], 0, 1, 16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        paged_kv_write(torch.zeros((2, 1, 2, 4, 16, 64)), 0, torch.zeros((4, 1, 64)),
                       torch.zeros((4, 1, 64)), [0])


def test_header_cites_the_reference():
    text = open(HEADER).read()
    for name, ref in (("kq_paged_kv_write_f32", "engine/model.py"),
                      ("kq_chunked_attention_f32", "engine/chunked_prefill.py")):
        block = text[:text.index(name + "(")].rsplit("/*", 1)[-1]
        assert ref in block, name
