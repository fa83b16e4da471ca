"""Many sequences over one pool (flour_kv_batch_*), bookkeeping on the CPU.

Each sequence behaves as the reference's KvCache (cache.rs allocate_kv, reset_sequence,
match_prefix, register_prefix; paged.rs BlockAllocator LIFO order and refcounts); what is new is
that the allocator and the prefix registry are shared, so one sequence reuses the full prefix
blocks another registered, and removing a sequence returns only the blocks nobody else holds.
"""
from __future__ import annotations

import pytest
import torch

from flour_amd import _lib
from flour_amd.kv_cache import KvBatch


def batch(num_blocks=8, max_seqs=3, max_seq_len=64, tokens=256):
    return KvBatch(2, num_blocks, max_seqs, max_seq_len, tokens, 2, 2, 4, torch.float32, 16,
                   device_pool=False)


def test_sequences_share_the_allocator():
    b = batch()
    s0, s1 = b.add_sequence(), b.add_sequence()
    b.allocate_kv(s0, 40)          # 3 blocks; the free list hands out 0, 1, 2 first
    b.allocate_kv(s1, 17)          # 2 blocks
    assert b.blocks(s0) == [0, 1, 2] and b.blocks(s1) == [3, 4]
    assert b.free_blocks() == 3 and b.len(s0) == 40 and b.len(s1) == 17
    b.remove_sequence(s0)          # LIFO: the last freed block comes back first
    assert b.free_blocks() == 6
    s2 = b.add_sequence()
    assert s2 == s0
    b.allocate_kv(s2, 1)
    assert b.blocks(s2) == [2]


def test_prefix_shared_across_sequences():
    b = batch()
    ids = list(range(40))
    a = b.add_sequence()
    b.allocate_kv(a, 40)
    b.register_prefix(a, ids)      # 2 full blocks registered
    c = b.add_sequence()
    assert b.match_prefix(c, ids) == 32
    assert b.blocks(c) == b.blocks(a)[:2] and b.len(c) == 32
    assert [b.ref_count(x) for x in b.blocks(a)] == [3, 3, 1]
    b.remove_sequence(a)           # the registry and c still hold the shared blocks
    assert [b.ref_count(x) for x in b.blocks(c)] == [2, 2] and b.free_blocks() == 6
    b.remove_sequence(c)
    assert b.free_blocks() == 6    # registry-only blocks stay cached
    b.clear_prefix_cache()
    assert b.free_blocks() == 8
    # a block-aligned prompt leaves its last block to compute (cache.rs:112-140)
    d = b.add_sequence()
    assert b.match_prefix(d, ids[:32]) == 0


def test_errors():
    b = batch(num_blocks=4, max_seqs=2)
    s0, s1 = b.add_sequence(), b.add_sequence()
    with pytest.raises(_lib.FlourError, match="all 2 sequence slots"):
        b.add_sequence()
    with pytest.raises(_lib.FlourError, match="paged kv cache overflow"):
        b.allocate_kv(s0, 65)
    b.allocate_kv(s0, 48)
    with pytest.raises(_lib.FlourError, match="out of kv blocks"):
        b.allocate_kv(s1, 32)
    with pytest.raises(_lib.FlourError, match="no live sequence 7"):
        b.allocate_kv(7, 1)
    with pytest.raises(_lib.FlourError, match="needs an empty sequence"):
        b.match_prefix(s0, range(48))
    b.remove_sequence(s1)
    with pytest.raises(_lib.FlourError, match="no live sequence 1"):
        b.len(s1)


def test_plan_validation():
    b = batch()
    s0, s1 = b.add_sequence(), b.add_sequence()
    b.allocate_kv(s0, 10)
    b.allocate_kv(s1, 5)
    with pytest.raises(_lib.FlourError, match="listed twice"):
        b.plan([s0, s0], [1, 1])
    with pytest.raises(_lib.FlourError, match="brings 6 new rows over 5"):
        b.plan([s0, s1], [1, 6])
    with pytest.raises(_lib.FlourError, match="exceed max_batch_tokens 8"):
        batch_small = batch(tokens=8)
        t = batch_small.add_sequence()
        batch_small.allocate_kv(t, 10)
        batch_small.plan([t], [10])
    with pytest.raises(_lib.FlourError, match="no device pool"):
        b.plan([s0, s1], [10, 5])


def test_step_checks_everything_before_allocating():
    """flour_kv_batch_step = allocate_kv on every listed sequence + plan; each refusal below
    leaves lengths, tables and the free list unchanged."""
    b = batch(num_blocks=4, max_seqs=3, max_seq_len=64, tokens=40)
    s0, s1 = b.add_sequence(), b.add_sequence()
    b.allocate_kv(s0, 16)          # one full block: its next row needs a new block
    b.allocate_kv(s1, 20)

    def state():
        return [b.len(s0), b.len(s1)], [b.blocks(s0), b.blocks(s1)], b.free_blocks()

    before = state()
    for ids, q, what in [([s0, s0], [1, 1], "listed twice"),
                         ([s0, 2], [1, 1], "no live sequence 2"),
                         ([s0, s1], [1, 0], "brings 0 new rows"),
                         ([s0, s1], [1, 45], "exceeds max_seq_len 64"),
                         ([s0, s1], [30, 11], "exceed max_batch_tokens 40"),
                         ([s0, s1], [17, 13], "out of kv blocks"),   # needs 2 + 1 > 1 free
                         ([s0, s1], [1, 1], "no device pool")]:       # all checks passed
        with pytest.raises(_lib.FlourError, match=what):
            b.step(ids, q)
        assert state() == before, what


def test_block_list_query_needs_a_buffer_for_a_positive_capacity():
    """flour_kv_batch_blocks reports the count with no buffer only when cap is 0; a null buffer
    with room claimed is refused, not written through."""
    import ctypes

    b = batch()
    s = b.add_sequence()
    b.allocate_kv(s, 20)
    n = ctypes.c_int(-1)
    assert _lib.lib().flour_kv_batch_blocks(b._h, s, None, 4, ctypes.byref(n)) == \
        _lib.ERR_INVALID_ARGUMENT
    assert _lib.lib().flour_kv_batch_blocks(b._h, s, None, 0, ctypes.byref(n)) == _lib.OK
    assert n.value == 2


def test_error_message_is_cleared_by_the_next_successful_call():
    """flour_hip_last_error describes the last failing call of this thread; every entry point
    clears it first, so a success leaves it empty."""
    b = batch()
    s = b.add_sequence()
    b.allocate_kv(s, 32)
    with pytest.raises(_lib.FlourError, match="register_prefix over 1000 full blocks"):
        b.register_prefix(s, list(range(16000)))
    assert _lib.lib().flour_hip_last_error().decode().startswith(
        "kv_batch: register_prefix over 1000 full blocks")
    b.allocate_kv(s, 1)
    assert _lib.lib().flour_hip_last_error().decode() == ""
