"""Host-side KV-cache bookkeeping (include/flour_cache.h), no GPU.

The cases restate the reference's own unit tests with their numbers:
  BlockAllocator / BlockTable: src/models/common/paged.rs tests
      allocator_hands_out_distinct_blocks_then_exhausts, allocator_refcounts_govern_when_a_block_is_freed,
      block_table_maps_logical_positions_to_physical_slots, block_table_exposes_blocks_and_clears
  Cache prefix reuse and sizing: src/models/common/cache.rs tests
      allocate_kv_overflow_past_max_seq_len_errors, match_prefix_is_empty_before_anything_is_registered,
      register_then_match_reuses_full_blocks_and_leaves_a_suffix,
      match_prefix_leaves_last_block_when_prompt_is_block_aligned,
      reset_sequence_frees_unregistered_blocks_but_keeps_registered_ones
(The caches here hold bookkeeping only, device_pool=False.)
"""
from __future__ import annotations

import pytest

from flour_amd import _lib
from flour_amd.kv_cache import BlockAllocator, BlockTable, KvCache


def host_cache(max_seq_len: int, **kw) -> KvCache:
    import torch

    return KvCache(num_layers=2, max_seq_len=max_seq_len, num_heads=4, kv_heads=2, head_dim=4,
                   dtype=torch.float32, block_size=16, device_pool=False, **kw)


# ---------------------------------------------------------------- paged.rs
def test_allocator_hands_out_distinct_blocks_then_exhausts():
    alloc = BlockAllocator(2)
    assert alloc.num_free() == 2
    a, b = alloc.allocate(), alloc.allocate()
    assert a != b
    assert alloc.allocate() is None
    assert alloc.decref(a)
    assert alloc.num_free() == 1
    assert alloc.allocate() == a


def test_allocator_first_block_is_zero_and_lifo():
    alloc = BlockAllocator(3)
    assert [alloc.allocate() for _ in range(3)] == [0, 1, 2]
    alloc.decref(1)
    alloc.decref(2)
    assert alloc.allocate() == 2  # last freed, first reused


def test_allocator_refcounts_govern_when_a_block_is_freed():
    alloc = BlockAllocator(2)
    assert alloc.num_free() == 2
    a = alloc.allocate()
    assert alloc.ref_count(a) == 1
    alloc.incref(a)
    assert alloc.ref_count(a) == 2
    assert not alloc.decref(a)  # still referenced
    assert alloc.num_free() == 1
    assert alloc.decref(a)
    assert alloc.ref_count(a) == 0
    assert alloc.num_free() == 2
    assert alloc.allocate() == a


def test_allocator_rejects_unreferenced_decref():
    alloc = BlockAllocator(1)
    with pytest.raises(_lib.FlourError, match="unreferenced"):
        alloc.decref(0)
    with pytest.raises(_lib.FlourError):
        alloc.incref(5)


def test_block_table_maps_logical_positions_to_physical_slots():
    table = BlockTable(2)
    assert table.is_empty()
    table.push_block(5)
    table.push_block(3)
    assert table.capacity() == 4
    assert [table.slot(p) for p in range(4)] == [10, 11, 6, 7]
    table.advance(3)
    assert table.len() == 3
    assert table.slots(0, 3) == [10, 11, 6]


def test_block_table_exposes_blocks_and_clears():
    table = BlockTable(2)
    table.push_block(5)
    table.push_block(3)
    table.advance(3)
    assert table.blocks() == [5, 3]
    assert table.block_at(0) == 5 and table.block_at(1) == 3
    table.clear()
    assert table.is_empty() and table.len() == 0
    assert table.blocks() == []
    assert table.block_size() == 2


def test_block_table_rejects_unmapped_positions():
    table = BlockTable(4)
    table.push_block(1)
    with pytest.raises(_lib.FlourError):
        table.slot(4)
    with pytest.raises(_lib.FlourError):
        table.slots(2, 6)


# ---------------------------------------------------------------- cache.rs
def test_allocate_kv_overflow_past_max_seq_len_errors():
    cache = host_cache(16)
    with pytest.raises(_lib.FlourError, match="paged kv cache overflow") as e:
        cache.allocate_kv(17)
    assert e.value.code == _lib.ERR_CAPACITY
    cache.allocate_kv(16)
    assert cache.len() == 16 and cache.capacity() == 16


def test_allocate_kv_grows_block_by_block_and_slots_follow_the_table():
    cache = host_cache(64)
    cache.allocate_kv(2)
    assert cache.blocks() == [0] and cache.len() == 2
    cache.allocate_kv(15)  # 17 live tokens -> a second block
    assert cache.blocks() == [0, 1]
    assert cache.slots(0, 17) == list(range(17))
    assert cache.free_blocks() == 2


def test_match_prefix_is_empty_before_anything_is_registered():
    cache = host_cache(64)
    cache.reset_sequence()
    assert cache.match_prefix(list(range(40))) == 0


def test_register_then_match_reuses_full_blocks_and_leaves_a_suffix():
    cache = host_cache(64)
    ids = list(range(40))  # 2 full blocks + 8
    cache.reset_sequence()
    assert cache.match_prefix(ids) == 0
    cache.allocate_kv(40)
    cache.register_prefix(ids)
    first = cache.blocks()
    cache.reset_sequence()
    assert cache.match_prefix(ids) == 32
    assert cache.blocks() == first[:2]  # the same physical blocks are shared
    assert cache.len() == 32
    cache.allocate_kv(8)  # the suffix gets a fresh block
    assert cache.blocks()[:2] == first[:2] and len(cache.blocks()) == 3


def test_match_prefix_leaves_last_block_when_prompt_is_block_aligned():
    cache = host_cache(64)
    ids = list(range(32))
    cache.reset_sequence()
    cache.match_prefix(ids)
    cache.allocate_kv(32)
    cache.register_prefix(ids)
    cache.reset_sequence()
    assert cache.match_prefix(ids) == 16


def test_match_prefix_stops_at_the_first_different_block():
    cache = host_cache(64)
    ids = list(range(40))
    cache.allocate_kv(40)
    cache.register_prefix(ids)
    cache.reset_sequence()
    other = ids[:16] + [999] + ids[17:]
    assert cache.match_prefix(other) == 16  # block 1 differs: its chained hash differs


def test_reset_sequence_frees_unregistered_blocks_but_keeps_registered_ones():
    cache = host_cache(64)
    ids = list(range(40))
    cache.reset_sequence()
    cache.match_prefix(ids)
    cache.allocate_kv(40)  # 3 blocks: 2 full + 1 partial
    cache.register_prefix(ids)
    free_after_first = cache.free_blocks()
    b = cache.blocks()
    assert [cache.ref_count(x) for x in b] == [2, 2, 1]
    cache.reset_sequence()
    assert cache.free_blocks() == free_after_first + 1  # the partial block returns
    assert [cache.ref_count(x) for x in b[:2]] == [1, 1]


def test_clear_prefix_cache_releases_registry_only_blocks():
    cache = host_cache(64)
    ids = list(range(40))
    cache.allocate_kv(40)
    cache.register_prefix(ids)
    cache.reset_sequence()
    assert cache.free_blocks() == 2  # 4 blocks, 2 held by the registry
    cache.clear_prefix_cache()
    assert cache.free_blocks() == 4
    assert cache.match_prefix(ids) == 0


def test_out_of_blocks_when_the_registry_holds_them():
    cache = host_cache(32)  # 2 blocks
    ids = list(range(20))
    cache.allocate_kv(20)
    cache.register_prefix(ids)  # 1 full block kept by the registry
    cache.reset_sequence()
    with pytest.raises(_lib.FlourError, match="out of kv blocks") as e:
        cache.allocate_kv(32)
    assert e.value.code == _lib.ERR_OUT_OF_BLOCKS


def test_device_operations_need_a_device_pool():
    cache = host_cache(16)
    cache.allocate_kv(1)
    lib = _lib.lib()
    rc = lib.flour_kv_cache_write_kv(cache._h, 0, None, None, 1, 4, 4, None)
    assert rc == _lib.ERR_UNSUPPORTED and "device pool" in _lib.last_error()
