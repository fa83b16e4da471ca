"""Device side of the host KV cache (include/flour_cache.h): write_kv lands bit-exactly at the
table's slots, and attention through the cache (kv_blocks + paged_attention in one call)
matches the oracle, for prefill, decode and a prefix-cached suffix.

The first cases restate src/models/common/cache.rs tests write_kv_then_blocks_spans_appended_batches,
write_kv_across_two_layers_shares_positions and kv_blocks_round_trips_written_values.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O
from _util import errors, to_np
from flour_amd.kv_cache import KvCache

pytestmark = pytest.mark.gpu


def pools_np(cache, layer):
    k, v = cache.pool(layer)
    torch.cuda.synchronize()
    return to_np(k), to_np(v)


def test_kv_blocks_round_trips_written_values(device):
    cache = KvCache(2, 16, num_heads=2, kv_heads=2, head_dim=4, dtype=torch.float32)
    cache.allocate_kv(2)
    k = torch.arange(16, dtype=torch.float32, device=device).view(1, 2, 2, 4)
    cache.write_kv(0, k, k)
    kp, vp = pools_np(cache, 0)
    slots = cache.slots(0, 2)
    want = to_np(k)[0]  # (heads, seq, D)
    assert np.array_equal(kp[:, slots, :], want) and np.array_equal(vp[:, slots, :], want)


def test_write_kv_spans_appended_batches_and_layers(device):
    g = torch.Generator(device="cpu").manual_seed(7)
    cache = KvCache(2, 64, num_heads=4, kv_heads=2, head_dim=8, dtype=torch.bfloat16)
    want = {0: [], 1: []}
    for n in (2, 1, 20):  # a second and third batch extend the live window
        cache.allocate_kv(n)
        for layer in (0, 1):  # allocate once, both layers write the same positions
            k = torch.randn(1, 2, n, 8, generator=g).to(torch.bfloat16).to(device)
            v = torch.randn(1, 2, n, 8, generator=g).to(torch.bfloat16).to(device)
            cache.write_kv(layer, k, v)
            want[layer].append((to_np(k)[0], to_np(v)[0]))
    assert cache.len() == 23
    slots = cache.slots(0, 23)
    for layer in (0, 1):
        kp, vp = pools_np(cache, layer)
        wk = np.concatenate([a for a, _ in want[layer]], axis=1)
        wv = np.concatenate([b for _, b in want[layer]], axis=1)
        assert np.array_equal(kp[:, slots, :], wk) and np.array_equal(vp[:, slots, :], wv)


def attention_ref(cache, layer, q_np, seq_q):
    """Oracle over the cache's own pool and table: rows = the last seq_q live positions."""
    kp, vp = pools_np(cache, layer)
    table = np.array([cache.blocks()], dtype=np.int32)
    q_rows = np.ascontiguousarray(q_np[0].transpose(1, 0, 2))  # (seq, H, D)
    cu = np.array([0, seq_q], np.int32)
    kl = np.array([cache.len()], np.int32)
    return O.paged_attention(q_rows, kp, vp, table, cu, kl, cache.block_size,
                             1.0 / math.sqrt(q_np.shape[-1]))  # (seq, H, D) fp64-accumulated


@pytest.mark.parametrize("H,G,D", [(32, 8, 128), (8, 2, 64)])
def test_prefill_then_decode_through_the_cache(device, H, G, D):
    g = torch.Generator(device="cpu").manual_seed(11)
    cache = KvCache(1, 512, num_heads=H, kv_heads=G, head_dim=D, dtype=torch.bfloat16)
    scale = 1.0 / math.sqrt(D)

    def step(n):
        cache.allocate_kv(n)
        k = torch.randn(1, G, n, D, generator=g).to(torch.bfloat16).to(device)
        v = torch.randn(1, G, n, D, generator=g).to(torch.bfloat16).to(device)
        q = torch.randn(1, H, n, D, generator=g).to(torch.bfloat16).to(device)
        cache.write_kv(0, k, v)
        out = cache.attention(0, q, scale, out_dtype=torch.float32)
        torch.cuda.synchronize()
        ref = attention_ref(cache, 0, to_np(q), n)
        got = to_np(out)[0].transpose(1, 0, 2)
        ma, rl = errors(got, ref)
        assert ma <= 2e-3 and rl <= 1e-3, (n, ma, rl)

    step(300)  # prefill
    for _ in range(3):  # decode steps
        step(1)
    step(40)  # a chunked continuation (suffix prefill over the cached rows)


def test_prefix_cached_suffix_matches_cold_prefill(device):
    """The attention-level form of the reference's prefix-reuse invariant (model.rs:244-360):
    a suffix attending to shared prefix blocks equals the same rows of a cold full prefill."""
    g = torch.Generator(device="cpu").manual_seed(5)
    H, G, D, L = 8, 2, 128, 72
    ids = list(range(1000, 1000 + L))
    k = torch.randn(1, G, L, D, generator=g).to(torch.bfloat16).to(device)
    v = torch.randn(1, G, L, D, generator=g).to(torch.bfloat16).to(device)
    q = torch.randn(1, H, L, D, generator=g).to(torch.bfloat16).to(device)
    scale = 1.0 / math.sqrt(D)
    cache = KvCache(1, 256, num_heads=H, kv_heads=G, head_dim=D, dtype=torch.bfloat16)
    cache.reset_sequence()
    assert cache.match_prefix(ids) == 0
    cache.allocate_kv(L)
    cache.write_kv(0, k, v)
    cold = cache.attention(0, q, scale, out_dtype=torch.float32)
    cache.register_prefix(ids)
    first_blocks = cache.blocks()

    cache.reset_sequence()
    m = cache.match_prefix(ids)
    assert m == 64 and cache.blocks() == first_blocks[:4]
    cache.allocate_kv(L - m)
    cache.write_kv(0, k[:, :, m:].contiguous(), v[:, :, m:].contiguous())
    warm = cache.attention(0, q[:, :, m:].contiguous(), scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ma, rl = errors(to_np(warm), to_np(cold)[:, :, m:])
    assert ma <= 1e-5 and rl <= 1e-6, (ma, rl)
