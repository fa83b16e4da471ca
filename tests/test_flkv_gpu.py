"""FLKV bundle export / import through the device pool (flour_kv_cache_export_bundle /
import_bundle): the frame is compared byte for byte with the oracle's encoding of the same pool
contents (oracle/flkv.py over host copies of the pools), and imports are checked block by block.

Restates the reference's cache tests cache.rs:728-889 (export captures the real block K/V;
import round-trips values and enables prefix reuse; mismatched prompt and dimension mismatch
are rejected without partial state; unaligned and oversized exports are rejected), then a
Llama-3-8B-shaped bundle (32 layers, 8 kv heads, head_dim 128, bf16, a 1,024-token prefix:
128 MiB, two staging chunks): export == oracle, import -> export reproduces the frame, and
attention over the imported prefix equals attention over the original.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import flkv as F
from _util import to_np
from flour_amd import _lib
from flour_amd.kv_cache import KvCache

pytestmark = pytest.mark.gpu

NAME = {torch.float32: "F32", torch.bfloat16: "BF16", torch.float16: "F16"}


def small_cache(head_dim=4):
    """prefix_config of the reference tests: 2 layers, kv_heads 2, head_dim 4, block 16."""
    return KvCache(2, 64, 2, 2, head_dim, torch.float32, 16)


def fill(cache, n, offset, device):
    cache.reset_sequence()
    cache.allocate_kv(n)
    for layer in range(cache.num_layers):
        m = cache.kv_heads * n * cache.head_dim
        k = (torch.arange(m, dtype=torch.float32) + layer * 1000 + offset).reshape(1, cache.kv_heads, n, cache.head_dim)
        cache.write_kv(layer, k.to(device), (k + 0.5).to(device))
    torch.cuda.synchronize()


def oracle_frame(cache, model_id, ids, count):
    ks, vs = zip(*[tuple(to_np(t) for t in cache.pool(l)) for l in range(cache.num_layers)])
    return F.export_frame(model_id, ids, count, list(ks), list(vs), cache.blocks(),
                          cache.block_size, NAME[cache.dtype])


def test_export_captures_real_block_kv(device):
    """cache.rs:728-781."""
    c = small_cache()
    fill(c, 32, 0, device)
    ids = list(range(32))
    data = c.export_prefix_bundle("m", ids, 32)
    meta, blocks = F.decode(data, np.float32)
    assert meta == {"model_id": "m", "token_count": 32, "token_ids": ids, "block_size": 16,
                    "num_layers": 2, "num_kv_heads": 2, "head_dim": 4, "dtype": "F32"}
    for layer in range(2):
        kp, vp = (to_np(t) for t in c.pool(layer))
        for b, phys in enumerate(c.blocks()):
            assert np.array_equal(blocks[b][layer][0], kp[:, phys * 16:(phys + 1) * 16])
            assert np.array_equal(blocks[b][layer][1], vp[:, phys * 16:(phys + 1) * 16])
    assert data == oracle_frame(c, "m", ids, 32)


def test_import_round_trips_values_and_enables_reuse(device):
    """cache.rs:787-825."""
    a = small_cache()
    fill(a, 32, 0.125, device)
    data = a.export_prefix_bundle("m", list(range(32)), 32)
    b = small_cache()
    b.allocate_kv(16)       # a live sequence the import replaces
    prompt = list(range(40))
    assert b.import_prefix_bundle(data, prompt) == 32
    assert b.len() == 32
    for layer in range(2):
        ka, va = (to_np(t) for t in a.pool(layer))
        kb, vb = (to_np(t) for t in b.pool(layer))
        for pa, pb in zip(a.blocks(), b.blocks()):
            assert np.array_equal(ka[:, pa * 16:(pa + 1) * 16], kb[:, pb * 16:(pb + 1) * 16])
            assert np.array_equal(va[:, pa * 16:(pa + 1) * 16], vb[:, pb * 16:(pb + 1) * 16])
    b.reset_sequence()
    assert b.match_prefix(prompt) == 32
    assert b.export_prefix_bundle("m", list(range(32)), 32) == data


def test_import_rejections_leave_no_partial_state(device):
    """cache.rs:829-851: a mismatched prompt prefix, and a head_dim mismatch."""
    a = small_cache()
    fill(a, 32, 0.0, device)
    data = a.export_prefix_bundle("m", list(range(32)), 32)
    b = small_cache()
    free = b.free_blocks()
    wrong = list(range(100, 140))
    with pytest.raises(_lib.FlourError, match="prompt does not start with bundle token ids"):
        b.import_prefix_bundle(data, wrong)
    b.reset_sequence()
    assert b.match_prefix(wrong) == 0 and b.free_blocks() == free
    c = small_cache(head_dim=8)
    with pytest.raises(_lib.FlourError, match="bundle head_dim 4 != model 8"):
        c.import_prefix_bundle(data, list(range(40)))


def test_export_rejects_unaligned_or_oversized_count(device):
    """cache.rs:855-866."""
    c = small_cache()
    fill(c, 32, 0.0, device)
    with pytest.raises(_lib.FlourError, match="not aligned to block size 16"):
        c.export_prefix_bundle("m", [0] * 32, 20)
    with pytest.raises(_lib.FlourError, match="exceeds live len 32"):
        c.export_prefix_bundle("m", [0] * 48, 48)


def test_llama3_8b_shaped_bundle_round_trip(device):
    L, G, D, P = 32, 8, 128, 1024
    a = KvCache(L, P + 64, 32, G, D, torch.bfloat16, 16)
    a.allocate_kv(P)
    g = torch.Generator(device="cpu").manual_seed(21)
    for layer in range(L):
        k = torch.randn((P, G, D), generator=g).to(torch.bfloat16).to(device)
        v = torch.randn((P, G, D), generator=g).to(torch.bfloat16).to(device)
        a.write_kv(layer, k, v)
    torch.cuda.synchronize()
    ids = list(range(7, 7 + P))
    data = a.export_prefix_bundle("meta-llama/Meta-Llama-3-8B", ids, P)
    assert len(data) > 128 << 20
    assert data == oracle_frame(a, "meta-llama/Meta-Llama-3-8B", ids, P)
    b = KvCache(L, P + 64, 32, G, D, torch.bfloat16, 16)
    assert b.import_prefix_bundle(data, ids + [1, 2, 3]) == P
    assert b.export_prefix_bundle("meta-llama/Meta-Llama-3-8B", ids, P) == data
    # one more row on both caches, then decode attention over the whole sequence
    k1 = torch.randn((1, G, D), generator=g).to(torch.bfloat16).to(device)
    v1 = torch.randn((1, G, D), generator=g).to(torch.bfloat16).to(device)
    q = torch.randn((1, 32, 1, D), generator=g).to(torch.bfloat16).to(device)
    outs = []
    for c in (a, b):
        c.allocate_kv(1)
        c.write_kv(5, k1, v1)
        outs.append(c.attention(5, q, D ** -0.5, out_dtype=torch.float32))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
