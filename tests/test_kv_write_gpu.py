"""Kernel (1) parity: the KV-cache write is bit-exact with the oracle's scatter
(PagedKvPool::write, src/models/common/paged.rs:186-204) on identical seeded inputs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from _util import to_np
from flour_amd import ops
from flour_amd.workloads import make_prefill, make_workload

pytestmark = pytest.mark.gpu


def _check_write(k, v, k_pool, v_pool, slot_mapping):
    """Run the kernel on device copies and the oracle on host copies; compare bits."""
    kp_ref, vp_ref = to_np(k_pool).copy(), to_np(v_pool).copy()
    O.kv_write_scatter(to_np(k), to_np(v), kp_ref, vp_ref, to_np(slot_mapping),
                       bf16=(k.dtype != torch.float16))
    ops.kv_write(k, v, k_pool, v_pool, slot_mapping)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(k_pool), kp_ref)
    assert np.array_equal(to_np(v_pool), vp_ref)


@pytest.mark.parametrize("name", ["prefill_bf16_varlen_llama3_8b", "prefill_bf16_prefix_qwen2_7b"])
def test_kv_write_workload_bit_exact(device, name):
    c = make_workload(name, device=device)
    print(f"{name}: tokens={c.k_new.shape[0]} pool_blocks={c.meta['pool_blocks']}", flush=True)
    _check_write(c.k_new, c.v_new, c.k_pool, c.v_pool, c.slot_mapping)
    # the slot mapping holds no padding: every new row is in place
    kp = c.k_pool.float()
    sm = c.slot_mapping.long()
    assert torch.equal(kp[:, sm, :].transpose(0, 1), c.k_new.float())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("G,D", [(8, 128), (2, 64), (1, 4), (3, 3), (4, 256)])
def test_kv_write_dtypes_and_shapes(device, dtype, G, D):
    g = torch.Generator(device=device).manual_seed(G * 1000 + D)
    T, num_slots = 37, 160
    k = torch.randn((T, G, D), generator=g, device=device).to(dtype)
    v = torch.randn((T, G, D), generator=g, device=device).to(dtype)
    kp = torch.randn((G, num_slots, D), generator=g, device=device).to(dtype)
    vp = torch.randn((G, num_slots, D), generator=g, device=device).to(dtype)
    perm = torch.randperm(num_slots, generator=torch.Generator().manual_seed(D))[:T].to(torch.int32)
    perm[5] = -1  # padding token: skipped
    perm[9] = -7
    _check_write(k, v, kp, vp, perm.to(device))


def test_kv_write_reference_layout_view(device):
    """k in the reference's (kv_heads, seq, head_dim) layout, passed as a transposed view."""
    g = torch.Generator(device=device).manual_seed(3)
    G, S, D, num_slots = 4, 50, 128, 256
    k_ref = torch.randn((G, S, D), generator=g, device=device).to(torch.bfloat16)
    v_ref = torch.randn((G, S, D), generator=g, device=device).to(torch.bfloat16)
    kp = torch.zeros((G, num_slots, D), dtype=torch.bfloat16, device=device)
    vp = torch.zeros_like(kp)
    sm = torch.randperm(num_slots)[:S].to(torch.int32).to(device)
    _check_write(k_ref.transpose(0, 1), v_ref.transpose(0, 1), kp, vp, sm)


def test_kv_write_decode_step_and_empty(device):
    """A decode step writes one row per sequence; zero tokens is a no-op."""
    c = make_prefill(num_seqs=4, num_heads=8, kv_heads=2, head_dim=128, block_size=16,
                     q_len=(1, 1), device=device, seed=9)
    _check_write(c.k_new, c.v_new, c.k_pool, c.v_pool, c.slot_mapping)
    before = c.k_pool.clone()
    ops.kv_write(c.k_new[:0], c.v_new[:0], c.k_pool, c.v_pool, c.slot_mapping[:0])
    torch.cuda.synchronize()
    assert torch.equal(before, c.k_pool)


def test_kv_write_quirk_mapping_follows_scatter(device):
    """A mapping whose run start equals its slot (the paged.rs:196 quirk): the kernel writes
    the documented scatter, which differs from the literal reference loop."""
    G, S, D, num_slots = 2, 6, 128, 64
    sl = np.array([0, 40, 7, 33, 21, 50], np.int32)
    assert O.kv_write_quirk_index(sl.astype(np.uint32)) == 0
    g = torch.Generator(device=device).manual_seed(5)
    k = torch.randn((S, G, D), generator=g, device=device).to(torch.bfloat16)
    v = torch.randn((S, G, D), generator=g, device=device).to(torch.bfloat16)
    kp = torch.zeros((G, num_slots, D), dtype=torch.bfloat16, device=device)
    vp = torch.zeros_like(kp)
    _check_write(k, v, kp, vp, torch.from_numpy(sl).to(device))
    kr = np.zeros((G, num_slots, D), np.uint16)
    vr = np.zeros_like(kr)
    O.kv_write_reference_loop(to_np(k).transpose(1, 0, 2), to_np(v).transpose(1, 0, 2), kr, vr,
                              sl.astype(np.uint32))
    assert not np.array_equal(kr, to_np(kp))


def test_kv_write_rejects_bad_arguments(device):
    k = torch.zeros((4, 2, 8), device=device)
    kp = torch.zeros((2, 16, 8), device=device)
    with pytest.raises(Exception):
        ops.kv_write(k, k, kp, kp, torch.zeros(3, dtype=torch.int32, device=device))
    with pytest.raises(Exception):
        ops.kv_write(k, k, kp.to(torch.bfloat16), kp.to(torch.bfloat16),
                     torch.zeros(4, dtype=torch.int32, device=device))
