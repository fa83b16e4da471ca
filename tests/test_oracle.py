"""Pins the CPU oracle (oracle/flour_oracle.c) before it is trusted as the checker.

Each check follows a reference test or a fact the mathematics fixes:
  * reference KATs: cpu.rs:244-262 ([10, 15]), paged.rs:287-306 (scatter / gather),
    paged.rs:308-331 (full-block write / view), paged.rs:377-395 (slot mapping);
  * the reference's paged == dense property tests (cpu.rs:190-242) against an fp64 brute force
    and against torch's scaled_dot_product_attention (an independent library routine);
  * closed forms: one visible key returns its V row, equal scores return the mean of V,
    constant V returns that constant (softmax weights sum to one);
  * invariance under physical-block permutation and under block size;
  * planted mistakes (oracle_set_mutation) must each be caught by these checks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle as O

from _util import bf16_bits_to_f32, f32_to_bf16_bits


def pool_from_dense(k, v, block_size, perm_seed=None, pool_factor=1.0):
    """Reference layout k, v (G, kv_len, D) -> pools (G, num_slots, D) + block table."""
    G, L, D = k.shape
    nblk = max(1, math.ceil(L / block_size))
    pool_blocks = max(nblk, math.ceil(pool_factor * nblk))
    ids = np.arange(pool_blocks)
    if perm_seed is not None:
        ids = np.random.default_rng(perm_seed).permutation(pool_blocks)
    bt = ids[:nblk].astype(np.int32)[None, :]
    num_slots = pool_blocks * block_size
    kp = np.zeros((G, num_slots, D), k.dtype)
    vp = np.zeros((G, num_slots, D), v.dtype)
    for j in range(L):
        s = bt[0, j // block_size] * block_size + j % block_size
        kp[:, s] = k[:, j]
        vp[:, s] = v[:, j]
    return kp, vp, bt


def run_paged(q_ref, k, v, block_size, scale, perm_seed=None, **kw):
    """q_ref (H, Sq, D), k/v (G, kv_len, D) in the reference layout -> (H, Sq, D)."""
    H, Sq, D = q_ref.shape
    kp, vp, bt = pool_from_dense(k, v, block_size, perm_seed)
    q = np.ascontiguousarray(q_ref.transpose(1, 0, 2))
    out = O.paged_attention(q, kp, vp, bt, np.array([0, Sq]), np.array([k.shape[1]]),
                            block_size, scale, **kw)
    return out.transpose(1, 0, 2)


def run_dense64(q_ref, k, v, scale):
    H, Sq, D = q_ref.shape
    kp, vp, bt = pool_from_dense(k, v, 4)
    q = np.ascontiguousarray(q_ref.transpose(1, 0, 2))
    out = O.dense_attention_f64(q, kp, vp, bt, np.array([0, Sq]), np.array([k.shape[1]]), 4, scale)
    return out.transpose(1, 0, 2)


def torch_sdpa64(q_ref, k, v, scale):
    """Independent library check: torch SDPA in fp64 with the reference's causal offset."""
    H, Sq, D = q_ref.shape
    G, L, _ = k.shape
    rep = H // G
    qt = torch.from_numpy(q_ref.astype(np.float64))[None]
    kt = torch.from_numpy(k.astype(np.float64)).repeat_interleave(rep, 0)[None]
    vt = torch.from_numpy(v.astype(np.float64)).repeat_interleave(rep, 0)[None]
    i = torch.arange(Sq)[:, None]
    j = torch.arange(L)[None, :]
    allowed = j <= (L - Sq) + i
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=allowed,
                                                           scale=scale)
    return out[0].numpy()


def rnd(shape, seed):
    return np.random.default_rng(seed).uniform(-1, 1, shape).astype(np.float32)


# ------------------------------------------------------------------ reference KATs

def test_kat_weighted_average_cpu_rs_244():
    # cpu.rs:244-262: 1 head, 2 positions, head_dim 1, q = k = 1, v = [10, 20], scale 1.
    q = np.array([[[1.0], [1.0]]], np.float32)
    k = np.array([[[1.0], [1.0]]], np.float32)
    v = np.array([[[10.0], [20.0]]], np.float32)
    for bs in (1, 2, 16):
        out = run_paged(q, k, v, bs, 1.0)
        assert abs(out[0, 0, 0] - 10.0) < 1e-6
        assert abs(out[0, 1, 0] - 15.0) < 1e-6


def test_kat_scatter_then_gather_paged_rs_287():
    # 1 kv head, head_dim 2, 4 slots; tokens written to slots [2, 0], gathered as [0, 2].
    k = np.array([[[1, 2]], [[3, 4]]], np.float32)  # (T=2, G=1, D=2)
    v = np.array([[[5, 6]], [[7, 8]]], np.float32)
    kp = np.zeros((1, 4, 2), np.float32)
    vp = np.zeros((1, 4, 2), np.float32)
    assert O.kv_write_scatter(k, v, kp, vp, np.array([2, 0])) == 0
    assert kp[0, [0, 2]].ravel().tolist() == [3, 4, 1, 2]
    assert vp[0, [0, 2]].ravel().tolist() == [7, 8, 5, 6]
    # the literal reference loop agrees on this mapping (no run starts at its own slot)
    kr = np.zeros_like(kp)
    vr = np.zeros_like(vp)
    assert O.kv_write_reference_loop(k.transpose(1, 0, 2), v.transpose(1, 0, 2), kr, vr,
                                     np.array([2, 0], np.uint32)) == 0
    assert np.array_equal(kr, kp) and np.array_equal(vr, vp)


def test_kat_full_block_write_paged_rs_308():
    # A full block of 2 slots written into physical block 1 (slots 2..3); block 0 stays zero.
    k = np.array([[[1, 2]], [[3, 4]]], np.float32)
    v = np.array([[[5, 6]], [[7, 8]]], np.float32)
    kp = np.zeros((1, 4, 2), np.float32)
    vp = np.zeros((1, 4, 2), np.float32)
    O.kv_write_scatter(k, v, kp, vp, np.array([2, 3]))
    assert kp[0, 2:4].ravel().tolist() == [1, 2, 3, 4]
    assert vp[0, 2:4].ravel().tolist() == [5, 6, 7, 8]
    assert kp[0, 0:2].ravel().tolist() == [0, 0, 0, 0]


def test_kat_slot_mapping_paged_rs_377():
    blocks = [5, 3]
    assert [O.slot(blocks, 2, p) for p in range(4)] == [10, 11, 6, 7]
    assert O.slots(blocks, 2, 0, 3).tolist() == [10, 11, 6]


def test_reference_write_loop_quirk_paged_rs_196():
    """Run start i with slots[i] == i extends the run to the end of the batch."""
    G, S, D = 1, 3, 2
    k = np.arange(G * S * D, dtype=np.float32).reshape(G, S, D) + 1
    v = -k
    sl = np.array([0, 9, 5], np.uint32)  # token 0 -> slot 0: the quirk fires at i = 0
    assert O.kv_write_quirk_index(sl) == 0
    kr = np.zeros((G, 16, D), np.float32)
    vr = np.zeros_like(kr)
    assert O.kv_write_reference_loop(k, v, kr, vr, sl) == 0
    # reference wrote tokens 0,1,2 contiguously to slots 0,1,2 ...
    assert np.array_equal(kr[0, 0:3], k[0])
    assert not kr[0, [5, 9]].any()
    # ... while the documented scatter puts them at 0, 9, 5
    ks = np.zeros_like(kr)
    vs = np.zeros_like(vr)
    O.kv_write_scatter(np.ascontiguousarray(k.transpose(1, 0, 2)),
                       np.ascontiguousarray(v.transpose(1, 0, 2)), ks, vs, sl.astype(np.int32))
    assert np.array_equal(ks[0, [0, 9, 5]], k[0])
    # a run that would end past num_slots is rejected, as candle's slice_set would
    small = np.zeros((G, 2, D), np.float32)
    assert O.kv_write_reference_loop(k, v, small, small.copy(), sl) == -1


def test_reference_loop_matches_scatter_without_fixed_points():
    rng = np.random.default_rng(7)
    G, S, D, num_slots = 2, 40, 8, 128
    for _ in range(20):
        sl = rng.permutation(num_slots)[:S].astype(np.uint32)
        if O.kv_write_quirk_index(sl) >= 0:
            continue
        k = rng.standard_normal((G, S, D)).astype(np.float32)
        v = rng.standard_normal((G, S, D)).astype(np.float32)
        kr = np.zeros((G, num_slots, D), np.float32)
        vr = np.zeros_like(kr)
        ks, vs = kr.copy(), vr.copy()
        assert O.kv_write_reference_loop(k, v, kr, vr, sl) == 0
        O.kv_write_scatter(np.ascontiguousarray(k.transpose(1, 0, 2)),
                           np.ascontiguousarray(v.transpose(1, 0, 2)), ks, vs, sl.astype(np.int32))
        assert np.array_equal(kr, ks) and np.array_equal(vr, vs)


def test_scatter_skips_padding_and_out_of_range():
    k = np.ones((3, 1, 4), np.float32)
    kp = np.zeros((1, 8, 4), np.float32)
    vp = np.zeros_like(kp)
    assert O.kv_write_scatter(k, k, kp, vp, np.array([-1, 3, 8])) == 1
    assert kp[0, 3].tolist() == [1, 1, 1, 1]
    assert kp.sum() == 4


# ------------------------------------------------------------------ paged == dense (cpu.rs:190-242)

@pytest.mark.parametrize("H,G,Sq,L,D,bs", [
    (2, 2, 5, 5, 4, 2),    # prefill, partial last block (cpu.rs:190-206)
    (2, 2, 1, 7, 4, 3),    # decode step, q-len 1, kv 7 (cpu.rs:208-224)
    (4, 2, 6, 6, 4, 4),    # GQA 4 q / 2 kv heads (cpu.rs:226-242)
    (4, 1, 3, 19, 8, 4),   # suffix over a cached prefix (offset 16)
    (8, 2, 1, 300, 64, 16),
])
def test_paged_matches_dense_fp64_and_torch(H, G, Sq, L, D, bs):
    q = rnd((H, Sq, D), 1)
    k = rnd((G, L, D), 2)
    v = rnd((G, L, D), 3)
    scale = 1 / math.sqrt(D)
    paged = run_paged(q, k, v, bs, scale)
    dense = run_dense64(q, k, v, scale)
    ref = torch_sdpa64(q, k, v, scale)
    assert np.max(np.abs(dense - ref)) < 1e-12  # fp64 brute force == library routine
    assert np.max(np.abs(paged - dense)) < 1e-5  # fp32 restatement within fp32 rounding


def test_closed_forms():
    rng = np.random.default_rng(11)
    H, G, L, D = 2, 1, 9, 8
    q = rng.standard_normal((H, L, D)).astype(np.float32)
    k = rng.standard_normal((G, L, D)).astype(np.float32)
    v = rng.standard_normal((G, L, D)).astype(np.float32)
    out = run_paged(q, k, v, 4, 0.3)
    # query 0 of a cold prefill sees only key 0: output is exactly V[0]
    assert np.array_equal(out[:, 0], np.repeat(v[:, 0], H, axis=0))
    # equal scores (q = 0): output is the mean of the visible V rows
    out0 = run_paged(np.zeros_like(q), k, v, 4, 0.3)
    for i in range(L):
        assert np.allclose(out0[0, i], v[0, : i + 1].mean(0), atol=1e-6)
    # constant V: softmax weights sum to one
    out1 = run_paged(q, k, np.full_like(v, 2.5), 4, 0.3)
    assert np.allclose(out1, 2.5, atol=1e-6)


def test_block_permutation_and_size_invariance():
    H, G, Sq, L, D = 4, 2, 5, 70, 16
    q, k, v = rnd((H, Sq, D), 4), rnd((G, L, D), 5), rnd((G, L, D), 6)
    base = run_paged(q, k, v, 16, 0.25)
    for seed in (1, 2, 3):  # same logical cache in other physical blocks: bit-identical
        assert np.array_equal(run_paged(q, k, v, 16, 0.25, perm_seed=seed), base)
    for bs in (1, 3, 7, 32):
        assert np.max(np.abs(run_paged(q, k, v, bs, 0.25) - base)) < 2e-6


def test_bf16_storage_is_widened_exactly():
    rng = np.random.default_rng(9)
    H, G, Sq, L, D = 4, 2, 3, 40, 32
    q = f32_to_bf16_bits(rng.standard_normal((H, Sq, D)).astype(np.float32))
    k = f32_to_bf16_bits(rng.standard_normal((G, L, D)).astype(np.float32))
    v = f32_to_bf16_bits(rng.standard_normal((G, L, D)).astype(np.float32))
    a = run_paged(q, k, v, 16, 0.2)
    b = run_paged(bf16_bits_to_f32(q), bf16_bits_to_f32(k), bf16_bits_to_f32(v), 16, 0.2)
    # same values, separately vectorised loops: equal up to fp32 summation order (a widening
    # mistake such as truncating or mis-shifting the bits would be off by >= 1e-2)
    assert np.max(np.abs(a - b)) < 1e-6


def test_conversions_match_torch_and_numpy():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3e38, -1e-40],
                                 np.float32)])
    bf = O.f32_to_bf16(x)
    tb = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf, tb)
    assert np.array_equal(O.bf16_to_f32(bf), bf16_bits_to_f32(bf))
    xf = x[np.abs(x) < 60000]
    hf = O.f32_to_f16(xf)
    assert np.array_equal(hf, xf.astype(np.float16).view(np.uint16))
    assert np.array_equal(O.f16_to_f32(hf), xf.astype(np.float16).astype(np.float32))


# ------------------------------------------------------------------ planted mistakes

def _battery() -> list[str]:
    """The pinning checks above, condensed; returns the names of those that fail."""
    failed = []
    q = np.array([[[1.0], [1.0]]], np.float32)
    out = run_paged(q, q.copy(), np.array([[[10.0], [20.0]]], np.float32), 1, 1.0)
    if abs(out[0, 0, 0] - 10) > 1e-6 or abs(out[0, 1, 0] - 15) > 1e-6:
        failed.append("kat")
    for (H, G, Sq, L, D, bs) in [(4, 2, 3, 19, 8, 4), (2, 2, 5, 5, 4, 2)]:
        qq, k, v = rnd((H, Sq, D), 1), rnd((G, L, D), 2) * 3, rnd((G, L, D), 3)
        if np.max(np.abs(run_paged(qq, k, v, bs, 0.35) - torch_sdpa64(qq, k, v, 0.35))) > 1e-5:
            failed.append(f"sdpa{H}{G}{Sq}{L}")
    if [O.slot([5, 3], 2, p) for p in range(4)] != [10, 11, 6, 7]:
        failed.append("slots")
    return failed


def test_battery_passes_on_faithful_oracle():
    O.set_mutation(O.MUT_NONE)
    assert _battery() == []


@pytest.mark.parametrize("mut", [O.MUT_MASK_OFF_BY_ONE, O.MUT_NO_CORRECTION, O.MUT_WRONG_KV_HEAD,
                                 O.MUT_NO_SCALE, O.MUT_OFFSET_ZERO, O.MUT_SLOT_SWAP])
def test_planted_mistake_is_caught(mut):
    O.set_mutation(mut)
    try:
        assert _battery() != [], f"mutation {mut} slipped through the pinning checks"
    finally:
        O.set_mutation(O.MUT_NONE)
