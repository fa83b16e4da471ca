"""RoPE + KV write (flour_hip_rope_kv_write) parity: bit-exact against the oracle's restatement
(oracle_rope_kv_write, attention.rs:96-104 — rope(q), rope(k), write_kv) on identical seeded
inputs: the rotated q rows, and the K and V pools. Covered: bf16 / f16 / f32, several sequences
at different positions, q rotated in place, the reference's head-major layout as strided views,
padding slots and positions outside the table, the one-pair-per-lane path for unaligned shapes,
the full Llama-3-8B-shaped varlen batch, and the prefill kernel run on the rotated rows.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from _util import errors, to_np
from flour_amd import ops
from flour_amd.workloads import make_prefill, make_workload

pytestmark = pytest.mark.gpu

TDT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def oracle_of(q, k, v, k_pool, v_pool, slots, positions, cos, sin, q_out_init=None):
    """Oracle result on host copies of the device inputs: (q_out, k_pool, v_pool) arrays."""
    kp, vp = to_np(k_pool).copy(), to_np(v_pool).copy()
    qo = to_np(q if q_out_init is None else q_out_init).copy()
    qo, _ = O.rope_kv_write(to_np(q), to_np(k), to_np(v), kp, vp, to_np(slots),
                            to_np(positions), to_np(cos), to_np(sin),
                            bf16=(q.dtype == torch.bfloat16), q_out=qo)
    return qo, kp, vp


def inputs(dt, T, H, G, D, num_slots, seed, device, max_pos=8192, theta=500000.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn((T, H, D), generator=g).to(TDT[dt]).to(device)
    k = torch.randn((T, G, D), generator=g).to(TDT[dt]).to(device)
    v = torch.randn((T, G, D), generator=g).to(TDT[dt]).to(device)
    k_pool = torch.randn((G, num_slots, D), generator=g).to(TDT[dt]).to(device)  # stale rows
    v_pool = torch.randn((G, num_slots, D), generator=g).to(TDT[dt]).to(device)
    slots = torch.randperm(num_slots, generator=g)[:T].to(torch.int32).to(device)
    cos, sin = ops.rope_tables(max_pos, D, theta, TDT[dt], device)
    return q, k, v, k_pool, v_pool, slots, cos, sin


def varlen_positions(lens, starts, device):
    return torch.cat([torch.arange(s, s + n, dtype=torch.int32) for n, s in zip(lens, starts)]).to(device)


@pytest.mark.parametrize("dt,H,G,D", [("bf16", 32, 8, 128), ("f16", 28, 4, 128),
                                      ("f32", 8, 8, 64), ("bf16", 8, 2, 64)])
def test_matches_oracle_bit_exact(device, dt, H, G, D):
    lens, starts = [70, 1, 129], [0, 4095, 1000]   # prefill, a decode step, a continuation
    T = sum(lens)
    q, k, v, kp, vp, slots, cos, sin = inputs(dt, T, H, G, D, 512, 11, device)
    pos = varlen_positions(lens, starts, device)
    ref = oracle_of(q, k, v, kp, vp, slots, pos, cos, sin)
    q_out = ops.rope_kv_write(q, k, v, kp, vp, slots, pos, cos, sin)
    torch.cuda.synchronize()
    for got, want, name in zip((q_out, kp, vp), ref, ("q", "k_pool", "v_pool")):
        assert np.array_equal(to_np(got), want), f"{dt} {name} differs from the oracle"


def test_in_place_and_reference_layout(device):
    """q rotated in place; q, k, v handed over in the reference's (heads, seq, head_dim)
    layout (attention.rs:92-94) as transposed views."""
    T, H, G, D = 45, 16, 4, 128
    q, k, v, kp, vp, slots, cos, sin = inputs("bf16", T, H, G, D, 128, 12, device)
    pos = torch.arange(300, 300 + T, dtype=torch.int32, device=device)
    q_hm = q.transpose(0, 1).contiguous()   # (H, T, D)
    k_hm, v_hm = k.transpose(0, 1).contiguous(), v.transpose(0, 1).contiguous()
    ref = oracle_of(q, k, v, kp, vp, slots, pos, cos, sin)
    qv = q_hm.transpose(0, 1)
    out = ops.rope_kv_write(qv, k_hm.transpose(0, 1), v_hm.transpose(0, 1), kp, vp, slots, pos,
                            cos, sin, q_out=qv)
    torch.cuda.synchronize()
    assert out.data_ptr() == q_hm.data_ptr()
    assert np.array_equal(to_np(q_hm.transpose(0, 1)), ref[0])
    assert np.array_equal(to_np(kp), ref[1]) and np.array_equal(to_np(vp), ref[2])


def test_padding_slots_and_positions_outside_the_table(device):
    T, H, G, D = 8, 4, 2, 64
    q, k, v, kp, vp, slots, cos, sin = inputs("bf16", T, H, G, D, 64, 13, device, max_pos=100)
    slots = torch.tensor([5, -1, 64, 7, 9, 11, 13, 15], dtype=torch.int32, device=device)
    pos = torch.tensor([0, 3, 4, -1, 100, 99, 50, 2], dtype=torch.int32, device=device)
    sentinel = torch.full_like(q, 7.0)
    ref = oracle_of(q, k, v, kp, vp, slots, pos, cos, sin, q_out_init=sentinel)
    q_out = sentinel.clone()
    ops.rope_kv_write(q, k, v, kp, vp, slots, pos, cos, sin, q_out=q_out)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(q_out), ref[0])
    assert np.array_equal(to_np(kp), ref[1]) and np.array_equal(to_np(vp), ref[2])
    assert bool((q_out[3:5] == 7.0).all()) and not bool((q_out[1] == 7.0).all())


@pytest.mark.parametrize("D,offset", [(6, 0), (128, 1)])
def test_one_pair_per_lane_path(device, D, offset):
    """Rows whose halves or bases are not 16-byte aligned (head_dim 6; views starting one
    element in) take the one-pair-per-lane kernel, with the same results."""
    T, H, G = 9, 4, 2
    q, k, v, kp, vp, slots, cos, sin = inputs("f16", T, H, G, D, 32, 14, device)
    if offset:
        buf = torch.zeros(q.numel() + offset, dtype=q.dtype, device=device)
        buf[offset:] = q.reshape(-1)
        q = buf[offset:].view(T, H, D)
    pos = torch.arange(T, dtype=torch.int32, device=device) * 37
    ref = oracle_of(q, k, v, kp, vp, slots, pos, cos, sin)
    q_out = ops.rope_kv_write(q, k, v, kp, vp, slots, pos, cos, sin)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(q_out), ref[0])
    assert np.array_equal(to_np(kp), ref[1]) and np.array_equal(to_np(vp), ref[2])


def prefill_positions(c, device):
    cu = c.cu_seqlens_q.cpu().tolist()
    kl = c.kv_lens.cpu().tolist()
    lens = [cu[s + 1] - cu[s] for s in range(len(kl))]
    starts = [kl[s] - lens[s] for s in range(len(kl))]
    return varlen_positions(lens, starts, device)


def test_full_varlen_batch_llama3_8b_shape(device):
    """The 8-sequence U[256, 2048] Llama-3-8B-shaped batch (9,625 tokens), bit for bit."""
    c = make_workload("prefill_bf16_varlen_llama3_8b", device=device)
    cos, sin = ops.rope_tables(4096, 128, 500000.0, torch.bfloat16, device)
    pos = prefill_positions(c, device)
    ref = oracle_of(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.slot_mapping, pos, cos, sin)
    q_out = ops.rope_kv_write(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.slot_mapping, pos,
                              cos, sin)
    torch.cuda.synchronize()
    assert np.array_equal(to_np(q_out), ref[0])
    assert np.array_equal(to_np(c.k_pool), ref[1]) and np.array_equal(to_np(c.v_pool), ref[2])


def test_prefill_on_rotated_rows_matches_oracle(device):
    """rope_kv_write, then the prefill kernel over the cache (with a shared cached prefix):
    the order of attention.rs:96-109, against the oracle's rope and paged_attention."""
    c = make_prefill(3, 16, 4, 128, 16, (1, 1), prefix=64, dtype=torch.bfloat16, seed=15,
                     device=device, q_lens=[100, 1, 257])
    cos, sin = ops.rope_tables(1024, 128, 10000.0, torch.bfloat16, device)
    pos = prefill_positions(c, device)
    q_ref, kp_ref, vp_ref = oracle_of(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool,
                                      c.slot_mapping, pos, cos, sin)
    q_rot = ops.rope_kv_write(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.slot_mapping, pos,
                              cos, sin)
    out = ops.varlen_prefill(q_rot, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                             c.block_tables, c.max_seqlen_q, c.scale, block_size=c.block_size,
                             out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.paged_attention(q_ref, kp_ref, vp_ref, to_np(c.block_tables), to_np(c.cu_seqlens_q),
                            to_np(c.kv_lens), c.block_size, c.scale, bf16=True)
    max_abs, rel = errors(to_np(out), ref)
    print(f"rope + prefill: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3
