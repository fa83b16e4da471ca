"""Writes the golden fixtures of tests/golden/ (run from the repository root:
``python tests/golden/make_golden.py``).

The reference (a Rust crate over candle 0.9.2) cannot be built or run here, so the expected
outputs come from an independent implementation of the same mathematics: torch's
scaled_dot_product_attention in float64 on the CPU, over the dense K/V gathered from the paged
pool, with the reference's causal rule (query i of q_len rows sees kv position j iff
j <= kv_len - q_len + i, src/backend/cpu.rs:68, :88-95) and head mapping (h -> h // n_rep,
cpu.rs:5-13). The KV-write expectation is numpy fancy-index assignment (the scatter of
src/models/common/paged.rs:186-187). Inputs are bf16 (stored as uint16 bit patterns), drawn
from numpy's PCG64 with the seeds below. Expected attention outputs are stored as float32
(rounded from float64).
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def widen(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def paged_case(rng, q_lens, kv_lens, H, G, D, bs, pool_factor=1.25):
    nblk = [math.ceil(k / bs) for k in kv_lens]
    pool_blocks = math.ceil(pool_factor * sum(nblk))
    perm = rng.permutation(pool_blocks).astype(np.int32)
    max_blocks = max(nblk)
    bt = np.zeros((len(kv_lens), max_blocks), np.int32)
    pos = 0
    for s, n in enumerate(nblk):
        bt[s, :n] = perm[pos:pos + n]
        pos += n
    num_slots = pool_blocks * bs
    k_pool = np.zeros((G, num_slots, D), np.uint16)
    v_pool = np.zeros((G, num_slots, D), np.uint16)
    for s, L in enumerate(kv_lens):
        for j in range(L):
            slot = bt[s, j // bs] * bs + j % bs
            k_pool[:, slot] = bf16_bits(rng.standard_normal((G, D)))
            v_pool[:, slot] = bf16_bits(rng.standard_normal((G, D)))
    q = bf16_bits(rng.standard_normal((sum(q_lens), H, D)))
    return q, k_pool, v_pool, bt


def expected_attention(q, k_pool, v_pool, bt, q_lens, kv_lens, bs, scale):
    H, n_rep = q.shape[1], q.shape[1] // k_pool.shape[0]
    out = np.zeros(q.shape, np.float64)
    row = 0
    for s, (ql, L) in enumerate(zip(q_lens, kv_lens)):
        slots = [bt[s, j // bs] * bs + j % bs for j in range(L)]
        k = torch.from_numpy(widen(k_pool[:, slots]).astype(np.float64))  # (G, L, D)
        v = torch.from_numpy(widen(v_pool[:, slots]).astype(np.float64))
        k = k.repeat_interleave(n_rep, dim=0)  # head h reads kv head h // n_rep
        v = v.repeat_interleave(n_rep, dim=0)
        qq = torch.from_numpy(widen(q[row:row + ql]).astype(np.float64)).transpose(0, 1)
        off = L - ql
        mask = torch.arange(L)[None, :] <= (off + torch.arange(ql))[:, None]
        o = torch.nn.functional.scaled_dot_product_attention(qq, k, v, attn_mask=mask,
                                                             scale=scale)
        out[row:row + ql] = o.transpose(0, 1).numpy()
        row += ql
    return out


def main():
    # decode: one query per sequence, GQA 4, head_dim 64, contexts that end inside a block
    rng = np.random.default_rng(20240611)
    kv = [1, 17, 80, 47]
    q, kp, vp, bt = paged_case(rng, [1] * 4, kv, H=8, G=2, D=64, bs=16)
    exp = expected_attention(q, kp, vp, bt, [1] * 4, kv, 16, 1 / 8)
    np.savez_compressed(HERE / "decode_gqa4_d64.npz", q=q, k_pool=kp, v_pool=vp,
                        block_tables=bt, context_lens=np.array(kv, np.int32), scale=1 / 8,
                        block_size=16, expected=exp.astype(np.float32))

    # prefill: packed sequences, the second and third over a 32-token prefix (kv_len > q_len)
    rng = np.random.default_rng(20240612)
    ql, kv = [16, 9, 24], [16, 41, 56]
    q, kp, vp, bt = paged_case(rng, ql, kv, H=4, G=2, D=128, bs=16)
    exp = expected_attention(q, kp, vp, bt, ql, kv, 16, 1 / math.sqrt(128))
    cu = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
    np.savez_compressed(HERE / "prefill_gqa2_d128.npz", q=q, k_pool=kp, v_pool=vp,
                        block_tables=bt, cu_seqlens_q=cu, kv_lens=np.array(kv, np.int32),
                        scale=1 / math.sqrt(128), block_size=16, expected=exp.astype(np.float32))

    # KV write: 12 tokens into a 64-slot pool, two padding tokens (-1), and a run start whose
    # token index equals its slot (the case the reference's run loop at paged.rs:196 mishandles)
    rng = np.random.default_rng(20240613)
    G, D, T, num_slots = 2, 32, 12, 64
    k = bf16_bits(rng.standard_normal((T, G, D)))
    v = bf16_bits(rng.standard_normal((T, G, D)))
    slots = rng.permutation(num_slots)[:T].astype(np.int32)
    slots[3] = 3
    slots[5] = -1
    slots[9] = -1
    k_pool = bf16_bits(rng.standard_normal((G, num_slots, D)))
    v_pool = bf16_bits(rng.standard_normal((G, num_slots, D)))
    k_exp, v_exp = k_pool.copy(), v_pool.copy()
    keep = slots >= 0
    k_exp[:, slots[keep]] = k[keep].transpose(1, 0, 2)
    v_exp[:, slots[keep]] = v[keep].transpose(1, 0, 2)
    np.savez_compressed(HERE / "kv_write_scatter.npz", k=k, v=v, slot_mapping=slots,
                        k_pool=k_pool, v_pool=v_pool, k_expected=k_exp, v_expected=v_exp)


if __name__ == "__main__":
    main()
