"""The reference's closed-form known answer (src/backend/cpu.rs:244-262) through the C-ABI on
every attention path: one head, two positions, q = k = 1, v = [10, 20], scale 1. Position 0
sees only itself (exactly 10); position 1 sees two equal scores (exactly the mean, 15).

head_dim 1 is the reference's own shape and runs on the generic kernel. The matrix-core and
vector-ALU kernels need 16-byte rows, so the same answer is embedded in dim 0 of wider rows
(every other dim 0): the scores, weights and outputs of dim 0 are those of the KAT, and the
other dims are exactly 0. Every path must return exactly [10, 15] (all values are exact in
bf16, fp16 and fp32, and equal scores give weights of exactly 1).
"""
from __future__ import annotations

import pytest
import torch

from flour_amd import ops

pytestmark = pytest.mark.gpu


def _pools(dtype, head_dim, block_size, device):
    """One kv head, one block holding positions 0 and 1 at slots 0 and 1."""
    k_pool = torch.zeros((1, block_size, head_dim), dtype=dtype, device=device)
    v_pool = torch.zeros_like(k_pool)
    k_pool[0, 0, 0] = 1.0
    k_pool[0, 1, 0] = 1.0
    v_pool[0, 0, 0] = 10.0
    v_pool[0, 1, 0] = 20.0
    table = torch.zeros((1, 1), dtype=torch.int32, device=device)
    return k_pool, v_pool, table


def _expect(out, rows):
    want = torch.zeros_like(out, dtype=torch.float32)
    for i, x in enumerate(rows):
        want[i, 0, 0] = x
    assert torch.equal(out.float(), want), out[:, 0, :4]


@pytest.mark.parametrize("dtype,head_dim,block_size,path", [
    (torch.float32, 1, 2, "generic kernel, the reference's head_dim 1 and block of 2"),
    (torch.float32, 64, 16, "vector-ALU kernel"),
    (torch.bfloat16, 64, 16, "vector-ALU kernel, 16-bit pool"),
    (torch.bfloat16, 128, 16, "matrix-core prefill (fp16 P.V over widened V)"),
    (torch.float16, 128, 16, "matrix-core prefill, fp16 pool"),
])
def test_kat_prefill_both_positions(device, dtype, head_dim, block_size, path):
    k_pool, v_pool, table = _pools(dtype, head_dim, block_size, device)
    q = torch.zeros((2, 1, head_dim), dtype=dtype, device=device)
    q[:, 0, 0] = 1.0
    cu = torch.tensor([0, 2], dtype=torch.int32, device=device)
    kv = torch.tensor([2], dtype=torch.int32, device=device)
    for out_dtype in (torch.float32, dtype):
        out = ops.varlen_prefill(q, k_pool, v_pool, cu, kv, table, 2, 1.0, block_size=block_size,
                                 out_dtype=out_dtype)
        torch.cuda.synchronize()
        print(f"KAT prefill {path} out {out_dtype}: {out[:, 0, 0].tolist()}", flush=True)
        _expect(out, [10.0, 15.0])


@pytest.mark.parametrize("dtype,head_dim,block_size", [
    (torch.float32, 1, 2),
    (torch.float32, 64, 16),
    (torch.bfloat16, 64, 16),
    (torch.bfloat16, 128, 16),
    (torch.float16, 128, 16),
])
def test_kat_decode_each_position(device, dtype, head_dim, block_size):
    """Decode of position 0 (context 1) and of position 1 (context 2) as a batch of two."""
    k_pool, v_pool, table = _pools(dtype, head_dim, block_size, device)
    q = torch.zeros((2, 1, head_dim), dtype=dtype, device=device)
    q[:, 0, 0] = 1.0
    tables = table.expand(2, 1).contiguous()
    ctx = torch.tensor([1, 2], dtype=torch.int32, device=device)
    out = ops.paged_decode(q, k_pool, v_pool, tables, ctx, 1.0, 2, block_size=block_size,
                           out_dtype=torch.float32)
    torch.cuda.synchronize()
    print(f"KAT decode {dtype} D{head_dim}: {out[:, 0, 0].tolist()}", flush=True)
    _expect(out, [10.0, 15.0])
