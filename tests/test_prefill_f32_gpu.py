"""fp32 causal varlen prefill on the fp32 matrix cores (head_dim 64 and 128) against the oracle's
restatement of paged_attention (src/backend/cpu.rs:57-112): max-abs <= 1e-5 on fp32 output,
16-bit outputs exactly the round-to-nearest-even of the fp32 result, zero rows where a
sequence's kv length is below its query count, and the same bounds at the fp32 benchmark
batch's full size."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from _util import errors, f32_to_bf16_bits, to_np
from flour_amd import _lib, ops
from flour_amd.workloads import make_prefill, make_workload

pytestmark = pytest.mark.gpu


def _run(c, out_dtype=torch.float32, out=None):
    res = ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens, c.block_tables,
                             c.max_seqlen_q, c.scale, block_size=c.block_size,
                             out_dtype=out_dtype, out=out)
    torch.cuda.synchronize()
    return res


def _oracle(c):
    return O.paged_attention(to_np(c.q), to_np(c.k_pool), to_np(c.v_pool), to_np(c.block_tables),
                             to_np(c.cu_seqlens_q), to_np(c.kv_lens), c.block_size, c.scale,
                             bf16=True)


def _case(H, G, D, bs, lens, prefix, seed):
    c = make_prefill(len(lens), H, G, D, bs, (1, 1), prefix=prefix, dtype=torch.float32,
                     seed=seed, device="cuda:0", q_lens=lens)
    ops.kv_write(c.k_new, c.v_new, c.k_pool, c.v_pool, c.slot_mapping)
    return c


@pytest.mark.parametrize("H,G,D,bs,lens,prefix", [
    (8, 8, 64, 16, [1, 17, 40, 300], 32),    # partial tiles, a cached prefix
    (16, 4, 128, 16, [129, 5], 0),            # GQA 4 at head_dim 128
    (14, 2, 64, 16, [300, 77, 1], 64),        # Qwen2.5-0.5B heads (GQA 7)
    (8, 2, 64, 7, [50, 33, 64], 14),          # 7-token pages: table lookups per position
    (4, 4, 128, 32, [32, 31, 33, 96], 0),     # tile edges
    (2, 1, 64, 16, [700], 0),                 # 22 tiles, the longest walking 22 steps
])
def test_prefill_f32_matrix_cores_match_oracle(device, H, G, D, bs, lens, prefix):
    c = _case(H, G, D, bs, lens, prefix, seed=H + D + bs)
    ref = _oracle(c)
    got = to_np(_run(c))
    max_abs, rel = errors(got, ref)
    print(f"fp32 mfma prefill H={H} G={G} D={D} bs={bs}: max_abs={max_abs:.3e} rel={rel:.3e}",
          flush=True)
    assert max_abs <= 1e-5


def test_prefill_f32_matches_the_vector_kernel(device):
    """The matrix-core and vector fp32 paths agree to the fp32 bound on the same batch."""
    c = _case(8, 2, 128, 16, [200, 31, 64], 16, seed=3)
    mfma = to_np(_run(c))
    assert _lib.lib().flour_hip_set_prefill_f32_mfma(0) == 0
    try:
        simt = to_np(_run(c))
    finally:
        _lib.lib().flour_hip_set_prefill_f32_mfma(1)
    assert errors(mfma, simt)[0] <= 1e-5


def test_prefill_f32_16bit_outputs_round_the_fp32_result(device):
    c = _case(8, 8, 64, 16, [90, 33, 1], 0, seed=11)
    got32 = to_np(_run(c))
    assert np.array_equal(to_np(_run(c, torch.bfloat16)), f32_to_bf16_bits(got32))
    assert np.array_equal(to_np(_run(c, torch.float16)), got32.astype(np.float16).view(np.uint16))


def test_prefill_f32_kv_shorter_than_q_gives_zero_rows(device):
    for D in (64, 128):
        c = _case(8, 2, D, 16, [40, 50, 200], 0, seed=29)
        c.kv_lens[1] = 49
        out = torch.full((c.q.shape[0], 8, D), 7.0, dtype=torch.float32, device=device)
        _run(c, out=out)
        got = to_np(out)
        assert np.array_equal(got[40:90], np.zeros_like(got[40:90])), D
        assert errors(got, _oracle(c))[0] <= 1e-5, D


def test_prefill_f32_strided_q_and_out(device):
    """q in the reference's head-major (H, seq, D) layout as a transposed view; strided out."""
    c = _case(8, 4, 64, 16, [150], 0, seed=8)
    q_hm = c.q.transpose(0, 1).contiguous()
    out_hm = torch.empty((8, 150, 64), dtype=torch.float32, device=device)
    ops.varlen_prefill(q_hm.transpose(0, 1), c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                       c.block_tables, c.max_seqlen_q, c.scale, out_dtype=torch.float32,
                       out=out_hm.transpose(0, 1))
    torch.cuda.synchronize()
    assert torch.equal(out_hm.transpose(0, 1), _run(c))


def test_prefill_f32_benchmark_batch_full_size(device):
    c = make_workload("prefill_f32_h8_d64", device)
    ops.kv_write(c.k_new, c.v_new, c.k_pool, c.v_pool, c.slot_mapping)
    got = to_np(_run(c))
    max_abs, rel = errors(got, _oracle(c))
    print(f"prefill_f32_h8_d64: max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    assert max_abs <= 1e-5
