"""Causal varlen prefill at head_dim 64 on the matrix-core kernel (the Qwen2.5-0.5B attention
shape the reference serves: 14 q / 2 kv heads, GQA 7, src/models/qwen2.rs:39 with
script/script.js:14), against the oracle's restatement of paged_attention (cpu.rs:57-112).

Bounds as for head_dim 128: the fp32 accumulator output within max-abs 2e-3 and rel-L2 1e-3 of
the fp32 oracle, the bf16 output within the ulp bounds of tests/_util.py. Covered: GQA 7, a
cached prefix shared by every sequence, partial last query tiles (the 4 x 64 and 8 x 32 item
shapes and the one-head 256-row items of an odd group), page sizes 16 and 32, kv_len < q_len,
the persistent schedule against one workgroup per item, V outside the fp16 range (the exact
redo), the hi + lo P mode and the whole benchmark batch.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import PREFILL_ULP_BOUNDS, check_bf16_output, errors, to_np
from flour_amd import _lib, ops
from flour_amd.workloads import make_prefill, make_workload
from test_prefill_gpu import oracle_prefill, run, write

pytestmark = pytest.mark.gpu

D = 64


def check(c, seqs=None, tag=""):
    ref, rows = oracle_prefill(c, seqs)
    got32 = to_np(run(c, torch.float32))[rows]
    max_abs, rel = errors(got32, ref)
    print(f"{tag} fp32-out max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3
    if c.q.dtype == torch.bfloat16:
        rep = check_bf16_output(to_np(run(c, torch.bfloat16))[rows], got32, ref,
                                PREFILL_ULP_BOUNDS)
        print(f"{tag} bf16-out {rep}", flush=True)
    return got32


def go(c, persistent=1, out_dtype=torch.float32):
    H = c.q.shape[1]
    out = torch.full((c.q.shape[0], H, D), 7.0, dtype=out_dtype, device=c.q.device)
    _lib.lib().flour_hip_set_prefill_persistent(persistent)
    try:
        ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens, c.block_tables,
                           c.max_seqlen_q, c.scale, block_size=c.block_size, out_dtype=out_dtype,
                           out=out)
        torch.cuda.synchronize()
    finally:
        _lib.lib().flour_hip_set_prefill_persistent(1)
    return out


@pytest.mark.parametrize("H,G,bs,lens,prefix", [
    (14, 2, 16, [300, 77, 1], 64),          # Qwen2.5-0.5B heads over a cached prefix
    (14, 2, 32, [129, 33, 64, 200], 32),    # 32-token pages
    (8, 2, 16, [1, 2, 31, 32, 33], 0),      # one-row and one-tile sequences
    (16, 16, 16, [257, 5], 48),             # n_rep 1
    (8, 1, 16, [1, 200], 160),              # n_rep 8
    (14, 2, 48, [150, 96], 96),             # 48-token pages
])
def test_prefill_d64_shapes(device, H, G, bs, lens, prefix):
    c = make_prefill(len(lens), H, G, D, bs, (1, 1), prefix=prefix, dtype=torch.bfloat16,
                     seed=H * 5 + G + bs, device=device, q_lens=lens)
    write(c)
    check(c, tag=f"D64 H={H} G={G} bs={bs} lens={lens} prefix={prefix}")


def test_prefill_d64_f16_pools(device):
    c = make_prefill(3, 14, 2, D, 16, (1, 1), prefix=32, dtype=torch.float16, seed=61,
                     device=device, q_lens=[200, 64, 9])
    write(c)
    check(c, tag="D64 f16")


def test_prefill_qwen25_05b_workload(device):
    """The head_dim-64 benchmark batch (8 prompts of U[256, 1024] rows, 14 / 2 heads): every
    row of every sequence against the oracle."""
    c = make_workload("prefill_bf16_qwen25_05b", device=device)
    write(c)
    lens = (c.cu_seqlens_q[1:] - c.cu_seqlens_q[:-1]).tolist()
    print(f"lens={lens}", flush=True)
    check(c, tag="qwen2.5-0.5b prefill (whole batch)")


@pytest.mark.parametrize("H,G", [(14, 2), (16, 4), (10, 2)])
def test_prefill_d64_persistent_and_partial_tiles(device, H, G):
    """Persistent schedule with the partial-last-tile item shapes (4 heads x 64 rows, 8 heads x
    32 rows, one-head 256-row items of odd groups 7 and 5) bit-identical to one workgroup per
    item, empty sequences and a sequence with kv_len < q_len (zero rows) included."""
    rng = np.random.default_rng(H * 7 + G)
    lens = []
    for i in range(30):
        full = int(rng.integers(0, 4)) * 128
        tail = [int(rng.integers(1, 33)), int(rng.integers(33, 65)), int(rng.integers(65, 129))][i % 3]
        lens.append(full + tail)
    lens[4] = 0
    c = make_prefill(len(lens), H, G, D, 16, (1, 1), prefix=64, dtype=torch.bfloat16,
                     seed=70 + H, device=device, q_lens=lens)
    write(c)
    c.kv_lens[9] = lens[9] - 1  # kv_len < q_len: the sequence attends nothing
    a, b = go(c, 1), go(c, 0)
    assert torch.equal(a, b)
    cu = to_np(c.cu_seqlens_q)
    assert bool((a[int(cu[9]):int(cu[10])] == 0.0).all())
    ref, rows = oracle_prefill(c, seqs=[0, 1, 2, 29])
    max_abs, rel = errors(to_np(a)[rows], ref)
    print(f"D64 persistent H={H} G={G}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


def test_prefill_d64_v_outside_fp16_range(device):
    """V rows of +-1e5 and 1e-30 among N(0,1) rows: the items that meet them are recomputed in
    exact mode (bf16 V, P split in two); judged against the output's own scale."""
    c = make_prefill(4, 14, 2, D, 16, (1, 1), prefix=32, dtype=torch.bfloat16, seed=81,
                     device=device, q_lens=[150, 40, 260, 7])
    c.v_new[10:14] *= 1e5
    c.v_new[100:103] *= 1e-30
    write(c)
    ref, rows = oracle_prefill(c)
    got = to_np(run(c, torch.float32))[rows]
    assert np.isfinite(got).all()
    scale = np.abs(ref).max(axis=-1, keepdims=True) + 1e-30
    err = np.abs(got - ref) / scale
    print(f"D64 V out of range: max rel-to-row-scale err={err.max():.3e}", flush=True)
    assert err.max() <= 2e-3


def test_prefill_d64_hilo_mode(device):
    c = make_prefill(3, 14, 2, D, 16, (1, 1), prefix=16, dtype=torch.bfloat16, seed=91,
                     device=device, q_lens=[333, 70, 1])
    write(c)
    assert _lib.lib().flour_hip_set_prefill_precise_p(1) == 0
    try:
        got = check(c, tag="D64 hi+lo P")
    finally:
        _lib.lib().flour_hip_set_prefill_precise_p(0)
    assert np.isfinite(got).all()


def test_prefill_d64_reference_layout(device):
    """q in the reference's head-major (1, heads, seq, D) layout and out written straight into
    (seq, heads, D): strided views on both sides."""
    c = make_prefill(1, 14, 2, D, 16, (1, 1), prefix=0, dtype=torch.bfloat16, seed=95,
                     device=device, q_lens=[190])
    write(c)
    q_hm = c.q.transpose(0, 1).contiguous()          # (heads, seq, D)
    q_view = q_hm.transpose(0, 1)                    # (seq, heads, D), strides (D, seq*D, 1)
    out = ops.varlen_prefill(q_view, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                             c.block_tables, c.max_seqlen_q, c.scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref, rows = oracle_prefill(c)
    max_abs, rel = errors(to_np(out)[rows], ref)
    assert max_abs <= 2e-3 and rel <= 1e-3
