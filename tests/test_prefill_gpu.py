"""Kernels (1)+(3) parity: KV write then causal varlen prefill attention against the oracle's
restatement of paged_attention (src/backend/cpu.rs:57-112) for seq_q >= 1, including suffixes
over prefix-cached shared blocks, on identical seeded inputs.

Tolerances: fp32 pools max-abs <= 1e-5; bf16 pools with fp32 output max-abs <= 2e-3 and
rel-L2 <= 1e-3 against the fp32 oracle; bf16 output exactly RNE(kernel fp32 result), its
rel-L2 within 5% of the floor set by rounding the exact result to bf16 (~1.5e-3), max-abs
within that floor + 2e-3, and within the bf16-ulp bounds of _util.PREFILL_ULP_BOUNDS of
RNE(reference). Inputs outside the N(0, 1) range (V values that fp16 cannot hold, tiny or
huge V) are judged relative to the output's own scale: rel-L2 <= 1e-3, max-abs <= 2e-3 of
max |reference|, and finite exactly where the reference is.
"""
from __future__ import annotations

import time

import numpy as np
import pytest
import torch

import oracle as O
from _util import PREFILL_ULP_BOUNDS, check_bf16_output, errors, to_np
from flour_amd import ops
from flour_amd.workloads import make_prefill, make_workload

pytestmark = pytest.mark.gpu


def write(c):
    ops.kv_write(c.k_new, c.v_new, c.k_pool, c.v_pool, c.slot_mapping)


def run(c, out_dtype=None, q=None, workspace=None):
    out = ops.varlen_prefill(c.q if q is None else q, c.k_pool, c.v_pool, c.cu_seqlens_q,
                             c.kv_lens, c.block_tables, c.max_seqlen_q, c.scale,
                             block_size=c.block_size, out_dtype=out_dtype, workspace=workspace)
    torch.cuda.synchronize()
    return out


def oracle_prefill(c, seqs=None) -> tuple[np.ndarray, np.ndarray]:
    """Oracle output for the listed sequences; returns (reference, packed row indices)."""
    cu = to_np(c.cu_seqlens_q)
    n = cu.size - 1
    seqs = list(range(n)) if seqs is None else list(seqs)
    rows = np.concatenate([np.arange(cu[s], cu[s + 1]) for s in seqs])
    sub_cu = np.concatenate([[0], np.cumsum([cu[s + 1] - cu[s] for s in seqs])]).astype(np.int32)
    ref = O.paged_attention(to_np(c.q)[rows], to_np(c.k_pool), to_np(c.v_pool),
                            to_np(c.block_tables)[seqs], sub_cu, to_np(c.kv_lens)[seqs],
                            c.block_size, c.scale, bf16=(c.q.dtype != torch.float16))
    return ref, rows


def check_bf16(c, seqs=None, tag=""):
    ref, rows = oracle_prefill(c, seqs)
    got32 = to_np(run(c, torch.float32))[rows]
    max_abs, rel = errors(got32, ref)
    print(f"{tag} fp32-out max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3
    rep = check_bf16_output(to_np(run(c, torch.bfloat16))[rows], got32, ref, PREFILL_ULP_BOUNDS)
    print(f"{tag} bf16-out {rep}", flush=True)


@pytest.mark.parametrize("H,G,D,bs,lens,prefix", [
    (2, 2, 4, 2, [5], 0),          # the reference's prefill test shape (cpu.rs:190-206)
    (4, 2, 4, 4, [6], 0),          # GQA (cpu.rs:226-242)
    (4, 1, 8, 4, [3, 5], 16),      # suffixes over a cached prefix
    (8, 8, 64, 16, [1, 17, 40], 32),
])
def test_prefill_fp32_small_shapes(device, H, G, D, bs, lens, prefix):
    c = make_prefill(len(lens), H, G, D, bs, (1, 1), prefix=prefix, dtype=torch.float32,
                     seed=H + D, device=device, q_lens=lens)
    write(c)
    ref, rows = oracle_prefill(c)
    max_abs, _ = errors(to_np(run(c))[rows], ref)
    assert max_abs <= 1e-5


@pytest.mark.parametrize("H,G,lens,prefix", [
    (8, 2, [1, 2, 31, 32, 33], 0),
    (32, 8, [64, 127, 128, 129, 300], 0),
    (28, 4, [130, 17], 1024),      # n_rep 7, cached prefix (Qwen2 shape)
    (16, 16, [257, 5], 48),        # n_rep 1
    (8, 1, [1, 200], 160),
])
def test_prefill_bf16_mfma_shapes(device, H, G, lens, prefix):
    c = make_prefill(len(lens), H, G, 128, 16, (1, 1), prefix=prefix, dtype=torch.bfloat16,
                     seed=H * 3 + G, device=device, q_lens=lens)
    write(c)
    check_bf16(c, tag=f"H={H} G={G} lens={lens} prefix={prefix}")


def test_prefill_varlen_llama3_8b_workload(device):
    """KV write + causal varlen prefill, 8 sequences U[256, 2048], 32/8 heads: every row of
    every sequence against the oracle."""
    c = make_workload("prefill_bf16_varlen_llama3_8b", device=device)
    write(c)
    lens = (c.cu_seqlens_q[1:] - c.cu_seqlens_q[:-1]).tolist()
    print(f"lens={lens} causal_pairs={c.causal_pairs()}", flush=True)
    check_bf16(c, tag="llama3-8b prefill (whole batch)")


def test_prefill_prefix_qwen2_7b_workload(device):
    """Prefix-cached prefill: 16 suffixes U[128, 512] over one shared 1024-token prefix; every
    row of every sequence against the oracle."""
    c = make_workload("prefill_bf16_prefix_qwen2_7b", device=device)
    write(c)
    check_bf16(c, tag="qwen2-7b prefix prefill (whole batch)")


def test_prefill_with_k_outlier_channels(device):
    """The decode workload's outliers in prefill: 0.1% of the K channels (at least one
    (kv head, dim) channel) scaled x20, in the cached prefix and in the new rows."""
    c = make_prefill(3, 32, 8, 128, 16, (1, 1), prefix=128, dtype=torch.bfloat16, seed=17,
                     device=device, q_lens=[700, 65, 300])
    g = torch.Generator(device="cpu").manual_seed(18)
    ch = torch.randperm(8 * 128, generator=g)[:max(1, round(0.001 * 8 * 128))].tolist()
    for x in ch:
        gh, d = divmod(x, 128)
        c.k_pool[gh, :, d] = (c.k_pool[gh, :, d].float() * 20).to(torch.bfloat16)
        c.k_new[:, gh, d] = (c.k_new[:, gh, d].float() * 20).to(torch.bfloat16)
    write(c)
    check_bf16(c, tag=f"K outlier channels {ch}")


def _check_scaled(got: np.ndarray, ref: np.ndarray, tag: str) -> None:
    """fp32 outputs far from unit scale: finite exactly where the reference is, rel-L2 <= 1e-3
    and max-abs <= 2e-3 of the largest reference magnitude, over the finite elements."""
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin), f"{tag}: non-finite outputs differ"
    scale = float(np.abs(ref[fin]).max()) if fin.any() else 1.0
    max_abs, rel = errors(got[fin] / scale, ref[fin] / scale)
    print(f"{tag}: scale={scale:.3e} max_abs/scale={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


def _check_scaled_bf16(got_bits: np.ndarray, got32: np.ndarray, ref: np.ndarray,
                       tag: str) -> None:
    """bf16 outputs far from unit scale: RNE of the kernel's fp32 result, rel-L2 within 5% of
    the bf16 rounding floor, and within 2 bf16 ulps of RNE(reference) wherever |ref| is at
    least 2^-4 of the largest reference magnitude."""
    from _util import bf16_bits_to_f32, bf16_ulp_distance, f32_to_bf16_bits
    fin = np.isfinite(ref)
    assert np.array_equal(got_bits[fin], f32_to_bf16_bits(got32[fin])), "bf16 != RNE(fp32 out)"
    scale = float(np.abs(ref[fin]).max()) if fin.any() else 1.0
    _, rel = errors(bf16_bits_to_f32(got_bits[fin]) / scale, ref[fin] / scale)
    _, floor = errors(bf16_bits_to_f32(f32_to_bf16_bits(ref[fin])) / scale, ref[fin] / scale)
    big = fin & (np.abs(ref) >= scale * 2.0 ** -4)
    ulp = int(bf16_ulp_distance(got_bits[big], ref[big]).max()) if big.any() else 0
    print(f"{tag}: rel_l2={rel:.3e} floor={floor:.3e} max_ulp={ulp}", flush=True)
    assert rel <= 1.05 * floor + 1e-5 and ulp <= 2


@pytest.mark.parametrize("case", ["mixed", "tiny", "small", "large", "huge"])
def test_prefill_v_outside_fp16_range(device, case):
    """bf16 V far from unit scale. The default P.V runs on fp16 MFMAs over V converted to
    fp16, exact for 2^-17 <= |v| <= 65504; an item whose output block is not finite (a value
    overflowed fp16) or whose root mean square is below 2^-25 / 5e-4 is recomputed in exact
    bf16 mode. The reference accumulates probs @ v.to_dtype(F32) for any finite bf16
    (cpu.rs:103-104).
      mixed: rows of +-1e5, one row of +-3e38 and rows of 1e-30 among N(0, 1) rows, in the
             cached prefix and in the new rows (one huge row per sequence, so every weighted
             sum stays in the fp32 range, as in the reference);
      tiny:  every V value scaled by 1e-30 (exact mode);
      small: every V value scaled by 1e-4 (outputs of ~1e-6: exact mode);
      large: every V value scaled by 300 (within fp16: the fp16 path);
      huge:  every V value scaled by 1e30."""
    c = make_prefill(3, 8, 2, 128, 16, (1, 1), prefix=64, dtype=torch.bfloat16, seed=23,
                     device=device, q_lens=[300, 77, 129])
    vp = c.v_pool.float()
    vn = c.v_new.float()
    if case == "mixed":
        g = torch.Generator(device="cpu").manual_seed(24)
        prefix_slots = [b * 16 + i for b in c.meta["prefix_blocks"] for i in range(16)]
        for s_ in prefix_slots[5:9]:
            vp[:, s_, :] *= 1e5
        vp[:, prefix_slots[40], :] = 1e-30
        cu = c.cu_seqlens_q.cpu().tolist()
        for s in range(3):
            rows = torch.randperm(cu[s + 1] - cu[s], generator=g)[:6] + cu[s]
            vn[rows[0], :, :] = 3e38 * torch.sign(vn[rows[0], :, :])
            vn[rows[1:3], :, :] *= 1e5
            vn[rows[3:6], :, :] = 1e-30
    else:
        f = {"tiny": 1e-30, "small": 1e-4, "large": 300.0, "huge": 1e30}[case]
        vp *= f
        vn *= f
    c.v_pool.copy_(vp.to(torch.bfloat16))
    c.v_new.copy_(vn.to(torch.bfloat16))
    write(c)
    ref, rows = oracle_prefill(c)
    got32 = to_np(run(c, torch.float32))[rows]
    _check_scaled(got32, ref, f"V {case} fp32-out")
    got16 = to_np(run(c, torch.bfloat16))[rows]
    _check_scaled_bf16(got16, got32, ref, f"V {case} bf16-out")


@pytest.mark.parametrize("bs,kv", [(32, 2200), (48, 3200), (64, 4300)])
def test_prefill_block_table_window_crossings(device, bs, kv):
    """Block ids reach the tile loads through a 64-entry window of the block table; these
    sequences cross it with 32-, 48- and 64-token pages (a 48-token page makes a tile's pages
    straddle the window end, the second-window read)."""
    c = make_prefill(2, 4, 1, 128, bs, (1, 1), prefix=0, dtype=torch.bfloat16, seed=bs,
                     device=device, q_lens=[kv, 33])
    write(c)
    check_bf16(c, tag=f"bs={bs} kv={kv}")


def test_prefill_kv_shorter_than_q_gives_zero_rows_on_every_path(device):
    """A sequence whose kv length is below its query count attends nothing: its rows are
    written as zeros by the MFMA path (bf16 pools) and by the fp32 path (fp32 pools), as
    the oracle does; the other sequences are unaffected."""
    for dt in (torch.bfloat16, torch.float32):
        c = make_prefill(3, 8, 2, 128, 16, (1, 1), prefix=0, dtype=dt, seed=29, device=device,
                         q_lens=[40, 50, 200])
        write(c)
        c.kv_lens[1] = 49
        out = torch.full((c.q.shape[0], 8, 128), 7.0, dtype=torch.float32, device=device)
        ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens, c.block_tables,
                           c.max_seqlen_q, c.scale, out_dtype=torch.float32, out=out)
        torch.cuda.synchronize()
        got = to_np(out)
        ref, rows = oracle_prefill(c)
        assert np.array_equal(got[40:90], np.zeros_like(got[40:90])), dt
        max_abs, _ = errors(got[rows], ref)
        assert max_abs <= (2e-3 if dt == torch.bfloat16 else 1e-5), (dt, max_abs)


def test_suffix_over_cached_prefix_matches_cold_prefill(device):
    """model.rs:244-360 at the attention level: the suffix rows of a cold full prefill equal a
    suffix-only prefill over the cached prefix blocks."""
    P, S, H, G = 96, 70, 8, 2
    cold = make_prefill(1, H, G, 128, 16, (1, 1), prefix=0, dtype=torch.bfloat16, seed=12,
                        device=device, q_lens=[P + S])
    write(cold)
    full = run(cold, torch.float32)
    # the same sequence: prefix rows already cached, only the last S rows are new queries
    cu = torch.tensor([0, S], dtype=torch.int32, device=device)
    kvl = torch.tensor([P + S], dtype=torch.int32, device=device)
    out = ops.varlen_prefill(cold.q[P:], cold.k_pool, cold.v_pool, cu, kvl, cold.block_tables,
                             S, cold.scale, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert errors(to_np(out), to_np(full[P:]))[0] <= 1e-5


def test_prefill_reference_layout_and_strided_output(device):
    """q in the reference's head-major (H, seq, D) layout as a transposed view; strided out."""
    c = make_prefill(1, 16, 4, 128, 16, (1, 1), dtype=torch.bfloat16, seed=8, device=device,
                     q_lens=[150])
    write(c)
    q_ref = c.q.transpose(0, 1).contiguous()       # (H, S, D)
    out_ref = torch.empty((16, 150, 128), dtype=torch.float32, device=device)
    ops.varlen_prefill(q_ref.transpose(0, 1), c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                       c.block_tables, c.max_seqlen_q, c.scale, out_dtype=torch.float32,
                       out=out_ref.transpose(0, 1))
    torch.cuda.synchronize()
    packed = run(c, torch.float32)
    assert torch.equal(out_ref.transpose(0, 1), packed)


def test_prefill_hilo_mode_meets_the_same_bounds(device):
    """The alternative P.V mode (P split into bf16 hi + lo parts, two MFMAs per product)
    meets the same fp32-accumulator bounds as the default fp16 P.V."""
    from flour_amd import _lib
    c = make_prefill(3, 32, 8, 128, 16, (1, 1), dtype=torch.bfloat16, seed=5, device=device,
                     q_lens=[300, 64, 1000], prefix=64)
    write(c)
    ref, rows = oracle_prefill(c)
    _lib.lib().flour_hip_set_prefill_precise_p(1)
    try:
        got = to_np(run(c, torch.float32))[rows]
    finally:
        _lib.lib().flour_hip_set_prefill_precise_p(0)
    max_abs, rel = errors(got, ref)
    print(f"hi+lo P: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


@pytest.mark.parametrize("bs", [32, 64])
def test_prefill_bf16_mfma_larger_blocks(device, bs):
    """The MFMA path with pages of 32 / 64 tokens (a 64-token tile spans one or two pages)."""
    c = make_prefill(3, 16, 4, 128, bs, (1, 1), prefix=2 * bs, dtype=torch.bfloat16, seed=bs,
                     device=device, q_lens=[70, 1, 200])
    write(c)
    check_bf16(c, tag=f"bs={bs}")


def test_prefill_f16_pools(device):
    """fp16 storage on the MFMA path (Q.K in fp16, P.V in fp16)."""
    c = make_prefill(2, 8, 2, 128, 16, (1, 1), prefix=32, dtype=torch.float16, seed=21,
                     device=device, q_lens=[90, 33])
    write(c)
    ref, rows = oracle_prefill(c)
    got = to_np(run(c, torch.float32))[rows]
    max_abs, rel = errors(got, ref)
    print(f"f16 fp32-out max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


def test_prefill_long_sequence_many_tiles(device):
    """One 4100-row sequence (33 query tiles, 65 kv tiles for the last) next to a 1-row one;
    the oracle checks every row of both."""
    c = make_prefill(2, 8, 2, 128, 16, (1, 1), prefix=0, dtype=torch.bfloat16, seed=31,
                     device=device, q_lens=[4100, 1])
    write(c)
    out = to_np(run(c, torch.float32))
    cu = to_np(c.cu_seqlens_q)
    ref, rows = oracle_prefill(c, seqs=[0])
    max_abs, rel = errors(out[rows], ref)
    print(f"long fp32-out max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3
    ref1, rows1 = oracle_prefill(c, seqs=[1])
    assert errors(out[rows1], ref1)[0] <= 2e-3
    assert cu[-1] == 4101


@pytest.mark.parametrize("H,G", [(12, 4), (8, 8)])
def test_prefill_persistent_schedule_matches_one_workgroup_per_tile(device, H, G):
    """The persistent schedule (one workgroup per CU walking the longest-first list of query
    tiles) gives bit-identical output to one workgroup per (tile, sequence, head pair), with
    empty sequences, a sequence whose kv length is below its query length (its rows are
    written as zeros) and an odd GQA group (a pair with one idle head)."""
    from flour_amd import _lib
    rng = np.random.default_rng(3)
    lens = [int(x) for x in rng.integers(0, 700, size=37)]
    lens[5] = 0
    lens[11] = 1
    lens[20] = 690
    lens[7] = 300  # three tiles: with an odd group the first two share a one-head item
    c = make_prefill(len(lens), H, G, 128, 16, (1, 1), prefix=32, dtype=torch.bfloat16, seed=9,
                     device=device, q_lens=lens)
    write(c)
    c.kv_lens[7] = 299  # kv_len < q_len: the sequence attends nothing

    def go(persistent):
        out = torch.full((c.q.shape[0], H, 128), 7.0, dtype=torch.float32, device=device)
        _lib.lib().flour_hip_set_prefill_persistent(persistent)
        try:
            ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                               c.block_tables, c.max_seqlen_q, c.scale, out_dtype=torch.float32,
                               out=out)
            torch.cuda.synchronize()
        finally:
            _lib.lib().flour_hip_set_prefill_persistent(1)
        return out

    a, b = go(1), go(0)
    assert torch.equal(a, b)
    cu = to_np(c.cu_seqlens_q)
    assert bool((a[int(cu[7]):int(cu[8])] == 0.0).all())
    ref, rows = oracle_prefill(c, seqs=[0, 20, 36])
    max_abs, rel = errors(to_np(a)[rows], ref)
    print(f"persistent H={H} G={G} max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


@pytest.mark.parametrize("n,max_len", [(64, 8064), (65, 900), (30, 8065)])
def test_prefill_schedule_order_on_both_sort_paths(device, n, max_len):
    """The sequence order of the persistent schedule is built in registers for up to 64
    sequences and 63 tiles, through LDS otherwise; on both sides of each limit (64 sequences
    with one of 63 tiles; 65 sequences; 64 tiles) the output is bit-identical to one workgroup
    per item, with equal tile counts (ties broken by index) and empty sequences."""
    from flour_amd import _lib
    rng = np.random.default_rng(n)
    lens = [int(x) for x in rng.integers(0, 400, size=n)]
    lens[0] = max_len
    lens[1] = 0
    lens[2] = lens[3] = 256  # equal tile counts
    c = make_prefill(n, 8, 2, 128, 16, (1, 1), prefix=0, dtype=torch.bfloat16, seed=n + 1,
                     device=device, q_lens=lens)
    write(c)

    def go(persistent):
        out = torch.full((c.q.shape[0], 8, 128), 7.0, dtype=torch.float32, device=device)
        _lib.lib().flour_hip_set_prefill_persistent(persistent)
        try:
            ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                               c.block_tables, c.max_seqlen_q, c.scale, out_dtype=torch.float32,
                               out=out)
            torch.cuda.synchronize()
        finally:
            _lib.lib().flour_hip_set_prefill_persistent(1)
        return out

    a, b = go(1), go(0)
    assert torch.equal(a, b)
    ref, rows = oracle_prefill(c, seqs=[2, 3, n - 1])
    max_abs, rel = errors(to_np(a)[rows], ref)
    assert max_abs <= 2e-3 and rel <= 1e-3


@pytest.mark.parametrize("H,G", [(20, 4), (28, 4), (32, 4)])
def test_prefill_partial_tile_shapes(device, H, G):
    """A sequence's last query tile with at most 64 (32) rows runs as items of 4 (8) heads x
    64 (32) rows instead of 2 heads x 128, and with an odd group the last head of two
    consecutive tiles as 1 head x 256 rows, with GQA groups of 5, 7 and 8 heads and sequences
    of 1 to 4 tiles: bit-identical to one workgroup per (tile, head pair), and against the
    oracle on short and long sequences."""
    from flour_amd import _lib
    rng = np.random.default_rng(H)
    lens = []
    for i in range(36):
        full = int(rng.integers(0, 4)) * 128
        tail = [int(rng.integers(1, 33)), int(rng.integers(33, 65)), int(rng.integers(65, 129))][i % 3]
        lens.append(full + tail)
    c = make_prefill(len(lens), H, G, 128, 16, (1, 1), prefix=64, dtype=torch.bfloat16,
                     seed=50 + H, device=device, q_lens=lens)
    write(c)

    def go(persistent):
        out = torch.full((c.q.shape[0], H, 128), 7.0, dtype=torch.float32, device=device)
        _lib.lib().flour_hip_set_prefill_persistent(persistent)
        try:
            ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                               c.block_tables, c.max_seqlen_q, c.scale, out_dtype=torch.float32,
                               out=out)
            torch.cuda.synchronize()
        finally:
            _lib.lib().flour_hip_set_prefill_persistent(1)
        return out

    a, b = go(1), go(0)
    assert torch.equal(a, b)
    ref, rows = oracle_prefill(c, seqs=[0, 1, 2, 35])
    max_abs, rel = errors(to_np(a)[rows], ref)
    print(f"partial tiles H={H} G={G}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


def test_prefill_long_entry_list_uses_plain_pairs(device):
    """More (tile, sequence) entries than the per-entry item tables hold (1,100 sequences of 4
    query tiles, 4,400 entries): the persistent list falls back to plain head pairs and stays
    bit-identical to one workgroup per item, with an odd GQA group of 7."""
    from flour_amd import _lib
    rng = np.random.default_rng(77)
    lens = [int(x) for x in rng.integers(385, 513, size=1100)]
    c = make_prefill(len(lens), 7, 1, 128, 16, (1, 1), prefix=16, dtype=torch.bfloat16,
                     seed=78, device=device, q_lens=lens)
    write(c)

    def go(persistent):
        out = torch.full((c.q.shape[0], 7, 128), 7.0, dtype=torch.float32, device=device)
        _lib.lib().flour_hip_set_prefill_persistent(persistent)
        try:
            ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                               c.block_tables, c.max_seqlen_q, c.scale, out_dtype=torch.float32,
                               out=out)
            torch.cuda.synchronize()
        finally:
            _lib.lib().flour_hip_set_prefill_persistent(1)
        return out

    a, b = go(1), go(0)
    assert torch.equal(a, b)
    ref, rows = oracle_prefill(c, seqs=[0, 549, 1099])
    max_abs, rel = errors(to_np(a.float())[rows], ref)
    print(f"long entry list: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


def test_prefill_graph_replay_matches_eager(device):
    """Prefill captured in a HIP graph and replayed, with eager work and synchronisations
    between replays: each replay gives the eager result bit for bit (several items per
    workgroup, so the Q staging loads, the cross-item tile loads and the output stores all run
    inside the graph)."""
    rng = np.random.default_rng(12)
    lens = [int(x) for x in rng.integers(100, 900, size=40)]
    c = make_prefill(len(lens), 32, 8, 128, 16, (1, 1), prefix=0, dtype=torch.bfloat16,
                     seed=14, device=device, q_lens=lens)
    write(c)
    eager = run(c, torch.bfloat16)
    out = torch.empty_like(eager)

    def step():
        ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens, c.block_tables,
                           c.max_seqlen_q, c.scale, block_size=c.block_size, out=out)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i in range(4):
        out.zero_()
        noise = torch.randn(1 << 20, device=device).sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs"
        assert torch.isfinite(noise)


@pytest.mark.parametrize("bs", [32, 48])
def test_prefill_persistent_schedule_other_page_sizes(device, bs):
    """Several items per workgroup with 32- and 48-token pages (a 64-token tile spans two or
    three pages, and the next item's first tiles are located through its block-table window
    while the current item runs): bit-identical to one workgroup per item, and against the
    oracle on two sequences."""
    from flour_amd import _lib
    rng = np.random.default_rng(5 + bs)
    lens = [int(x) for x in rng.integers(1, 600, size=48)]
    c = make_prefill(len(lens), 16, 4, 128, bs, (1, 1), prefix=2 * bs, dtype=torch.bfloat16,
                     seed=40 + bs, device=device, q_lens=lens)
    write(c)

    def go(persistent):
        out = torch.full((c.q.shape[0], 16, 128), 7.0, dtype=torch.float32, device=device)
        _lib.lib().flour_hip_set_prefill_persistent(persistent)
        try:
            ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                               c.block_tables, c.max_seqlen_q, c.scale, block_size=bs,
                               out_dtype=torch.float32, out=out, workspace=ops.Workspace(device))
            torch.cuda.synchronize()
        finally:
            _lib.lib().flour_hip_set_prefill_persistent(1)
        return out

    a, b = go(1), go(0)
    assert torch.equal(a, b)
    ref, rows = oracle_prefill(c, seqs=[0, 47])
    max_abs, rel = errors(to_np(a)[rows], ref)
    print(f"persistent bs={bs}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


def test_prefill_persistent_schedule_with_exact_redo(device):
    """Several items per workgroup, where an item's first K / V tiles and Q rows are fetched
    while the item before it runs, and some items take the exact-mode redo (V rows of +-1e5
    overflow the fp16 widening): bit-identical to one workgroup per item, and within the
    scaled bounds of the oracle on sequences with and without the large rows."""
    from flour_amd import _lib
    rng = np.random.default_rng(17)
    lens = [int(x) for x in rng.integers(90, 700, size=60)]
    lens[4] = 0
    lens[9] = 20
    c = make_prefill(len(lens), 16, 4, 128, 16, (1, 1), prefix=64, dtype=torch.bfloat16,
                     seed=31, device=device, q_lens=lens)
    vn = c.v_new.float()
    cu = c.cu_seqlens_q.cpu().tolist()
    big = [s for s in range(len(lens)) if s % 3 == 1 and lens[s] > 0]
    for s in big:
        vn[cu[s] + lens[s] // 2, :, :] *= 1e5
    c.v_new.copy_(vn.to(torch.bfloat16))
    write(c)
    c.kv_lens[9] = 19  # kv_len < q_len: the sequence attends nothing

    def go(persistent):
        out = torch.full((c.q.shape[0], 16, 128), 7.0, dtype=torch.float32, device=device)
        _lib.lib().flour_hip_set_prefill_persistent(persistent)
        try:
            ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                               c.block_tables, c.max_seqlen_q, c.scale, out_dtype=torch.float32,
                               out=out)
            torch.cuda.synchronize()
        finally:
            _lib.lib().flour_hip_set_prefill_persistent(1)
        return out

    a, b = go(1), go(0)
    assert torch.equal(a, b)
    assert bool((a[cu[9]:cu[10]] == 0.0).all())
    for s in (0, 59):  # no large rows: the unit-scale bounds
        ref, rows = oracle_prefill(c, seqs=[s])
        max_abs, rel = errors(to_np(a)[rows], ref)
        print(f"persistent redo seq {s}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
        assert max_abs <= 2e-3 and rel <= 1e-3
    for s in (big[0], big[-1]):
        ref, rows = oracle_prefill(c, seqs=[s])
        _check_scaled(to_np(a)[rows], ref, f"persistent redo seq {s}")


@pytest.mark.parametrize("case", ["varlen", "prefix", "bs64", "f16", "v_huge", "crossings",
                                  "short_items", "long"])
def test_prefill_dma_staging_matches_register_staging(device, case):
    """Direct-to-LDS staging (K rows from the pool and V pages from a transposed fp16 staging
    copy, both by buffer loads into LDS) gives bit-identical output to register staging: ragged lengths with empty sequences and
    kv_len < q_len, prefix-cached kv, 64-token blocks, fp16 pools, V outside the fp16 range (the
    exact-mode redo), tiles straddling blocks, items of one to three kv tiles, and a long
    sequence whose block-table window moves."""
    from flour_amd import _lib
    rng = np.random.default_rng(17)
    H, G, bs, prefix, dt = 8, 2, 16, 0, torch.bfloat16
    lens = [int(x) for x in rng.integers(0, 600, size=11)]
    lens[3] = 0
    if case == "prefix":
        prefix = 96
    elif case == "bs64":
        bs, prefix = 64, 64
    elif case == "f16":
        dt = torch.float16
    elif case == "crossings":
        H, G, bs, prefix, lens = 14, 2, 32, 32, [333, 65, 1, 130]
    elif case == "short_items":
        lens = [1, 2, 63, 64, 65, 127, 128, 129, 191, 192]
    elif case == "long":
        H, G, lens = 4, 1, [4100, 70, 700]
    c = make_prefill(len(lens), H, G, 128, bs, (1, 1), prefix=prefix, dtype=dt, seed=23,
                     device=device, q_lens=lens)
    if case == "v_huge":
        c.v_new[5:9] *= 1e5  # beyond fp16 after widening: those items take the exact redo
    write(c)
    if case == "varlen":
        c.kv_lens[4] = max(int(c.kv_lens[4]) - 3, 0)  # kv_len < q_len for one sequence

    def go(mode):
        out = torch.full((c.q.shape[0], H, 128), 7.0, dtype=torch.float32, device=device)
        assert _lib.lib().flour_hip_set_prefill_dma(mode) == 0
        try:
            ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens,
                               c.block_tables, c.max_seqlen_q, c.scale, block_size=bs,
                               out_dtype=torch.float32, out=out, workspace=ops.Workspace(device))
            torch.cuda.synchronize()
        finally:
            _lib.lib().flour_hip_set_prefill_dma(1)
        return out

    a, b = go(2), go(0)
    assert torch.equal(a, b)
    ref, rows = oracle_prefill(c, seqs=[0, 1, 2])
    rel = errors(to_np(a)[rows], ref)[1]
    print(f"dma {case} rel_l2={rel:.3e}", flush=True)
    assert rel <= 1e-3


def test_prefill_long_workload_dma_staging(device):
    """The long-prompt workload (2 x 8,192 rows, Llama-3-8B heads) takes direct-to-LDS staging
    by default: bit-identical to register staging, and every row of the batch against the
    oracle (~1.1 TFLOP of causal attention on the host cores)."""
    from flour_amd import _lib
    c = make_workload("prefill_bf16_long_llama3_8b", device=device)
    write(c)

    ws = ops.Workspace(device)

    def go(mode):
        assert _lib.lib().flour_hip_set_prefill_dma(mode) == 0
        try:
            out = run(c, torch.float32, workspace=ws)
            torch.cuda.synchronize()
        finally:
            _lib.lib().flour_hip_set_prefill_dma(1)
        return out

    b = go(0)
    ws.buf.fill_(0x7F)  # the staged path rewrites every page it reads
    a = go(1)
    assert ws.buf.numel() >= ops.prefill_workspace_bytes(2, c.block_tables.shape[1],
                                                         c.block_size, 8, 128, c.q.dtype) > 0
    assert torch.equal(a, b)
    t0 = time.perf_counter()
    ref = O.paged_attention(to_np(c.q), to_np(c.k_pool), to_np(c.v_pool), to_np(c.block_tables),
                            to_np(c.cu_seqlens_q), to_np(c.kv_lens), c.block_size, c.scale,
                            bf16=True)
    max_abs, rel = errors(to_np(a), ref)
    print(f"long workload, all rows: max_abs={max_abs:.3e} rel_l2={rel:.3e} "
          f"(oracle {time.perf_counter() - t0:.1f} s)", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


def test_prefill_staged_path_under_graph_replay(device):
    """The staged path (V pre-pass into the caller's workspace, then direct-to-LDS loads)
    captured in a HIP graph and replayed, with eager work and a workspace overwrite between
    replays: each replay equals the eager call bit for bit (no allocation or capture check on
    the launch path, so nothing changes under capture)."""
    from flour_amd import _lib
    rng = np.random.default_rng(31)
    lens = [int(x) for x in rng.integers(300, 900, size=12)]
    c = make_prefill(len(lens), 16, 4, 128, 16, (1, 1), prefix=32, dtype=torch.bfloat16,
                     seed=33, device=device, q_lens=lens)
    write(c)
    ws = ops.Workspace(device)
    out = torch.empty((c.q.shape[0], 16, 128), dtype=torch.bfloat16, device=device)

    def step():
        ops.varlen_prefill(c.q, c.k_pool, c.v_pool, c.cu_seqlens_q, c.kv_lens, c.block_tables,
                           c.max_seqlen_q, c.scale, block_size=c.block_size, out=out,
                           workspace=ws)

    assert _lib.lib().flour_hip_set_prefill_dma(2) == 0
    try:
        step()
        torch.cuda.synchronize()
        eager = out.clone()
        reg = run(c, torch.bfloat16)  # no workspace: register staging
        assert torch.equal(eager, reg)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        for i in range(3):
            out.zero_()
            ws.buf.fill_(0x55)  # stale staging contents between replays
            noise = torch.randn(1 << 20, device=device).sum()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {i} differs"
            assert torch.isfinite(noise)
    finally:
        _lib.lib().flour_hip_set_prefill_dma(1)


def test_prefill_workspace_too_small_uses_register_staging(device):
    """A workspace below the size query's bytes is never touched: the call runs register
    staging, bit-identical to the call without a workspace."""
    from flour_amd import _lib
    c = make_prefill(3, 8, 2, 128, 16, (1, 1), prefix=16, dtype=torch.bfloat16, seed=35,
                     device=device, q_lens=[700, 300, 90])
    write(c)
    need = ops.prefill_workspace_bytes(3, c.block_tables.shape[1], 16, 2, 128, torch.bfloat16)
    small = ops.Workspace(device)
    small.buf = torch.full((need - 256,), 0x3C, dtype=torch.uint8, device=device)
    assert _lib.lib().flour_hip_set_prefill_dma(2) == 0
    try:
        nb = c.block_tables.shape[1]
        out = torch.empty((c.q.shape[0], 8, 128), dtype=torch.float32, device=device)
        rc = _lib.lib().flour_hip_varlen_prefill_ws(
            out.data_ptr(), 0, out.stride(0), out.stride(1), c.q.data_ptr(), c.q.stride(0),
            c.q.stride(1), c.k_pool.data_ptr(), c.v_pool.data_ptr(), c.cu_seqlens_q.data_ptr(),
            c.kv_lens.data_ptr(), c.block_tables.data_ptr(), nb, 3, c.max_seqlen_q,
            c.q.shape[0], 8, 2, 128, 16, c.k_pool.shape[1], c.scale, 1, small.buf.data_ptr(),
            small.buf.numel(), None)
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
    finally:
        _lib.lib().flour_hip_set_prefill_dma(1)
    assert torch.equal(out, run(c, torch.float32))
    assert bool((small.buf == 0x3C).all())


def test_prefill_dma_switch_rejects_bad_mode():
    from flour_amd import _lib
    assert _lib.lib().flour_hip_set_prefill_dma(3) != 0
    assert _lib.lib().flour_hip_set_prefill_dma(-1) != 0


@pytest.mark.parametrize("dt,H,G,D,bs,lens,prefix", [
    (torch.float32, 8, 8, 64, 16, [1, 17, 40, 300], 32),   # eight rows per workgroup
    (torch.float32, 16, 4, 128, 16, [129, 5], 0),           # two rows x four heads
    (torch.float32, 16, 1, 32, 7, [50, 1], 14),             # n_rep 16: two head groups
    (torch.bfloat16, 14, 2, 64, 8, [300, 77, 1], 64),       # Qwen2.5-0.5B heads, 8-token pages
    (torch.float16, 8, 2, 64, 32, [90, 33], 32),
])
def test_prefill_vector_kernel_shapes(device, dt, H, G, D, bs, lens, prefix):
    """Shapes the matrix-core prefill does not take run on the vector kernel: fp32 max-abs
    <= 1e-5 against the oracle, 16-bit pools 2e-3 / 1e-3 (fp32 output)."""
    from flour_amd import _lib
    c = make_prefill(len(lens), H, G, D, bs, (1, 1), prefix=prefix, dtype=dt, seed=H + D,
                     device=device, q_lens=lens)
    write(c)
    ref, rows = oracle_prefill(c)
    assert _lib.lib().flour_hip_set_prefill_f32_mfma(0) == 0  # fp32 at 64 / 128 too
    try:
        got = to_np(run(c, torch.float32))[rows]
    finally:
        _lib.lib().flour_hip_set_prefill_f32_mfma(1)
    max_abs, rel = errors(got, ref)
    print(f"vector prefill {dt} H={H} G={G} D={D}: max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    if dt == torch.float32:
        assert max_abs <= 1e-5
    else:
        assert max_abs <= 2e-3 and rel <= 1e-3
