"""Kernel (2) parity: paged decode attention against the oracle's restatement of
paged_attention (src/backend/cpu.rs:57-112) for seq_q == 1, on identical seeded inputs.

Tolerances (written here, per the path's contract):
  * fp32 pools:                      max-abs <= 1e-5 against the fp32 oracle;
  * bf16 pools, fp32 output:         max-abs <= 2e-3 and rel-L2 <= 1e-3 against the fp32
                                     oracle (the kernel's fp32 accumulator, before rounding);
  * bf16 pools, bf16 output:         exactly RNE(kernel fp32 result); rel-L2 within 5% of the
                                     floor set by rounding the exact result to bf16 (~1.5e-3,
                                     above the fp32 limit), max-abs within floor + 2e-3, and
                                     within 1 bf16 ulp of RNE(reference) where |ref| >= 2^-10.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from _util import DECODE_ULP_BOUNDS, check_bf16_output, errors, to_np
from flour_amd import ops
from flour_amd.workloads import make_decode, make_workload

pytestmark = pytest.mark.gpu


def oracle_decode(c) -> np.ndarray:
    B = c.q.shape[0]
    return O.paged_attention(to_np(c.q), to_np(c.k_pool), to_np(c.v_pool), to_np(c.block_tables),
                             np.arange(B + 1, dtype=np.int32), to_np(c.context_lens),
                             c.block_size, c.scale, bf16=(c.q.dtype != torch.float16))


def run(c, out_dtype=None):
    out = ops.paged_decode(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens, c.scale,
                           c.max_context_len, block_size=c.block_size, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out


def check_bf16(c, tag=""):
    ref = oracle_decode(c)
    got32 = to_np(run(c, torch.float32))
    max_abs, rel = errors(got32, ref)
    print(f"{tag} fp32-out max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3
    rep = check_bf16_output(to_np(run(c, torch.bfloat16)), got32, ref, DECODE_ULP_BOUNDS)
    print(f"{tag} bf16-out {rep}", flush=True)
    return max_abs, rel


def test_decode_fp32_workload(device):
    """fp32 decode: batch 4, 8/8 heads, head_dim 64, contexts U[1, 256]."""
    c = make_workload("decode_f32_b4_h8_d64", device=device)
    got = to_np(run(c))
    ref = oracle_decode(c)
    max_abs, _ = errors(got, ref)
    print(f"fp32 workload max_abs={max_abs:.3e}", flush=True)
    assert max_abs <= 1e-5


@pytest.mark.parametrize("H,G,D,bs,ctx", [
    (2, 2, 4, 3, [7]),            # the reference's decode-step test shape (cpu.rs:208-224)
    (4, 2, 4, 4, [6, 1, 9]),      # GQA
    (8, 8, 64, 16, [1, 16, 17, 255]),
    (6, 3, 96, 5, [33, 2]),
])
def test_decode_fp32_small_shapes(device, H, G, D, bs, ctx):
    c = make_decode(len(ctx), H, G, D, bs, (1, 1), dtype=torch.float32, seed=H * D + bs,
                    device=device, context_lens=ctx)
    max_abs, _ = errors(to_np(run(c)), oracle_decode(c))
    assert max_abs <= 1e-5


@pytest.mark.parametrize("H,G,ctx", [
    (32, 8, [1, 2, 15, 16, 17, 31, 63, 64, 65, 100]),   # partial tiles, one split
    (8, 8, [1000, 513, 2049]),                          # n_rep 1, several splits
    (28, 4, [1500, 40, 777]),                           # n_rep 7 (Qwen2 shape)
    (64, 8, [3000, 5]),                                 # n_rep 8
    (16, 1, [4100, 300]),                               # n_rep 16
])
def test_decode_bf16_mfma_shapes(device, H, G, ctx):
    c = make_decode(len(ctx), H, G, 128, 16, (1, 1), dtype=torch.bfloat16, seed=H + G,
                    device=device, context_lens=ctx)
    check_bf16(c, f"H={H} G={G}")


def test_decode_bf16_block_size_32(device):
    c = make_decode(3, 16, 4, 128, 32, (1, 1), dtype=torch.bfloat16, seed=77, device=device,
                    context_lens=[31, 32, 1000])
    check_bf16(c, "bs32")


def test_decode_f16(device):
    c = make_decode(3, 16, 4, 128, 16, (1, 1), dtype=torch.float16, seed=78, device=device,
                    context_lens=[31, 600, 1000])
    ref = oracle_decode(c)
    max_abs, rel = errors(to_np(run(c, torch.float32)), ref)
    assert max_abs <= 2e-3 and rel <= 1e-3


def test_decode_llama3_8b_workload(device):
    """bf16 decode, batch 64, 32/8 heads, contexts U[512, 4096], 0.1% K outlier channels x20."""
    c = make_workload("decode_bf16_llama3_8b", device=device)
    print(f"outliers={c.meta['k_outlier_channels']}", flush=True)
    check_bf16(c, "llama3-8b decode")


def test_decode_long_context_workload(device):
    """bf16 decode, batch 8, 64/8 heads, contexts U[16384, 32768] (split-context merge)."""
    c = make_workload("decode_bf16_long_llama3_70b", device=device)
    check_bf16(c, "long-context decode")


def test_decode_repeat_calls_reuse_workspace(device):
    """A reused (never cleared) workspace gives identical results call after call, also when
    a smaller batch runs in between and when stale bytes fill it."""
    c = make_decode(5, 32, 8, 128, 16, (2000, 5000), dtype=torch.bfloat16, seed=21, device=device)
    small = make_decode(2, 32, 8, 128, 16, (600, 900), dtype=torch.bfloat16, seed=22, device=device)
    ws = ops.DecodeWorkspace(device)
    args = lambda x: (x.q, x.k_pool, x.v_pool, x.block_tables, x.context_lens, x.scale,  # noqa: E731
                      x.max_context_len)
    a = ops.paged_decode(*args(c), workspace=ws)
    ws.buf.fill_(0x7f)  # stale garbage must not leak into results
    s1 = ops.paged_decode(*args(small), workspace=ws)
    b = ops.paged_decode(*args(c), workspace=ws)
    s2 = ops.paged_decode(*args(small), workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(s1, s2)


@pytest.mark.parametrize("w", [0, 2, 16])
@pytest.mark.parametrize("nwg", [1, 3, 7, 100, 513, 4096])
def test_decode_workgroup_partitions_agree(device, nwg, w):
    """Any number of workgroups and any weighting of the ranges between even and odd workgroups
    (hence any cut of the chunk list into pieces, including more workgroups than chunks and
    empty ranges) meets the same fp32-accumulator bound."""
    from flour_amd import _lib
    c = make_decode(6, 32, 8, 128, 16, (1, 5000), dtype=torch.bfloat16, seed=23, device=device,
                    context_lens=[4999, 1, 0, 33, 2048, 700])
    ref = oracle_decode(c)
    lib = _lib.lib()
    assert lib.flour_hip_set_decode_workgroups(nwg) == 0
    assert lib.flour_hip_set_decode_xcd_weight(w) == 0
    try:
        got = to_np(run(c, torch.float32))
    finally:
        lib.flour_hip_set_decode_workgroups(0)
        lib.flour_hip_set_decode_xcd_weight(2)
    max_abs, rel = errors(got, ref)
    assert max_abs <= 2e-3 and rel <= 1e-3
    assert not got[2].any()  # empty context


def test_decode_block_permutation_invariance(device):
    """The same logical cache in other physical blocks gives bit-identical outputs."""
    c = make_decode(4, 32, 8, 128, 16, (100, 3000), dtype=torch.bfloat16, seed=31, device=device)
    a = run(c, torch.float32)
    nb = c.k_pool.shape[1] // 16
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(1)).to(device)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb, device=device)
    # physical block p moves to perm[p]
    kp = c.k_pool.view(8, nb, 16, 128)[:, inv].reshape_as(c.k_pool).contiguous()
    vp = c.v_pool.view(8, nb, 16, 128)[:, inv].reshape_as(c.v_pool).contiguous()
    bt = perm[c.block_tables.long()].to(torch.int32).contiguous()
    b = ops.paged_decode(c.q, kp, vp, bt, c.context_lens, c.scale, c.max_context_len,
                         out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_decode_empty_context_gives_zeros(device):
    c = make_decode(2, 8, 2, 128, 16, (1, 1), dtype=torch.bfloat16, seed=3, device=device,
                    context_lens=[0, 5])
    out = to_np(run(c, torch.float32))
    assert not out[0].any()
    ref = oracle_decode(c)
    assert errors(out[1], ref[1])[0] <= 2e-3


def test_decode_graph_replay_matches_eager(device):
    """The decode step (main + merge kernel) captured in a HIP graph and replayed, with eager
    work and synchronisations between replays, gives the eager result bit for bit each time."""
    d = make_decode(16, 32, 8, 128, 16, (1, 3000), dtype=torch.bfloat16, seed=9, device=device)
    ws = ops.DecodeWorkspace(device)
    eager = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens, d.scale,
                             d.max_context_len, workspace=ws)
    torch.cuda.synchronize()
    out = torch.empty_like(d.q)

    def step():
        ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens, d.scale,
                         d.max_context_len, out=out, workspace=ws)

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


def test_decode_batch_beyond_the_mfma_limit_uses_the_generic_kernel(device):
    """5000 sequences (past the 4096-sequence bound of the MFMA decode) still decode correctly
    on the generic kernel; short contexts keep the oracle fast."""
    d = make_decode(5000, 8, 2, 128, 16, (1, 40), dtype=torch.bfloat16, seed=3, device=device)
    out = ops.paged_decode(d.q, d.k_pool, d.v_pool, d.block_tables, d.context_lens, d.scale,
                           d.max_context_len, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref = O.paged_attention(to_np(d.q), to_np(d.k_pool), to_np(d.v_pool), to_np(d.block_tables),
                            np.arange(5001, dtype=np.int32), to_np(d.context_lens), 16, d.scale)
    max_abs, rel = errors(to_np(out), ref)
    assert max_abs <= 2e-3 and rel <= 1e-3, (max_abs, rel)


def test_decode_context_beyond_max_context_len_is_clamped_on_every_path(device):
    """context_lens[b] above max_context_len attends the first max_context_len positions, on
    the MFMA path (bf16) and on the generic path (fp32 pools) alike."""
    for dt, tol in ((torch.bfloat16, 2e-3), (torch.float32, 1e-5)):
        c = make_decode(3, 8, 2, 128, 16, (1, 1), dtype=dt, seed=5, device=device,
                        context_lens=[300, 700, 40])
        out = ops.paged_decode(c.q, c.k_pool, c.v_pool, c.block_tables, c.context_lens, c.scale,
                               500, out_dtype=torch.float32)
        torch.cuda.synchronize()
        clamped = np.minimum(to_np(c.context_lens), 500).astype(np.int32)
        ref = O.paged_attention(to_np(c.q), to_np(c.k_pool), to_np(c.v_pool),
                                to_np(c.block_tables), np.arange(4, dtype=np.int32), clamped, 16,
                                c.scale, bf16=True)
        max_abs, _ = errors(to_np(out), ref)
        assert max_abs <= tol, (dt, max_abs)


def test_decode_v_far_from_unit_scale(device):
    """V rows of +-1e5, one of +-3e38 per sequence and rows of 1e-30 among N(0, 1) rows: the
    decode P.V runs in the pool's own type (bf16 V is never narrowed) with an exact running
    max, so every weight is at most 1. Judged relative to the output scale."""
    c = make_decode(4, 16, 4, 128, 16, (1, 1), dtype=torch.bfloat16, seed=8, device=device,
                    context_lens=[900, 37, 2000, 513])
    vp = c.v_pool.float()
    g = torch.Generator(device="cpu").manual_seed(9)
    for b, n in enumerate(c.context_lens.tolist()):
        pos = torch.randperm(n, generator=g)[:6]
        sl = [int(c.block_tables[b, p // 16]) * 16 + int(p) % 16 for p in pos]
        vp[:, sl[0], :] = 3e38 * torch.sign(vp[:, sl[0], :])
        for s_ in sl[1:3]:
            vp[:, s_, :] *= 1e5
        for s_ in sl[3:]:
            vp[:, s_, :] = 1e-30
    c.v_pool.copy_(vp.to(torch.bfloat16))
    ref = oracle_decode(c)
    got = to_np(run(c, torch.float32))
    fin = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), fin)
    scale = float(np.abs(ref[fin]).max())
    max_abs, rel = errors(got[fin] / scale, ref[fin] / scale)
    print(f"decode V far from unit scale: scale={scale:.3e} max_abs={max_abs:.3e} rel={rel:.3e}",
          flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


@pytest.mark.parametrize("dt,H,G,D,bs,ctx", [
    (torch.float32, 8, 8, 64, 16, [1, 2, 255, 256]),     # the fp32 decode workload's shape
    (torch.float32, 16, 2, 128, 16, [1000, 3]),          # fp32 at head_dim 128, n_rep 8
    (torch.float32, 32, 2, 32, 7, [77, 500]),            # n_rep 16: two head groups; odd pages
    (torch.float32, 4, 4, 256, 16, [300]),               # one lane group per wave
    (torch.bfloat16, 14, 2, 64, 16, [1, 900, 2049]),     # Qwen2.5-0.5B attention shape
    (torch.float16, 8, 4, 64, 32, [33, 700]),
    (torch.bfloat16, 8, 2, 16, 16, [5, 130]),            # two lanes per row
])
def test_decode_vector_kernel_shapes(device, dt, H, G, D, bs, ctx):
    """Shapes the matrix-core decode does not take (fp32 pools, head_dim != 128, any page
    size) run on the vector kernel: fp32 max-abs <= 1e-5, 16-bit pools 2e-3 / 1e-3."""
    c = make_decode(len(ctx), H, G, D, bs, (1, 1), dtype=dt, seed=H * D + bs, device=device,
                    context_lens=ctx)
    got = to_np(run(c, torch.float32))
    ref = O.paged_attention(to_np(c.q), to_np(c.k_pool), to_np(c.v_pool), to_np(c.block_tables),
                            np.arange(len(ctx) + 1, dtype=np.int32), to_np(c.context_lens), bs,
                            c.scale, bf16=(dt != torch.float16))
    max_abs, rel = errors(got, ref)
    print(f"vector decode {dt} H={H} G={G} D={D}: max_abs={max_abs:.3e} rel={rel:.3e}", flush=True)
    if dt == torch.float32:
        assert max_abs <= 1e-5
    else:
        assert max_abs <= 2e-3 and rel <= 1e-3


@pytest.mark.parametrize("H,G,ctx", [
    (14, 2, [1, 2, 15, 16, 17, 31, 63, 64, 65, 100]),   # n_rep 7, partial tiles
    (8, 8, [1000, 513, 2049]),                          # n_rep 1, several splits
    (32, 2, [3000, 5]),                                 # n_rep 16
])
def test_decode_bf16_mfma_head_dim_64(device, H, G, ctx):
    """The matrix-core decode at head_dim 64 (Qwen2.5-0.5B-sized heads): 8-byte lane loads,
    K through the LDS tile, V^T packed in-lane, 16-dim output blocks."""
    c = make_decode(len(ctx), H, G, 64, 16, (1, 1), dtype=torch.bfloat16, seed=H + G + 64,
                    device=device, context_lens=ctx)
    check_bf16(c, f"D=64 H={H} G={G}")


def test_decode_head_dim_64_workload(device):
    """bf16 decode, batch 64, 14 q / 2 kv heads, head_dim 64, contexts U[512, 4096]."""
    c = make_workload("decode_bf16_qwen25_05b", device=device)
    check_bf16(c, "qwen2.5-0.5b decode")
