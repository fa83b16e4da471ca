"""Many sequences over one pool (flour_kv_batch_*) on the GPU, against the oracle.

A step plans the batch once and every layer runs the KV write and attention over it. Each
sequence's output is checked against the oracle's paged_attention (cpu.rs:57-112) over that
sequence's own block table in the shared pool: a mixed prefill of sequences of different
lengths, decode steps for all of them (the paged decode kernel), a shared cached prefix matched
through the common registry with the suffixes prefilled in one call, sequences removed and
added between steps, and the fused RoPE + KV write of a planned step (bit-exact against the
oracle's rope_kv_write). Tolerances as for the kernels: bf16 max-abs <= 2e-3 and rel-L2 <= 1e-3
against the fp32 oracle (fp32 output).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from _util import errors, to_np
from flour_amd import _lib, ops
from flour_amd.kv_cache import KvBatch

pytestmark = pytest.mark.gpu

H, G, D, BS = 16, 4, 128, 16
SCALE = D ** -0.5


def make(num_blocks=512, max_seqs=8, max_seq_len=1024, tokens=4096, layers=2):
    return KvBatch(layers, num_blocks, max_seqs, max_seq_len, tokens, H, G, D, torch.bfloat16, BS)


def rows(n, g, scale=1.0):
    return (torch.randn((n, G, D), generator=g) * scale).to(torch.bfloat16).cuda()


def step(b, layer, sids, qn, g, plan=True):
    """Plan, write new K/V rows, attend: returns (q, out) packed in plan order."""
    if plan:
        b.plan(sids, qn)
    T = sum(qn)
    k, v = rows(T, g), rows(T, g)
    b.write_kv(layer, k, v)
    q = torch.randn((T, H, D), generator=g).to(torch.bfloat16).cuda()
    out = b.attention(layer, q, SCALE, out_dtype=torch.float32)
    torch.cuda.synchronize()
    return q, out


def check(b, layer, sids, qn, q, out, tag):
    kp, vp = (to_np(t) for t in b.pool(layer))
    mb = max(len(b.blocks(s)) for s in sids)
    bt = np.zeros((len(sids), mb), np.int32)
    for i, s in enumerate(sids):
        bl = b.blocks(s)
        bt[i, :len(bl)] = bl
    cu = np.concatenate([[0], np.cumsum(qn)]).astype(np.int32)
    kl = np.array([b.len(s) for s in sids], np.int32)
    ref = O.paged_attention(to_np(q), kp, vp, bt, cu, kl, BS, SCALE, bf16=True)
    max_abs, rel = errors(to_np(out), ref)
    print(f"{tag}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


def test_mixed_prefill_then_decode_steps(device):
    g = torch.Generator(device="cpu").manual_seed(1)
    b = make()
    lens = [300, 17, 1, 129, 512, 64]
    sids = [b.add_sequence() for _ in lens]
    for s, n in zip(sids, lens):
        b.allocate_kv(s, n)
    for layer in range(2):
        q, out = step(b, layer, sids, lens, g)
        check(b, layer, sids, lens, q, out, f"prefill layer {layer}")
    for t in range(3):  # decode steps: one new row per sequence, the paged decode kernel
        if t == 0:       # allocate_kv per sequence, then plan once per layer
            for s in sids:
                b.allocate_kv(s, 1)
        else:            # flour_kv_batch_step: allocation + plan in one call, kept by all layers
            b.step(sids, [1] * len(sids))
        for layer in range(2):
            q, out = step(b, layer, sids, [1] * len(sids), g, plan=t == 0)
            check(b, layer, sids, [1] * len(sids), q, out, f"decode {t} layer {layer}")


def test_shared_prefix_through_the_registry(device):
    """One sequence computes and registers a 256-token prefix; five more match it from the
    shared registry (same physical blocks) and prefill their own suffixes in one call."""
    g = torch.Generator(device="cpu").manual_seed(2)
    b = make()
    prefix = list(range(1000, 1256))
    s0 = b.add_sequence()
    assert b.match_prefix(s0, prefix + [1]) == 0
    b.allocate_kv(s0, 256 + 1)
    step(b, 0, [s0], [257], g)
    b.register_prefix(s0, prefix + [1])
    shared = b.blocks(s0)[:16]
    others, suffix = [], [33, 1, 200, 77, 128]
    for n in suffix:
        s = b.add_sequence()
        assert b.match_prefix(s, prefix + list(range(n))) == 256
        assert b.blocks(s) == shared
        b.allocate_kv(s, n)
        others.append(s)
    assert all(b.ref_count(x) == 7 for x in shared)  # s0, the registry and five sequences
    q, out = step(b, 0, others, suffix, g)
    check(b, 0, others, suffix, q, out, "suffixes over the shared prefix")


def test_sequences_leave_and_join_between_steps(device):
    g = torch.Generator(device="cpu").manual_seed(3)
    b = make(num_blocks=64)
    sids = [b.add_sequence() for _ in range(4)]
    for s in sids:
        b.allocate_kv(s, 100)
    step(b, 0, sids, [100] * 4, g)
    free = b.free_blocks()
    b.remove_sequence(sids[1])
    assert b.free_blocks() == free + 7
    s_new = b.add_sequence()
    assert s_new == sids[1]
    b.allocate_kv(s_new, 40)
    live = [sids[0], s_new, sids[2], sids[3]]
    q, out = step(b, 0, live, [1, 40, 1, 1], g)  # decode rows and a new prefill together
    check(b, 0, live, [1, 40, 1, 1], q, out, "after churn")
    b.allocate_kv(sids[0], 1)
    with pytest.raises(_lib.FlourError, match="no current plan"):
        b.write_kv(0, rows(1, g), rows(1, g))


def test_rope_write_then_attention(device):
    """flour_kv_batch_rope_write_kv: RoPE at each planned row's position in its sequence (the
    reference's rope_for_cache rows, attention.rs:96-99), rotated k and v into the layer's
    pool (attention.rs:104), q rotated: bit-exact against the oracle's rope_kv_write on the
    same rows with slots and positions derived on the host from each sequence's blocks; then
    attention over the rotated rows against paged_attention. A prefill step, then a decode
    step."""
    g = torch.Generator(device="cpu").manual_seed(4)
    b = make(max_seq_len=1024)
    cos, sin = ops.rope_tables(1024, D, 500000.0, torch.bfloat16, device)
    sids = [b.add_sequence() for _ in range(3)]
    for qn in ([70, 1, 33], [1, 1, 1]):
        b.step(sids, qn)
        T = sum(qn)
        q = torch.randn((T, H, D), generator=g).to(torch.bfloat16).cuda()
        k, v = rows(T, g), rows(T, g)
        kp0, vp0 = (to_np(t).copy() for t in b.pool(1))
        pos, slots = [], []
        for s, n in zip(sids, qn):
            bl, L = b.blocks(s), b.len(s)
            for p in range(L - n, L):
                pos.append(p)
                slots.append(bl[p // BS] * BS + p % BS)
        q_ref, _ = O.rope_kv_write(to_np(q), to_np(k), to_np(v), kp0, vp0,
                                   np.array(slots, np.int32), np.array(pos, np.int32),
                                   to_np(cos), to_np(sin), bf16=True)
        q_rot = b.rope_write_kv(1, q, k, v, cos, sin)
        torch.cuda.synchronize()
        kp, vp = (to_np(t) for t in b.pool(1))
        assert np.array_equal(to_np(q_rot), q_ref)
        assert np.array_equal(kp, kp0) and np.array_equal(vp, vp0)
        out = b.attention(1, q_rot, SCALE, out_dtype=torch.float32)
        torch.cuda.synchronize()
        check(b, 1, sids, qn, q_rot, out, f"rope + attention, rows {qn}")
    with pytest.raises(_lib.FlourError, match="cover"):
        short_cos, short_sin = ops.rope_tables(512, D, 500000.0, torch.bfloat16, device)
        b.rope_write_kv(1, q, k, v, short_cos, short_sin)


def _fill(b, sids, lens, layer, seed):
    """Context rows for the listed sequences, written through planned steps (KV write only)."""
    gd = torch.Generator(device="cuda").manual_seed(seed)
    G_, D_ = b.kv_heads, b.head_dim
    for i in range(0, len(sids), 8):
        ids, ns = sids[i:i + 8], lens[i:i + 8]
        b.step(ids, ns)
        T = sum(ns)
        k = torch.randn((T, G_, D_), generator=gd, device="cuda").to(b.dtype)
        v = torch.randn((T, G_, D_), generator=gd, device="cuda").to(b.dtype)
        b.write_kv(layer, k, v)


def test_mixed_step_runs_decode_rows_on_the_decode_kernel(device):
    """A continuous-batching step at the Llama-3-8B attention shape: 60 sequences decoding one
    row each over contexts U[512, 4096] while 4 prompts of U[128, 512] rows prefill, listed
    interleaved. The one-row sequences run as one paged-decode launch and the prompts as one
    prefill launch, each over its rows of the packed layout: every row against the oracle,
    the decode rows bit-identical to paged_decode over those sequences alone, the prompt rows
    bit-identical to varlen_prefill over the prompts alone, and the all-prefill route (the
    split switched off) against the oracle too."""
    Hq, Gk, Dh = 32, 8, 128
    rng = np.random.default_rng(41)
    b = KvBatch(1, 10000, 64, 4096 + 16, 8 * 4096, Hq, Gk, Dh, torch.bfloat16, BS)
    n_dec = 60
    ctx = [int(x) for x in rng.integers(512, 4097, size=n_dec)]
    prompts = [int(x) for x in rng.integers(128, 513, size=4)]
    dec = [b.add_sequence() for _ in range(n_dec)]
    _fill(b, dec, [c - 1 for c in ctx], 0, 5)
    pro = [b.add_sequence() for _ in prompts]
    order = dec[:5] + [pro[0]] + dec[5:20] + [pro[1]] + dec[20:33] + [pro[2]] + dec[33:] + [pro[3]]
    qn = [prompts[pro.index(s)] if s in pro else 1 for s in order]
    b.step(order, qn)
    T = sum(qn)
    gd = torch.Generator(device="cuda").manual_seed(6)
    k = torch.randn((T, Gk, Dh), generator=gd, device="cuda").to(torch.bfloat16)
    v = torch.randn((T, Gk, Dh), generator=gd, device="cuda").to(torch.bfloat16)
    b.write_kv(0, k, v)
    q = torch.randn((T, Hq, Dh), generator=gd, device="cuda").to(torch.bfloat16)
    split = b.attention(0, q, SCALE, out_dtype=torch.float32)
    assert _lib.lib().flour_hip_set_batch_split(0) == 0
    try:
        whole = b.attention(0, q, SCALE, out_dtype=torch.float32)
    finally:
        _lib.lib().flour_hip_set_batch_split(1)
    torch.cuda.synchronize()

    kp, vp = (to_np(t) for t in b.pool(0))
    mb = max(len(b.blocks(s)) for s in order)
    bt = np.zeros((len(order), mb), np.int32)
    for i, s in enumerate(order):
        bl = b.blocks(s)
        bt[i, :len(bl)] = bl
    cu = np.concatenate([[0], np.cumsum(qn)]).astype(np.int32)
    kl = np.array([b.len(s) for s in order], np.int32)
    ref = O.paged_attention(to_np(q), kp, vp, bt, cu, kl, BS, SCALE, bf16=True)
    for tag, out in (("split", split), ("all-prefill", whole)):
        max_abs, rel = errors(to_np(out), ref)
        print(f"mixed step {tag}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
        assert max_abs <= 2e-3 and rel <= 1e-3

    # the decode rows are the decode kernel's over the one-row sequences alone
    di = [i for i, n in enumerate(qn) if n == 1]
    d_rows = torch.tensor(cu[di], dtype=torch.long, device=device)
    d_bt = torch.tensor(bt[di], device=device)
    d_ctx = torch.tensor(kl[di], device=device)
    alone = ops.paged_decode(q[d_rows].contiguous(), *b.pool(0), d_bt, d_ctx, SCALE,
                             int(kl[di].max()), block_size=BS, out_dtype=torch.float32)
    assert torch.equal(split[d_rows], alone)
    # the prompt rows are the prefill kernel's over the prompts alone
    pi = [i for i, n in enumerate(qn) if n > 1]
    p_rows = torch.cat([torch.arange(cu[i], cu[i + 1]) for i in pi]).to(device)
    p_cu = torch.tensor(np.concatenate([[0], np.cumsum([qn[i] for i in pi])]), dtype=torch.int32,
                        device=device)
    p_out = ops.varlen_prefill(q[p_rows].contiguous(), *b.pool(0), p_cu,
                               torch.tensor(kl[pi], device=device),
                               torch.tensor(bt[pi], device=device), max(qn), SCALE,
                               block_size=BS, out_dtype=torch.float32)
    assert torch.equal(split[p_rows], p_out)


@pytest.mark.parametrize("Hq,Gk,Dh,bs", [(32, 8, 128, 16), (14, 2, 64, 16), (16, 4, 128, 32)])
def test_fused_write_and_decode_equals_two_launches(device, Hq, Gk, Dh, bs):
    """flour_kv_batch_write_kv_attention on a decode step: the decode kernel writes each new K / V
    row into the pool before it attends to it, in one launch. Output (fp32 and bf16) and both
    pools bit-identical to the KV write followed by the attention (the switch set to two
    launches), and the output against the oracle. Contexts put the new position at every place
    of its 16-token tile (1 .. 48 tokens) next to long ones (U[512, 3000]), so workgroup ranges
    start and end inside, at and past a pair's last chunk. 32-token pages take the two launches
    (the fused instantiation is built for 16-token pages) and must give the same."""
    rng = np.random.default_rng(Dh + bs)
    b = KvBatch(1, 12000 // (bs // 16), 64, 3072, 64 * 3072, Hq, Gk, Dh, torch.bfloat16, bs)
    ctx = list(range(1, 49)) + [int(x) for x in rng.integers(512, 3001, size=16)]
    sids = [b.add_sequence() for _ in ctx]
    _fill(b, [s for s, c in zip(sids, ctx) if c > 1], [c - 1 for c in ctx if c > 1], 0, 11)
    b.step(sids, [1] * len(sids))
    assert [b.len(s) for s in sids] == ctx
    n = len(sids)
    gd = torch.Generator(device="cuda").manual_seed(12)
    k = torch.randn((n, Gk, Dh), generator=gd, device="cuda").to(torch.bfloat16)
    v = torch.randn((n, Gk, Dh), generator=gd, device="cuda").to(torch.bfloat16)
    q = torch.randn((n, Hq, Dh), generator=gd, device="cuda").to(torch.bfloat16)
    kp, vp = b.pool(0)
    kp0, vp0 = kp.clone(), vp.clone()

    def run(fuse, out_dtype):
        kp.copy_(kp0)
        vp.copy_(vp0)
        assert _lib.lib().flour_hip_set_batch_fuse(fuse) == 0
        try:
            out = b.write_kv_attention(0, k, v, q, SCALE, out_dtype=out_dtype)
        finally:
            _lib.lib().flour_hip_set_batch_fuse(1)
        torch.cuda.synchronize()
        return out, kp.clone(), vp.clone()

    for od in (torch.float32, torch.bfloat16):
        f_out, f_k, f_v = run(1, od)
        u_out, u_k, u_v = run(0, od)
        assert torch.equal(f_k, u_k) and torch.equal(f_v, u_v)
        assert not torch.equal(f_k, kp0)  # the new rows were written
        assert torch.equal(f_out, u_out)
    f_out, _, _ = run(1, torch.float32)
    mb = max(len(b.blocks(s)) for s in sids)
    bt = np.zeros((n, mb), np.int32)
    for i, s in enumerate(sids):
        bl = b.blocks(s)
        bt[i, :len(bl)] = bl
    cu = np.arange(n + 1, dtype=np.int32)
    kl = np.array([b.len(s) for s in sids], np.int32)
    ref = O.paged_attention(to_np(q), to_np(kp), to_np(vp), bt, cu, kl, bs, SCALE, bf16=True)
    max_abs, rel = errors(to_np(f_out), ref)
    print(f"fused write + decode H={Hq} G={Gk} D={Dh} bs={bs}: max_abs={max_abs:.3e} "
          f"rel_l2={rel:.3e}", flush=True)
    assert max_abs <= 2e-3 and rel <= 1e-3


def test_fused_entry_point_runs_other_steps_as_two_calls(device):
    """A mixed step (and a prefill step) through flour_kv_batch_write_kv_attention takes the
    KV write and the attention as two calls: the same pools and output as calling them."""
    g = torch.Generator(device="cpu").manual_seed(13)
    b = make()
    sids = [b.add_sequence() for _ in range(3)]
    for qn in ([40, 7, 1], [1, 1, 5]):
        b.step(sids, qn)
        T = sum(qn)
        k, v = rows(T, g), rows(T, g)
        q = torch.randn((T, H, D), generator=g).to(torch.bfloat16).cuda()
        kp, vp = b.pool(0)
        kp0, vp0 = kp.clone(), vp.clone()
        out = b.write_kv_attention(0, k, v, q, SCALE, out_dtype=torch.float32)
        torch.cuda.synchronize()
        k1, v1 = kp.clone(), vp.clone()
        kp.copy_(kp0)
        vp.copy_(vp0)
        b.write_kv(0, k, v)
        ref = b.attention(0, q, SCALE, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(kp, k1) and torch.equal(vp, v1) and torch.equal(out, ref)
        check(b, 0, sids, qn, q, out, f"write + attention in one call, rows {qn}")
