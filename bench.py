#!/usr/bin/env python3
"""Benchmark of the attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--workload decode_bf16_llama3_8b]

A step is one pass of the hot path over one batch of synthetic input already resident in HBM:
for a decode workload one paged-decode launch over the whole batch; for a prefill workload
one KV write of the new rows plus one causal varlen prefill launch. The default workload is
bf16 paged decode at the Llama-3-8B attention shape (batch 64, 32 q / 8 kv heads, head_dim
128, block 16, contexts U[512, 4096], 0.1% of K channels x20).

Prints ONE JSON line: the headline value is decode HBM throughput in GB/s of algorithmic
bytes (K+V rows read once + q + out + block-table entries + context lengths) per second.
`roofline` compares the dominant kernel's average launch duration (back-to-back launches, HIP
events on the launch stream at the two ends of the timed region; events around every single
call add their own overhead and are reported beside it) against the 8 TB/s HBM peak; `cpu_baseline` is the repo's C restatement of the
reference CPU backend (oracle/) timed on this host's cores on a bounded sample of the same
workload. `extra` carries the other workloads (prefill TFLOP/s against the 2.5 PFLOP/s dense
bf16 peak, long-context decode, KV write) measured the same way.

Consecutive timed launches rotate over copies of the large inputs (pools, new rows, q), at
least 1 GiB per rotation, so every launch reads from HBM rather than from the 256 MB
Infinity Cache that a re-read of the same 577 MB pool would partly hit.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
F32_PEAK_TFLOPS = 157.3        # MI355X dense fp32 matrix, TFLOP/s


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode_bf16_llama3_8b")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the other workloads")
    ap.add_argument("--graph", action="store_true",
                    help="replay the decode step from a HIP graph instead of launching it eagerly "
                         "(measured slower than eager launches for this two-kernel step)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the baseline sample")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run plain 1 GiB device copies (a known-size reference for the "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    return ap.parse_args()


COPY_BYTES = 1 << 30


def copy_calibration():
    """Three device-to-device copies of COPY_BYTES each: every launch reads and writes exactly
    COPY_BYTES, which scales the HBM byte counters of the profiler."""
    import torch

    a = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda:0")
    a.fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": COPY_BYTES, "launches": 3}), flush=True)


def event_timed(torch, fn, steps: int, warmup: int):
    """Run fn warmup+steps times; returns (ms per step over the bracketed region, list of
    per-launch ms from events recorded around each call on the current stream)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return wall, per


def loop_timed(torch, fn, steps: int, warmup: int) -> float:
    """ms per step of `steps` back-to-back calls, bracketed by synchronisations and two events."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


# Every timed launch reads inputs that no launch of the previous ~1 GiB touched: a step
# re-reading the same pools would be served partly by the 256 MB Infinity Cache (measured: the
# Llama-3-8B decode reads 5.76 TB/s from one resident copy, 5.23 TB/s rotating over two or
# more), which is not HBM throughput.
COLD_BYTES = 1 << 30


def cold_copies(per_copy_bytes: int) -> int:
    """Copies of a step's large inputs so that one rotation touches >= COLD_BYTES (2..16)."""
    return int(max(2, min(16, -(-COLD_BYTES // max(1, per_copy_bytes)))))


def rotating(fns):
    """A callable that runs fns[0], fns[1], ... in turn, one per call."""
    state = {"i": 0}

    def run():
        f = fns[state["i"] % len(fns)]
        state["i"] += 1
        f()

    return run


def read_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by a
    copy-kernel calibration), from the committed summary profiles/<name>.pmc.md, if any."""
    p = ROOT / "profiles" / f"{name}.pmc.md"
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def cpu_decode_baseline(case, seconds: float):
    """Oracle (C restatement of cpu.rs:57-112, OpenMP over sequence x kv head) on host copies."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O  # noqa: E402  (the checker / CPU baseline, never the product)

    def host(t):
        t = t.detach().cpu().contiguous()
        return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()

    q, kp, vp = host(case.q), host(case.k_pool), host(case.v_pool)
    bt, cl = host(case.block_tables), host(case.context_lens)
    B = q.shape[0]
    cu = np.arange(B + 1, dtype=np.int32)
    threads = O.num_threads()
    run = lambda: O.paged_attention(q, kp, vp, bt, cu, cl, case.block_size, case.scale,  # noqa: E731
                                    out_dtype=np.uint16, threads=threads)
    run()  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    med = float(np.median(times))
    return med, threads, len(times)


BUNDLE = dict(num_layers=32, kv_heads=8, head_dim=128, block_size=16, prefix=1024)


def bench_bundle(torch, steps: int, warmup: int, cpu: bool):
    """FLKV export / import of a 1,024-token prefix of a Llama-3-8B-shaped cache (32 layers,
    8 kv heads, head_dim 128, bf16): the frame is 134 MB. Export = device gather into staging +
    device-to-host copy into the caller's buffer; import = host-to-device copy + scatter into
    freshly allocated blocks + bookkeeping. Both end with a stream synchronisation, so the wall
    time is the host-visible one."""
    from flour_amd.kv_cache import KvCache

    c = BUNDLE
    P, dev = c["prefix"], torch.device("cuda:0")
    mk = lambda: KvCache(c["num_layers"], P + 64, 32, c["kv_heads"], c["head_dim"],  # noqa: E731
                         torch.bfloat16, c["block_size"])
    a, b = mk(), mk()
    a.allocate_kv(P)
    g = torch.Generator(device="cpu").manual_seed(5)
    for layer in range(c["num_layers"]):
        kv = torch.randn((2, P, c["kv_heads"], c["head_dim"]), generator=g).to(torch.bfloat16).to(dev)
        a.write_kv(layer, kv[0], kv[1])
    torch.cuda.synchronize()
    ids = list(range(P))

    def timed(fn):
        for _ in range(warmup):
            fn()
        t = []
        for _ in range(steps):
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        t.sort()
        return t[len(t) // 2]

    # frames live in pinned host buffers, as a serving process would keep them for transfer
    n = a.bundle_size("llama3-8b", ids, P)
    buf = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    assert a.export_prefix_bundle("llama3-8b", ids, P, out=buf) == n
    t_exp = timed(lambda: a.export_prefix_bundle("llama3-8b", ids, P, out=buf))
    # each import registers its blocks as a cached prefix; drop that before the next one
    t_imp = timed(lambda: (b.clear_prefix_cache(), b.import_prefix_bundle(buf, ids)))
    data = bytes(buf.numpy())
    r = {"bytes": n, "export_GB/s": round(n / t_exp / 1e9, 2),
         "export_ms": round(t_exp * 1e3, 3), "import_GB/s": round(n / t_imp / 1e9, 2),
         "import_ms": round(t_imp * 1e3, 3), "host_buffer": "pinned"}
    b.clear_prefix_cache()
    b.import_prefix_bundle(buf, ids)
    assert b.export_prefix_bundle("llama3-8b", ids, P) == data  # the frame survives the trip
    if cpu:
        import numpy as np

        sys.path.insert(0, str(ROOT / "oracle"))
        import flkv as F  # noqa: E402

        pools = [[p.cpu().view(torch.int16).numpy().view(np.uint16) for p in a.pool(layer)]
                 for layer in range(c["num_layers"])]
        ks, vs = [p[0] for p in pools], [p[1] for p in pools]
        blocks = a.blocks()
        t = []
        for _ in range(3):
            t0 = time.perf_counter()
            F.export_frame("llama3-8b", ids, P, ks, vs, blocks, c["block_size"], "BF16")
            t.append(time.perf_counter() - t0)
        t.sort()
        r["cpu_export_GB/s"] = round(n / t[1] / 1e9, 3)
        r["cpu_sample"] = ("the oracle's export (numpy gather of the host pool copies + frame "
                           "encoding), whole bundle, median of 3, 1 thread")
    return r


BATCH_DECODE = dict(num_layers=32, batch=64, num_heads=32, kv_heads=8, head_dim=128,
                    block_size=16, ctx=(512, 4096), seed=2)


def bench_batch_decode(torch, steps: int, warmup: int, cpu: bool, cpu_seconds: float):
    """Continuous-batching decode over a Llama-3-8B-shaped cache (32 layers, 32 q / 8 kv heads,
    head_dim 128, bf16, block 16): 64 sequences with the decode workload's seeded contexts
    U[512, 4096] live in one KvBatch pool. A step is one flour_kv_batch_step (one new row per
    sequence: allocation + plan upload) and, for each of the 32 layers, the KV write of the 64
    new rows and paged decode attention over the whole batch, as one
    flour_kv_batch_write_kv_attention call (one decode launch that writes the new rows first,
    plus its merge). `kernels_ms` times the same layers with no step call between them, so
    step_ms - kernels_ms is the host share; `kernels_two_launch_ms` the same with the KV write
    as its own launch."""
    import types

    from flour_amd.kv_cache import KvBatch

    c = BATCH_DECODE
    L, B, H, G, D, bs = (c[k] for k in ("num_layers", "batch", "num_heads", "kv_heads",
                                        "head_dim", "block_size"))
    g = torch.Generator(device="cpu").manual_seed(c["seed"])
    ctx = torch.randint(c["ctx"][0], c["ctx"][1] + 1, (B,), generator=g).tolist()
    grow = 2 * (warmup + steps) + 2
    max_len = -(-(c["ctx"][1] + grow) // bs) * bs
    nblk = sum(-(-(n + grow) // bs) for n in ctx) + B
    b = KvBatch(L, nblk, B, max_len, B, H, G, D, torch.bfloat16, bs)
    torch.manual_seed(c["seed"] + 1000)
    for layer in range(L):
        for p in b.pool(layer):
            p.normal_()
    sids = [b.add_sequence() for _ in range(B)]
    for s, n in zip(sids, ctx):
        b.allocate_kv(s, n - 1)    # the first step brings row n
    dev = torch.device("cuda:0")
    q = torch.randn((L, B, H, D), device=dev).to(torch.bfloat16)
    k = torch.randn((L, B, G, D), device=dev).to(torch.bfloat16)
    v = torch.randn((L, B, G, D), device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    ones, scale = [1] * B, D ** -0.5
    torch.cuda.synchronize()

    def layers():
        for layer in range(L):
            b.write_kv_attention(layer, k[layer], v[layer], q[layer], scale, out=out[layer])

    def step():
        b.step(sids, ones)
        layers()

    t0 = sum(b.len(s) for s in sids)
    step_ms = loop_timed(torch, step, steps, warmup)
    t1 = sum(b.len(s) for s in sids)
    kern_ms = loop_timed(torch, layers, steps, warmup)
    lib = __import__("flour_amd._lib", fromlist=["lib"]).lib()
    lib.flour_hip_set_batch_fuse(0)
    try:
        kern2_ms = loop_timed(torch, layers, steps, warmup)
    finally:
        lib.flour_hip_set_batch_fuse(1)
    # mean live rows over the timed steps (each step adds one row per sequence)
    rows = t1 - B * (steps - 1) / 2.0
    nb = sum(len(b.blocks(s)) for s in sids)
    per_layer = rows * G * D * 2 * 2 + B * H * D * 2 * 2 + nb * 4 + B * 4 + (B * G * D * 2 * 2 * 2 + B * 4)
    nbytes = int(L * per_layer)
    assert t1 - t0 == B * (warmup + steps)
    r = {"sequences": B, "layers": L, "step_ms": round(step_ms, 4),
         "kernels_ms": round(kern_ms, 4), "kernels_two_launch_ms": round(kern2_ms, 4),
         "host_share": round(max(0.0, step_ms - kern_ms) / step_ms, 4),
         "tokens/s": round(B / (step_ms * 1e-3), 1), "algorithmic_bytes": nbytes,
         "GB/s": round(nbytes / (step_ms * 1e-3) / 1e9, 1),
         "hbm_frac": round(nbytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    if cpu:
        mb = max(len(b.blocks(s)) for s in sids)
        bt = torch.zeros((B, mb), dtype=torch.int32)
        for i, s in enumerate(sids):
            bl = b.blocks(s)
            bt[i, :len(bl)] = torch.tensor(bl, dtype=torch.int32)
        kp, vp = b.pool(0)
        case = types.SimpleNamespace(q=q[0], k_pool=kp, v_pool=vp, block_tables=bt,
                                     context_lens=torch.tensor([b.len(s) for s in sids],
                                                               dtype=torch.int32),
                                     block_size=bs, scale=scale)
        med, threads, reps = cpu_decode_baseline(case, cpu_seconds)
        r["cpu_tokens/s"] = round(B / (med * L), 2)
        r["cpu_sample"] = (f"one layer of the batch (64 sequences, C restatement of cpu.rs:57-112, "
                           f"{threads} threads, median of {reps}), x{L} layers; the KV write and "
                           "bookkeeping not counted")
        r["speedup"] = round(r["tokens/s"] / r["cpu_tokens/s"], 1)
    del b
    return r


MIXED_STEP = dict(layers=4, decoding=60, prompts=4, num_heads=32, kv_heads=8, head_dim=128,
                  block_size=16, ctx=(512, 4096), prompt=(128, 512), seed=7)


def bench_mixed_step(torch, steps: int, warmup: int):
    """One continuous-batching step in which 60 sequences decode one row each (contexts
    U[512, 4096]) while 4 prompts of U[128, 512] rows prefill, listed interleaved, at the
    Llama-3-8B attention shape (bf16, block 16): attention of the planned step timed with its
    one-row sequences on the decode kernel (one decode launch + one prefill launch over the
    packed rows) against every row on the prefill kernel. Four layers of pools rotate, so each
    launch reads from HBM."""
    from flour_amd import _lib
    from flour_amd.kv_cache import KvBatch

    c = MIXED_STEP
    L, H, G, D, bs = (c[k] for k in ("layers", "num_heads", "kv_heads", "head_dim", "block_size"))
    g = torch.Generator(device="cpu").manual_seed(c["seed"])
    ctx = torch.randint(c["ctx"][0], c["ctx"][1] + 1, (c["decoding"],), generator=g).tolist()
    pl = torch.randint(c["prompt"][0], c["prompt"][1] + 1, (c["prompts"],), generator=g).tolist()
    nblk = sum(-(-n // bs) for n in ctx + pl) + len(ctx) + len(pl)
    n_seq = len(ctx) + len(pl)
    b = KvBatch(L, nblk, n_seq, -(-c["ctx"][1] // bs) * bs, sum(pl) + len(ctx), H, G, D,
                torch.bfloat16, bs)
    torch.manual_seed(c["seed"] + 1000)
    for layer in range(L):
        for p in b.pool(layer):
            p.normal_()
    dec = [b.add_sequence() for _ in ctx]
    pro = [b.add_sequence() for _ in pl]
    for s, n in zip(dec, ctx):
        b.allocate_kv(s, n)
    for s, n in zip(pro, pl):
        b.allocate_kv(s, n)
    # prompts at four places among the decoding sequences
    order = dec[:5] + [pro[0]] + dec[5:20] + [pro[1]] + dec[20:33] + [pro[2]] + dec[33:] + [pro[3]]
    qn = [pl[pro.index(s)] if s in pro else 1 for s in order]
    b.plan(order, qn)
    T = sum(qn)
    dev = torch.device("cuda:0")
    q = torch.randn((T, H, D), device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    scale = D ** -0.5
    st = {"i": 0}

    def attn():
        b.attention(st["i"] % L, q, scale, out=out)
        st["i"] += 1

    split_ms = loop_timed(torch, attn, steps, warmup)
    assert _lib.lib().flour_hip_set_batch_split(0) == 0
    try:
        whole_ms = loop_timed(torch, attn, steps, warmup)
    finally:
        _lib.lib().flour_hip_set_batch_split(1)
    dec_bytes = sum(ctx) * G * D * 2 * 2 + len(ctx) * H * D * 2 * 2
    pf_flops = sum(H * 4 * D * n * (n + 1) // 2 for n in pl)
    del b
    return {"decoding": len(ctx), "prompts": len(pl), "prompt_rows": pl,
            "split_us": round(split_ms * 1e3, 2), "all_prefill_us": round(whole_ms * 1e3, 2),
            "speedup": round(whole_ms / split_ms, 2), "decode_bytes": dec_bytes,
            "prefill_flops": pf_flops,
            "note": "attention of one planned step (one layer); split = one paged-decode launch "
                    "over the 60 one-row sequences + one prefill launch over the 4 prompts"}


def cpu_rope_baseline(case, theta: float):
    """Oracle RoPE + KV write over the whole batch on host copies; (median seconds, runs)."""
    import numpy as np
    import torch

    from flour_amd import ops

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O  # noqa: E402

    def host(t):
        t = t.detach().cpu().contiguous()
        return t.view(torch.int16).numpy().view(np.uint16) if t.dtype in (torch.bfloat16, torch.float16) else t.numpy()

    pos, cos, sin = rope_inputs(torch, ops, case, theta)
    args = [host(case.q), host(case.k_new), host(case.v_new), host(case.k_pool).copy(),
            host(case.v_pool).copy(), host(case.slot_mapping), host(pos), host(cos), host(sin)]
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        O.rope_kv_write(*args, bf16=(case.q.dtype == torch.bfloat16))
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_prefill_baseline(case, seconds: float):
    """Oracle (C restatement of cpu.rs:57-112, OpenMP over (sequence, kv head, 16-row chunk))
    on host copies of the whole batch, the same work the GPU's TFLOP/s is measured on;
    returns (TFLOP/s, threads, runs)."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O  # noqa: E402

    def host(t):
        t = t.detach().cpu().contiguous()
        return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()

    q, kp, vp = host(case.q), host(case.k_pool), host(case.v_pool)
    bt, cu, kl = host(case.block_tables), host(case.cu_seqlens_q), host(case.kv_lens)
    threads = O.num_threads()
    f32 = case.q.dtype == torch.float32
    run = lambda: O.paged_attention(q, kp, vp, bt, cu, kl, case.block_size, case.scale,  # noqa: E731
                                    out_dtype=np.float32 if f32 else np.uint16,
                                    bf16=case.q.dtype == torch.bfloat16, threads=threads)
    run()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
        if len(times) >= 20:
            break
    med = float(np.median(times))
    return case.flops() / med / 1e12, threads, len(times)


def _dtype_names():
    import torch

    return {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


class _LazyNames(dict):
    def __missing__(self, key):
        self.update(_dtype_names())
        return dict.__getitem__(self, key)


DTYPE_NAME = _LazyNames()


def prefill_kernel_name(case) -> str:
    """The kernel a prefill workload runs on (the dispatch rule of flour_hip_varlen_prefill)."""
    import torch

    d = case.q.shape[2]
    if case.q.dtype in (torch.bfloat16, torch.float16) and d in (64, 128) and case.block_size % 16 == 0:
        return "varlen_prefill_mfma_kernel"
    if case.q.dtype == torch.float32 and d in (64, 128):
        return "prefill_f32_mfma_kernel (fp32 matrix cores)"
    return "attn_simt_kernel"


def decode_kernel_name(case) -> str:
    """Which kernel the library runs for a decode case (its dispatch rule, restated)."""
    import torch

    B, H, D = case.q.shape
    G = case.k_pool.shape[0]
    mfma = (case.q.dtype in (torch.bfloat16, torch.float16) and D in (64, 128) and
            case.block_size % 16 == 0 and H // G <= 16 and B <= 4096)
    return ("paged_decode_mfma_kernel + paged_decode_merge_kernel" if mfma
            else "attn_simt_kernel (vector ALUs)")


def launch_floor_ms(torch, steps: int, warmup: int) -> float:
    """ms per launch of an empty one-wave kernel, back to back on the current stream: the floor
    under which no launch of this library can finish."""
    from flour_amd import _lib
    from flour_amd.ops import _stream

    fn, st = _lib.lib().flour_hip_empty_launch, _stream()
    return loop_timed(torch, lambda: fn(st), max(steps, 50), warmup)


def bench_decode(torch, ops, case, steps, warmup, graph: bool = False):
    """Times decode steps. With graph=True the step (main + merge kernel) is captured once in a
    HIP graph and replayed, as a serving loop would, which removes the host launch overhead;
    the kernels and their arguments are the same as in the eager call."""
    ws = ops.DecodeWorkspace(case.q.device)
    out = torch.empty_like(case.q)
    n = cold_copies(case.k_pool.nbytes + case.v_pool.nbytes)
    kps = [case.k_pool] + [case.k_pool.clone() for _ in range(n - 1)]
    vps = [case.v_pool] + [case.v_pool.clone() for _ in range(n - 1)]

    def step(i):
        ops.paged_decode(case.q, kps[i], vps[i], case.block_tables, case.context_lens,
                         case.scale, case.max_context_len, block_size=case.block_size, out=out,
                         workspace=ws)

    runs = [ops.prepare_paged_decode(case.q, kps[i], vps[i], case.block_tables,
                                     case.context_lens, case.scale, case.max_context_len, out, ws,
                                     block_size=case.block_size) for i in range(n)]
    if graph:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step(0)  # sizes the workspace before capture
        torch.cuda.current_stream().wait_stream(side)
        graphs = []
        for i in range(n):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step(i)
            graphs.append(g)
        runs = [g.replay for g in graphs]
    run = rotating(runs)
    _, per = event_timed(torch, run, steps, warmup)  # events around every call (diagnostic)
    call_ms = sum(per) / len(per)
    # Average launch duration: back-to-back launches, events only at the two ends of the timed
    # region (per-call events add their own overhead to a ~100 us call).
    wall_ms = loop_timed(torch, run, steps, warmup)
    kern_ms = wall_ms
    nbytes = case.algorithmic_bytes()
    del kps, vps, runs
    return dict(ms_per_step=wall_ms, kernel_ms=kern_ms, call_event_ms=call_ms, bytes=nbytes, copies=n,
                gbs_step=nbytes / (wall_ms * 1e-3) / 1e9, gbs_kernel=nbytes / (kern_ms * 1e-3) / 1e9)


ROPE_THETA = {"prefill_bf16_varlen_llama3_8b": 500000.0, "prefill_bf16_prefix_qwen2_7b": 1000000.0,
              "prefill_bf16_qwen25_05b": 1000000.0}


def rope_inputs(torch, ops, case, theta):
    """Each new row's position (kv_len - q_len + i within its sequence) and the cos / sin
    tables up to the longest sequence."""
    cu = case.cu_seqlens_q.cpu().tolist()
    kl = case.kv_lens.cpu().tolist()
    pos = torch.cat([torch.arange(kl[s] - (cu[s + 1] - cu[s]), kl[s], dtype=torch.int32)
                     for s in range(len(kl))]).to(case.q.device)
    cos, sin = ops.rope_tables(max(kl), case.q.shape[2], theta, case.q.dtype, case.q.device)
    return pos, cos, sin


def rope_bytes(case) -> int:
    """Fused RoPE + KV write: read + write of every q, k and v row, one table row (cos and
    sin halves) and the slot / position per token."""
    T, H, D = case.q.shape
    G = case.k_new.shape[1]
    es = case.q.element_size()
    return 2 * T * (H + 2 * G) * D * es + T * D * es + 8 * T


def bench_prefill(torch, ops, case, steps, warmup, theta=500000.0):
    out = torch.empty_like(case.q)
    big = (case.q, case.k_new, case.v_new, case.k_pool, case.v_pool)
    n = cold_copies(sum(t.nbytes for t in big))
    sets = [big] + [tuple(t.clone() for t in big) for _ in range(n - 1)]

    def write_i(i):
        _, k, v, kp, vp = sets[i]
        ops.kv_write(k, v, kp, vp, case.slot_mapping)

    # the caller-owned workspace of the long-prompt path (V staged once into LDS-ready pages);
    # sized before the timed region, untouched by calls that stay on register staging
    ws = ops.Workspace(case.q.device)
    ws.get(ops.prefill_workspace_bytes(case.cu_seqlens_q.numel() - 1, case.block_tables.shape[1],
                                       case.block_size, case.k_pool.shape[0], case.q.shape[2],
                                       case.q.dtype))

    def attn_i(i):
        q, _, _, kp, vp = sets[i]
        ops.varlen_prefill(q, kp, vp, case.cu_seqlens_q, case.kv_lens,
                           case.block_tables, case.max_seqlen_q, case.scale,
                           block_size=case.block_size, out=out, workspace=ws)

    def step_i(i):
        write_i(i)
        attn_i(i)

    pos, cos, sin = rope_inputs(torch, ops, case, theta)
    q_rot = torch.empty_like(case.q)

    def rope_i(i):
        q, k, v, kp, vp = sets[i]
        ops.rope_kv_write(q, k, v, kp, vp, case.slot_mapping, pos, cos, sin, q_out=q_rot)

    each = lambda f: rotating([(lambda i=i: f(i)) for i in range(n)])  # noqa: E731
    wall_ms = loop_timed(torch, each(step_i), steps, warmup)
    # Per-kernel averages: back-to-back launches of that kernel alone, events only at the ends.
    w_ms = loop_timed(torch, each(write_i), steps, 1)
    a_ms = loop_timed(torch, each(attn_i), steps, 1)
    r_ms = loop_timed(torch, each(rope_i), steps, 1)
    del sets
    # The KV write's practical ceiling at its size: one contiguous device copy of the same
    # bytes (the new K and V rows), timed the same way over as many cold copies.
    nb = case.k_new.nbytes + case.v_new.nbytes
    srcs = [torch.empty(nb, dtype=torch.uint8, device=case.q.device) for _ in range(n)]
    dsts = [torch.empty(nb, dtype=torch.uint8, device=case.q.device) for _ in range(n)]
    c_ms = loop_timed(torch, rotating([(lambda i=i: dsts[i].copy_(srcs[i])) for i in range(n)]),
                      steps, 1)
    del srcs, dsts
    flops = case.flops()
    return dict(ms_per_step=wall_ms, attn_ms=a_ms, write_ms=w_ms, flops=flops, copies=n,
                copy_ms=c_ms, copy_gbs=2 * nb / (c_ms * 1e-3) / 1e9,
                tflops=flops / (a_ms * 1e-3) / 1e12, write_bytes=case.write_bytes(),
                write_gbs=case.write_bytes() / (w_ms * 1e-3) / 1e9,
                causal_pairs=case.causal_pairs(), rope_ms=r_ms, rope_bytes=rope_bytes(case),
                rope_gbs=rope_bytes(case) / (r_ms * 1e-3) / 1e9)


def prefill_line(torch, ops, case, name, cfg, args):
    """One JSON line for a prefill workload (KV write + causal varlen prefill per step)."""
    r = bench_prefill(torch, ops, case, args.steps, args.warmup, ROPE_THETA.get(name, 500000.0))
    peak = F32_PEAK_TFLOPS if case.q.dtype == torch.float32 else BF16_PEAK_TFLOPS
    line = {
        "metric": "causal varlen prefill attention throughput (useful causal FLOPs)",
        "value": round(r["flops"] / (r["ms_per_step"] * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": DTYPE_NAME[case.q.dtype],
        "data": "synthetic (seeded N(0,1); random slot mapping into a 1.25x pool)",
        "config": {"workload": name, "num_seqs": cfg["num_seqs"], "num_heads": cfg["num_heads"],
                   "kv_heads": cfg["kv_heads"], "head_dim": cfg["head_dim"],
                   "block_size": cfg["block_size"], "q_len": f"U[{cfg['q_len'][0]},{cfg['q_len'][1]}]",
                   "prefix": cfg["prefix"], "flops_per_step": r["flops"],
                   "input_copies": r["copies"]},
        "roofline": {"bound": "mfma", "kernel": prefill_kernel_name(case),
                     "achieved": round(r["tflops"], 2), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(r["tflops"] / peak, 4),
                     "avg_launch_us": round(r["attn_ms"] * 1e3, 3), "traffic": read_traffic(name)},
        "kv_write": {"GB/s": round(r["write_gbs"], 1), "hbm_frac": round(r["write_gbs"] / HBM_PEAK_GBS, 4),
                     "avg_launch_us": round(r["write_ms"] * 1e3, 3), "bytes": r["write_bytes"],
                     "traffic": read_traffic(name.replace("prefill_", "kv_write_")),
                     "same_bytes_copy": {"GB/s": round(r["copy_gbs"], 1),
                                         "hbm_frac": round(r["copy_gbs"] / HBM_PEAK_GBS, 4),
                                         "avg_launch_us": round(r["copy_ms"] * 1e3, 3)}},
        "rope_kv_write": {"GB/s": round(r["rope_gbs"], 1), "hbm_frac": round(r["rope_gbs"] / HBM_PEAK_GBS, 4),
                          "avg_launch_us": round(r["rope_ms"] * 1e3, 3), "bytes": r["rope_bytes"]},
    }
    if not args.no_cpu:
        rs, rn = cpu_rope_baseline(case, ROPE_THETA.get(name, 500000.0))
        line["rope_kv_write"]["cpu_GB/s"] = round(r["rope_bytes"] / rs / 1e9, 3)
        line["rope_kv_write"]["cpu_sample"] = (f"full batch, median of {rn} runs of the C "
                                               "restatement (attention.rs:96-104), 1 thread")
        tf, th, reps = cpu_prefill_baseline(case, args.cpu_seconds)
        line["cpu_baseline"] = {"value": round(tf, 5), "unit": "TFLOP/s", "cores": th, "kind": "port",
                                "sample": f"the whole batch (the GPU's workload), median of {reps} "
                                          "runs of the C restatement of cpu.rs:57-112, OpenMP over "
                                          "(sequence, kv head, 16-row chunk)",
                                "speedup": round(r["tflops"] / tf, 1)}
    else:
        line["cpu_baseline"] = None
    return line


def main():
    args = parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (every kernel of "
              "this path runs on a single MI355X; the multi-GPU sharding is a design note only).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from flour_amd import ops
    from flour_amd.workloads import WORKLOADS, make_workload

    dev = torch.device("cuda:0")
    name = args.workload
    if name == "kv_bundle_llama3_8b":
        r = bench_bundle(torch, args.steps, args.warmup, not args.no_cpu)
        print(json.dumps({"metric": "FLKV bundle export throughput (frame bytes, host-visible)",
                          "value": r["export_GB/s"], "unit": "GB/s", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": r["export_ms"], "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                          "data": "synthetic (seeded N(0,1) K/V)",
                          "config": dict(BUNDLE, workload=name), "bundle": r}), flush=True)
        return
    if name == "mixed_step_llama3_8b":
        r = bench_mixed_step(torch, args.steps, args.warmup)
        print(json.dumps({"metric": "continuous-batching mixed step attention (60 decoding + 4 "
                                    "prompts)", "value": r["split_us"], "unit": "us",
                          "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": r["split_us"] / 1e3, "higher_is_better": False,
                          "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                          "data": "synthetic (seeded N(0,1) pools and q)",
                          "config": dict(MIXED_STEP, workload=name), "mixed_step": r}),
              flush=True)
        return
    if name == "decode_batch_llama3_8b":
        r = bench_batch_decode(torch, args.steps, args.warmup, not args.no_cpu, args.cpu_seconds)
        print(json.dumps({"metric": "continuous-batching decode steps (64 sequences x 32 layers)",
                          "value": r["tokens/s"], "unit": "tokens/s", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup,
                          "ms_per_step": r["step_ms"], "higher_is_better": True,
                          "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                          "data": "synthetic (seeded N(0,1) pools, q, k, v)",
                          "config": dict(BATCH_DECODE, workload=name), "batch_decode": r}),
              flush=True)
        return
    cfg = WORKLOADS[name]
    case = make_workload(name, device=dev)
    torch.cuda.synchronize()
    if cfg["kind"] != "decode":
        print(json.dumps(prefill_line(torch, ops, case, name, cfg, args)), flush=True)
        return
    r = bench_decode(torch, ops, case, args.steps, args.warmup, graph=args.graph)
    value = r["gbs_step"]

    result = {
        "metric": "paged decode attention HBM throughput (algorithmic bytes)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DTYPE_NAME[case.q.dtype],
        "data": "synthetic (seeded N(0,1); block tables a random permutation of a 1.25x pool)",
        "config": {
            "workload": name, "batch": cfg["batch"], "num_heads": cfg["num_heads"],
            "kv_heads": cfg["kv_heads"], "head_dim": cfg["head_dim"],
            "block_size": cfg["block_size"], "context_lens": f"U[{cfg['ctx'][0]},{cfg['ctx'][1]}]",
            "total_context_tokens": int(case.context_lens.sum().item()),
            "algorithmic_bytes_per_step": r["bytes"], "out_dtype": DTYPE_NAME[case.q.dtype],
            "pool_copies": r["copies"],
            "launch": "HIP graph replay of the step" if args.graph else "eager",
        },
        "roofline": {
            "bound": "hbm", "kernel": decode_kernel_name(case),
            "achieved": round(r["gbs_kernel"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(r["gbs_kernel"] / HBM_PEAK_GBS, 4),
            "avg_launch_us": round(r["kernel_ms"] * 1e3, 3),
            "per_call_events_us": round(r["call_event_ms"] * 1e3, 3),
            "traffic": read_traffic(name),
        },
    }

    if not args.no_cpu:
        med, threads, reps = cpu_decode_baseline(case, args.cpu_seconds)
        cpu_gbs = r["bytes"] / med / 1e9
        result["cpu_baseline"] = {
            "value": round(cpu_gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"full batch ({cfg['batch']} sequences) of the same workload, median of "
                      f"{reps} runs ({med * 1e3:.1f} ms each) of the C restatement of "
                      "cpu.rs:57-112, OpenMP over (sequence, kv head)",
            "speedup": round(value / cpu_gbs, 1),
        }
    else:
        result["cpu_baseline"] = None

    if not args.no_extra:
        extra = {}
        for nm, c in WORKLOADS.items():
            if nm == name:
                continue
            cs = make_workload(nm, device=dev)
            torch.cuda.synchronize()
            if c["kind"] == "decode":
                rr = bench_decode(torch, ops, cs, args.steps, args.warmup)
                e = {"GB/s": round(rr["gbs_kernel"], 1),
                     "hbm_frac": round(rr["gbs_kernel"] / HBM_PEAK_GBS, 4),
                     "avg_launch_us": round(rr["kernel_ms"] * 1e3, 2),
                     "empty_launch_us": round(launch_floor_ms(torch, args.steps, args.warmup) * 1e3, 2),
                     "algorithmic_bytes": rr["bytes"],
                     "traffic": read_traffic(nm),
                     "kernel": decode_kernel_name(cs)}
                if not args.no_cpu:
                    med, th, reps = cpu_decode_baseline(cs, 3.0)
                    e["cpu_GB/s"] = round(rr["bytes"] / med / 1e9, 3)
                    e["cpu_sample"] = f"whole batch, median of {reps} runs, {th} threads"
                    e["speedup"] = round(rr["gbs_kernel"] / (rr["bytes"] / med / 1e9), 1)
                extra[nm] = e
            else:
                rr = bench_prefill(torch, ops, cs, args.steps, args.warmup, ROPE_THETA.get(nm, 500000.0))
                peak = F32_PEAK_TFLOPS if cs.q.dtype == torch.float32 else BF16_PEAK_TFLOPS
                e = {"TFLOP/s": round(rr["tflops"], 1),
                     "mfma_frac": round(rr["tflops"] / peak, 4), "peak_TFLOP/s": peak,
                     "kernel": prefill_kernel_name(cs),
                     "attn_us": round(rr["attn_ms"] * 1e3, 2), "flops": rr["flops"],
                     "traffic": read_traffic(nm),
                     "kv_write_traffic": read_traffic(nm.replace("prefill_", "kv_write_")),
                     "kv_write_GB/s": round(rr["write_gbs"], 1),
                     "kv_write_us": round(rr["write_ms"] * 1e3, 2),
                     "same_bytes_copy_GB/s": round(rr["copy_gbs"], 1),
                     "rope_kv_write_GB/s": round(rr["rope_gbs"], 1),
                     "rope_kv_write_us": round(rr["rope_ms"] * 1e3, 2),
                     "step_ms": round(rr["ms_per_step"], 4)}
                if not args.no_cpu:
                    tf, th, reps = cpu_prefill_baseline(cs, 3.0)
                    e["cpu_TFLOP/s"] = round(tf, 5)
                    e["cpu_sample"] = f"whole batch, median of {reps} runs, {th} threads"
                    e["speedup"] = round(rr["tflops"] / tf, 1)
                extra[nm] = e
            del cs
            torch.cuda.empty_cache()
        extra["kv_bundle_llama3_8b"] = bench_bundle(torch, 5, 2, not args.no_cpu)
        torch.cuda.empty_cache()
        extra["decode_batch_llama3_8b"] = bench_batch_decode(torch, 10, 3, not args.no_cpu, 3.0)
        torch.cuda.empty_cache()
        extra["mixed_step_llama3_8b"] = bench_mixed_step(torch, 20, 5)
        torch.cuda.empty_cache()
        result["extra"] = extra

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
