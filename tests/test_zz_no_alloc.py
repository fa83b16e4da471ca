"""flour_hip_paged_decode_noalloc: paged decode whose split-context workspace is the library's
per-GPU scratch array instead of a caller buffer. It must give exactly what
flour_hip_paged_decode gives with a caller workspace (same kernels, same split), on calls in a
row that reuse the scratch (the second one smaller), and meet the decode tolerance against
the oracle's paged_attention (src/backend/cpu.rs:57-112): fp32 output max-abs <= 2e-3 and
rel-L2 <= 1e-3 for bf16 pools.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from _util import errors, to_np
from flour_amd import _lib, ops
from flour_amd.workloads import make_decode

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _args(c, out):
    B, H, D = c.q.shape
    G, num_slots, _ = c.k_pool.shape
    return [_p(out), ops.dtype_code(out.dtype), _p(c.q), _p(c.k_pool), _p(c.v_pool),
            _p(c.block_tables), c.block_tables.shape[1], _p(c.context_lens), B, H, G, D,
            c.block_size, num_slots, c.max_context_len, float(c.scale), ops.dtype_code(c.q.dtype)]


def noalloc(c, out_dtype=torch.float32):
    out = torch.full(c.q.shape, float("nan"), dtype=out_dtype, device=c.q.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().flour_hip_paged_decode_noalloc(*_args(c, out), stream))
    torch.cuda.synchronize()
    return out


def with_workspace(c, out_dtype=torch.float32):
    out = torch.full(c.q.shape, float("nan"), dtype=out_dtype, device=c.q.device)
    nbytes = ops.decode_workspace_bytes(c.q.shape[0], c.q.shape[1], c.k_pool.shape[0],
                                        c.q.shape[2], c.max_context_len)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=c.q.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().flour_hip_paged_decode(*_args(c, out), _p(ws), ws.numel(), stream))
    torch.cuda.synchronize()
    return out


def oracle_decode(c):
    B = c.q.shape[0]
    return O.paged_attention(to_np(c.q), to_np(c.k_pool), to_np(c.v_pool), to_np(c.block_tables),
                             np.arange(B + 1, dtype=np.int32), to_np(c.context_lens),
                             c.block_size, c.scale, bf16=True)


def test_noalloc_matches_workspace_entry_on_two_calls_in_a_row(device):
    big = make_decode(24, 32, 8, 128, 16, (1, 4096), dtype=torch.bfloat16, seed=41,
                      device=device, k_outlier_frac=0.001, k_outlier_scale=20.0)
    small = make_decode(3, 28, 4, 128, 16, (1, 900), dtype=torch.bfloat16, seed=42,
                        device=device)
    for tag, c in (("big", big), ("small", small)):
        print(f"noalloc case {tag}: q {tuple(c.q.shape)} max_ctx {c.max_context_len}", flush=True)
        got = noalloc(c)
        ref_ws = with_workspace(c)
        assert torch.equal(got, ref_ws), f"{tag}: differs from flour_hip_paged_decode"
        max_abs, rel = errors(to_np(got), oracle_decode(c))
        print(f"noalloc {tag}: max_abs={max_abs:.3e} rel_l2={rel:.3e}", flush=True)
        assert max_abs <= 2e-3 and rel <= 1e-3
    # bf16 output through the same scratch, after the two calls above
    assert torch.equal(noalloc(small, torch.bfloat16), with_workspace(small, torch.bfloat16))


def test_noalloc_rejects_a_workspace_beyond_its_scratch(device):
    """With the split forced to 4096 waves, a GQA group of 16 needs ~68 MB of partials, more
    than the 40 MiB scratch: the call fails on the host before any launch."""
    lib = _lib.lib()
    assert lib.flour_hip_paged_decode_noalloc_max_workspace() == 40 << 20
    c = make_decode(2, 16, 1, 128, 16, (1, 64), dtype=torch.bfloat16, seed=43, device=device)
    out = torch.zeros(c.q.shape, dtype=torch.float32, device=device)
    assert lib.flour_hip_set_decode_workgroups(4096) == 0
    try:
        rc = lib.flour_hip_paged_decode_noalloc(*_args(c, out), None)
    finally:
        lib.flour_hip_set_decode_workgroups(0)
    assert rc == _lib.ERR_WORKSPACE
    assert "scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert bool((out == 0).all())


def test_noalloc_graph_replay_matches_eager(device):
    """The allocation-free call captured in a HIP graph (the use it exists for) and replayed,
    with eager allocation-free calls of another batch between replays (they rewrite the shared
    scratch), gives the eager result bit for bit on every replay."""
    c = make_decode(16, 32, 8, 128, 16, (1, 3000), dtype=torch.bfloat16, seed=44, device=device)
    other = make_decode(5, 28, 4, 128, 16, (1, 2000), dtype=torch.bfloat16, seed=45,
                        device=device)
    eager = noalloc(c)
    other_ref = noalloc(other)
    out = torch.empty(c.q.shape, dtype=torch.float32, device=device)
    lib = _lib.lib()

    def step():
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.flour_hip_paged_decode_noalloc(*_args(c, out), stream))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for i in range(4):
        out.zero_()
        assert torch.equal(noalloc(other), other_ref), f"eager call before replay {i} differs"
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs"
