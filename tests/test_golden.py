"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): expected outputs
from torch's float64 scaled_dot_product_attention over the gathered K/V and from numpy
fancy-index scatter, i.e. from implementations independent of the oracle and of the kernels.

CPU: the oracle reproduces every fixture. GPU: the kernels reproduce them through the C-ABI
(attention within the fp32 bound, the KV write bit for bit).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O
from _util import errors

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_decode_fixture():
    f = load("decode_gqa4_d64.npz")
    B = len(f["context_lens"])
    got = O.paged_attention(f["q"], f["k_pool"], f["v_pool"], f["block_tables"],
                            np.arange(B + 1, dtype=np.int32), f["context_lens"],
                            int(f["block_size"]), float(f["scale"]))
    ma, rl = errors(got, f["expected"])
    assert ma <= 1e-5 and rl <= 1e-6, (ma, rl)


def test_oracle_reproduces_prefill_fixture():
    f = load("prefill_gqa2_d128.npz")
    got = O.paged_attention(f["q"], f["k_pool"], f["v_pool"], f["block_tables"],
                            f["cu_seqlens_q"], f["kv_lens"], int(f["block_size"]),
                            float(f["scale"]))
    ma, rl = errors(got, f["expected"])
    assert ma <= 1e-5 and rl <= 1e-6, (ma, rl)


def test_oracle_reproduces_kv_write_fixture():
    f = load("kv_write_scatter.npz")
    kp, vp = f["k_pool"].copy(), f["v_pool"].copy()
    O.kv_write_scatter(f["k"], f["v"], kp, vp, f["slot_mapping"])
    assert np.array_equal(kp, f["k_expected"]) and np.array_equal(vp, f["v_expected"])


def _bf16_dev(a, device):
    return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).to(device)


@pytest.mark.gpu
def test_decode_kernel_reproduces_fixture(device):
    from flour_amd import ops

    f = load("decode_gqa4_d64.npz")
    q = _bf16_dev(f["q"], device)
    kp, vp = _bf16_dev(f["k_pool"], device), _bf16_dev(f["v_pool"], device)
    bt = torch.from_numpy(f["block_tables"]).to(device)
    cl = torch.from_numpy(f["context_lens"]).to(device)
    out = ops.paged_decode(q, kp, vp, bt, cl, float(f["scale"]), int(cl.max()),
                           block_size=int(f["block_size"]), out_dtype=torch.float32)
    ma, rl = errors(out.cpu().numpy(), f["expected"])
    assert ma <= 1e-5 and rl <= 1e-5, (ma, rl)


@pytest.mark.gpu
def test_prefill_kernel_reproduces_fixture(device):
    from flour_amd import ops

    f = load("prefill_gqa2_d128.npz")
    q = _bf16_dev(f["q"], device)
    kp, vp = _bf16_dev(f["k_pool"], device), _bf16_dev(f["v_pool"], device)
    cu = torch.from_numpy(f["cu_seqlens_q"]).to(device)
    kl = torch.from_numpy(f["kv_lens"]).to(device)
    bt = torch.from_numpy(f["block_tables"]).to(device)
    max_q = int(np.diff(f["cu_seqlens_q"]).max())
    out = ops.varlen_prefill(q, kp, vp, cu, kl, bt, max_q, float(f["scale"]),
                             block_size=int(f["block_size"]), out_dtype=torch.float32)
    ma, rl = errors(out.cpu().numpy(), f["expected"])
    assert ma <= 2e-3 and rl <= 1e-3, (ma, rl)


@pytest.mark.gpu
def test_kv_write_kernel_reproduces_fixture(device):
    from flour_amd import ops

    f = load("kv_write_scatter.npz")
    k, v = _bf16_dev(f["k"], device), _bf16_dev(f["v"], device)
    kp, vp = _bf16_dev(f["k_pool"], device), _bf16_dev(f["v_pool"], device)
    sm = torch.from_numpy(f["slot_mapping"]).to(device)
    ops.kv_write(k, v, kp, vp, sm)
    torch.cuda.synchronize()
    got_k = kp.cpu().view(torch.int16).numpy().view(np.uint16)
    got_v = vp.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got_k, f["k_expected"]) and np.array_equal(got_v, f["v_expected"])
