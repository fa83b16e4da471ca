"""Pins the oracle's RoPE + KV-write restatement (oracle_rope_kv_write) before it is trusted.

The reference applies candle_nn::rotary_emb::rope to q and k (src/models/common/attention.rs:
96-99) with the tables of Cache::new (cache.rs:377-393), then write_kv (:104). candle is not
vendored and the reference's tests hold no RoPE vectors, so the restatement is pinned by what
the mathematics fixes:
  * position 0 (cos 1, sin 0) is the identity, bit for bit, and a quarter / half turn is an
    exact permutation with sign changes of the halves (non-interleaved "rotate half" pairs);
  * against an fp64 rotation with the same table values, every element is within the bound of
    one rounding per product and one per sum in the element type;
  * the table builder follows cache.rs:377-393 (theta_i = rope_theta^(-2i/d), angle = pos *
    theta_i, then cos / sin) within fp32 error;
  * tokens with a padding slot write no K/V, tokens without a table row write nothing;
  * planted mistakes (interleaved pairs, rotation sign) are each caught.
The last bit of the rounding sequence (each operation rounded in the element type, as candle's
CPU kernel evaluates it in half::bf16 / f16 arithmetic) is restated, not pinned.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from _util import bf16_bits_to_f32, f32_to_bf16_bits
from flour_amd import ops

U = {"f32": 2.0 ** -24, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}  # unit roundoff


def to_store(x: np.ndarray, dt: str) -> np.ndarray:
    if dt == "f32":
        return x.astype(np.float32)
    if dt == "bf16":
        return f32_to_bf16_bits(x.astype(np.float32))
    return x.astype(np.float16).view(np.uint16)


def to_f32(x: np.ndarray, dt: str) -> np.ndarray:
    if dt == "f32":
        return x
    if dt == "bf16":
        return bf16_bits_to_f32(x)
    return x.view(np.float16).astype(np.float32)


def tables(max_pos: int, D: int, theta: float, dt: str):
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dt]
    c, s = ops.rope_tables(max_pos, D, theta, tdt)
    if dt == "f32":
        return c.numpy(), s.numpy()
    return (c.view(torch.int16).numpy().view(np.uint16), s.view(torch.int16).numpy().view(np.uint16))


def run(dt, T=6, H=4, G=2, D=16, positions=None, slots=None, cos=None, sin=None, seed=0,
        num_slots=32):
    rng = np.random.default_rng(seed)
    q = to_store(rng.standard_normal((T, H, D)), dt)
    k = to_store(rng.standard_normal((T, G, D)), dt)
    v = to_store(rng.standard_normal((T, G, D)), dt)
    if cos is None:
        cos, sin = tables(64, D, 10000.0, dt)
    positions = np.arange(T, dtype=np.int32) if positions is None else np.asarray(positions, np.int32)
    slots = rng.permutation(num_slots)[:T].astype(np.int32) if slots is None else np.asarray(slots, np.int32)
    kp = np.zeros((G, num_slots, D), q.dtype)
    vp = np.zeros((G, num_slots, D), q.dtype)
    qo, skipped = O.rope_kv_write(q, k, v, kp, vp, slots, positions, cos, sin,
                                  bf16=(dt == "bf16"), q_out=np.zeros_like(q))
    return dict(q=q, k=k, v=v, qo=qo, kp=kp, vp=vp, slots=slots, pos=positions, cos=cos,
                sin=sin, skipped=skipped)


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_position_zero_is_identity(dt):
    r = run(dt, positions=np.zeros(6, np.int32))
    assert np.array_equal(r["qo"], r["q"])
    for t, s in enumerate(r["slots"]):
        assert np.array_equal(r["kp"][:, s], r["k"][t]) and np.array_equal(r["vp"][:, s], r["v"][t])


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_quarter_and_half_turns_are_exact(dt):
    D = 16
    c = np.zeros((3, D // 2), np.float32)
    s = np.zeros((3, D // 2), np.float32)
    c[1], s[1] = 0.0, 1.0    # quarter turn: (x1, x2) -> (-x2, x1)
    c[2], s[2] = -1.0, 0.0   # half turn: (x1, x2) -> (-x1, -x2)
    r = run(dt, D=D, positions=[1, 2, 1, 2, 1, 2], cos=to_store(c, dt), sin=to_store(s, dt))
    q, qo = to_f32(r["q"], dt), to_f32(r["qo"], dt)
    h = D // 2
    for t in range(6):
        if r["pos"][t] == 1:
            assert np.array_equal(qo[t, :, :h], -q[t, :, h:]) and np.array_equal(qo[t, :, h:], q[t, :, :h])
        else:
            assert np.array_equal(qo[t], -q[t])


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("theta", [10000.0, 500000.0])
def test_matches_fp64_rotation_within_rounding(dt, theta):
    D, T = 128, 40
    cos, sin = tables(4096, D, theta, dt)
    pos = np.random.default_rng(1).integers(0, 4096, T)
    r = run(dt, T=T, H=3, G=2, D=D, positions=pos, cos=cos, sin=sin, num_slots=64)
    h = D // 2
    c = to_f32(cos, dt)[pos].astype(np.float64)[:, None, :]
    s = to_f32(sin, dt)[pos].astype(np.float64)[:, None, :]
    for x, y in [(r["q"], r["qo"]), (r["k"], r["kp"].transpose(1, 0, 2)[r["slots"]])]:
        x = to_f32(x, dt).astype(np.float64)
        y = to_f32(y, dt).astype(np.float64)
        x1, x2 = x[..., :h], x[..., h:]
        exact1, exact2 = x1 * c - x2 * s, x1 * s + x2 * c
        # one rounding per product and one per sum: |err| <= 2u (|a| + |b|) (+ u^2 terms)
        bound1 = 2.01 * U[dt] * (np.abs(x1 * c) + np.abs(x2 * s)) + 1e-30
        bound2 = 2.01 * U[dt] * (np.abs(x1 * s) + np.abs(x2 * c)) + 1e-30
        assert np.all(np.abs(y[..., :h] - exact1) <= bound1)
        assert np.all(np.abs(y[..., h:] - exact2) <= bound2)
        # a rotation keeps the norm of every pair
        n_in, n_out = np.hypot(x1, x2), np.hypot(y[..., :h], y[..., h:])
        assert np.all(np.abs(n_out - n_in) <= 4.1 * U[dt] * (n_in + 1e-30))


@pytest.mark.parametrize("theta", [10000.0, 500000.0, 1000000.0])
def test_tables_follow_cache_rs_377(theta):
    D, P = 128, 8192
    c, s = ops.rope_tables(P, D, theta, torch.float32)
    i = np.arange(D // 2)
    th = np.float32(1.0) / np.power(np.float32(theta), (2 * i).astype(np.float32) / np.float32(D))
    ang = np.arange(P, dtype=np.float64)[:, None] * th.astype(np.float64)[None, :]
    tol = 4 * 2.0 ** -24 * (1.0 + ang)  # fp32 theta and product rounding, then cos / sin
    assert np.all(np.abs(c.numpy() - np.cos(ang)) <= tol)
    assert np.all(np.abs(s.numpy() - np.sin(ang)) <= tol)
    assert np.array_equal(c[0].numpy(), np.ones(D // 2, np.float32))
    assert np.array_equal(s[0].numpy(), np.zeros(D // 2, np.float32))
    cb, sb = ops.rope_tables(P, D, theta, torch.bfloat16)
    assert torch.equal(cb, c.to(torch.bfloat16)) and torch.equal(sb, s.to(torch.bfloat16))


def test_padding_slot_and_missing_position():
    r = run("bf16", T=4, positions=[0, 5, 64, -1], slots=[3, -1, 7, 9], num_slots=16)
    assert r["skipped"] == 2
    assert np.array_equal(r["qo"][2:], np.zeros_like(r["qo"][2:]))  # no table row: untouched
    assert np.any(r["qo"][1] != 0)                                    # q rotated without a slot
    assert np.array_equal(r["kp"][:, 3], r["k"][0])
    written = {3}
    for s in range(16):
        if s not in written:
            assert not r["kp"][:, s].any() and not r["vp"][:, s].any()


# ------------------------------------------------------------------ planted mistakes

def _battery() -> list[str]:
    failed = []
    for dt in ["f32", "bf16"]:
        try:
            test_quarter_and_half_turns_are_exact(dt)
        except AssertionError:
            failed.append(f"turns-{dt}")
        try:
            test_matches_fp64_rotation_within_rounding(dt, 10000.0)
        except AssertionError:
            failed.append(f"fp64-{dt}")
    return failed


def test_battery_passes_on_faithful_oracle():
    O.set_mutation(O.MUT_NONE)
    assert _battery() == []


@pytest.mark.parametrize("mut", [O.MUT_ROPE_INTERLEAVED, O.MUT_ROPE_SIGN])
def test_planted_mistake_is_caught(mut):
    O.set_mutation(mut)
    try:
        assert _battery() != [], f"mutation {mut} slipped through the pinning checks"
    finally:
        O.set_mutation(O.MUT_NONE)
