"""Helpers shared by the parity tests: host copies for the oracle and tolerance checks."""
from __future__ import annotations

import numpy as np
import torch


def to_np(t: torch.Tensor) -> np.ndarray:
    """Host copy; bf16/f16 come back as their uint16 bit patterns (the oracle's storage)."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def bf16_bits_to_f32(u: np.ndarray) -> np.ndarray:
    return (u.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round to nearest even (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (u >> 16) & 1
    return ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)


def errors(got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    """(max-abs error, relative L2 error) of got against ref."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    diff = got - ref
    max_abs = float(np.max(np.abs(diff))) if diff.size else 0.0
    den = float(np.linalg.norm(ref))
    rel_l2 = float(np.linalg.norm(diff) / den) if den > 0 else float(np.linalg.norm(diff))
    return max_abs, rel_l2


def bf16_ulp_distance(got_bits: np.ndarray, ref_f32: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between bf16 results and RNE(fp32 reference)."""
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(ordered(got_bits) - ordered(f32_to_bf16_bits(ref_f32)))


SMALL = 2.0 ** -10  # below this |ref|, one bf16 ulp (<= 2^-18) is finer than fp32 kernel error


def check_bf16_output(got_bits: np.ndarray, got32: np.ndarray, ref: np.ndarray) -> dict:
    """The bf16-output contract.

    (a) the bf16 output is exactly round-to-nearest-even of the kernel's own fp32 result;
    (b) it is within 1 bf16 ulp of RNE(fp32 reference) wherever |ref| >= 2^-10, and within
        1e-5 absolute below that (where a bf16 ulp is smaller than fp32 accumulation error).
    Also reports the raw bf16-vs-fp32-reference figures next to the rounding floor.
    """
    assert np.array_equal(got_bits, f32_to_bf16_bits(got32)), "bf16 output != RNE(fp32 result)"
    big = np.abs(ref) >= SMALL
    ulps = bf16_ulp_distance(got_bits, ref)
    max_ulp = int(ulps[big].max()) if big.any() else 0
    got_f = bf16_bits_to_f32(got_bits)
    small_err = float(np.max(np.abs(got_f[~big] - ref[~big]))) if (~big).any() else 0.0
    raw_abs, raw_rel = errors(got_f, ref)
    floor_abs, floor_rel = errors(bf16_bits_to_f32(f32_to_bf16_bits(ref)), ref)
    rep = dict(max_ulp=max_ulp, small_abs=small_err, raw_max_abs=raw_abs, raw_rel_l2=raw_rel,
               floor_max_abs=floor_abs, floor_rel_l2=floor_rel)
    assert max_ulp <= 1, rep
    assert small_err <= 1e-5, rep
    return rep
