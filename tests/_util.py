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


def max_ulp_above(got_bits: np.ndarray, ref: np.ndarray, exp2: int) -> int:
    """Largest bf16-ulp distance from RNE(ref) over the elements with |ref| >= 2^exp2."""
    big = np.abs(ref) >= 2.0 ** exp2
    return int(bf16_ulp_distance(got_bits, ref)[big].max()) if big.any() else 0


# Largest distance, in bf16 ulps, between a kernel's bf16 output and RNE(fp32 reference), by
# magnitude of the reference (|ref| >= 2^e for each key e). A bf16 ulp at 2^e is 2^(e-7): the
# decode accumulator (P split hi + lo, ~1e-6 relative) is within one ulp of the exact result
# wherever |ref| >= 2^-10. The default prefill (P rounded once to fp16) has an fp32 max-abs
# error of up to ~6e-4 at the configs, so its bound at |ref| >= 2^e is 1 + 6e-4 / 2^(e-7)
# ulps, rounded up: 2 at 2^-4, 12 at 2^-7 and 96 at 2^-10 (measured maxima: 1, 5 and 73).
DECODE_ULP_BOUNDS = {-10: 1}
PREFILL_ULP_BOUNDS = {-4: 2, -7: 12, -10: 96}


def check_bf16_output(got_bits: np.ndarray, got32: np.ndarray, ref: np.ndarray,
                      ulp_bounds: dict[int, int] | None = None) -> dict:
    """The bf16-output contract.

    Rounding an exact fp32 result to bf16 already costs rel-L2 ~1.5e-3 (the "floor"), above the
    1e-3 fp32 limit, so the bf16 output is judged against that floor:
    (a) the bf16 output is exactly round-to-nearest-even of the kernel's own fp32 result
        (whose own error is checked separately against 2e-3 max-abs / 1e-3 rel-L2);
    (b) its rel-L2 against the fp32 reference is within 5% of the floor's;
    (c) its max-abs is within the floor's plus the fp32 max-abs bound (2e-3);
    (d) with `ulp_bounds` {e: n}, it is within n bf16 ulps of RNE(reference) wherever
        |ref| >= 2^e.
    """
    assert np.array_equal(got_bits, f32_to_bf16_bits(got32)), "bf16 output != RNE(fp32 result)"
    got_f = bf16_bits_to_f32(got_bits)
    raw_abs, raw_rel = errors(got_f, ref)
    floor_abs, floor_rel = errors(bf16_bits_to_f32(f32_to_bf16_bits(ref)), ref)
    ulps = {e: max_ulp_above(got_bits, ref, e) for e in (-10, -7, -4, -2)}
    rep = dict(raw_max_abs=raw_abs, raw_rel_l2=raw_rel, floor_max_abs=floor_abs,
               floor_rel_l2=floor_rel, max_ulp_vs_rne_ref=ulps)
    assert raw_rel <= 1.05 * floor_rel + 1e-5, rep
    assert raw_abs <= floor_abs + 2e-3, rep
    for e, n in (ulp_bounds or {}).items():
        assert max_ulp_above(got_bits, ref, e) <= n, (f"more than {n} bf16 ulps from "
                                                      f"RNE(reference) where |ref| >= 2^{e}", rep)
    return rep
