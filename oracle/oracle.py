"""ctypes binding of oracle/liboracle.so — the CPU restatement of flour's attention hot path.

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg as the checker / CPU baseline; never by the product path (flour_amd/).

Functions mirror the reference (lltsdyp/flour) — see flour_oracle.c for file:line citations:
  slot / slots                  src/models/common/paged.rs:114-121
  kv_write_scatter              src/models/common/paged.rs:186-187 (documented semantics)
  kv_write_reference_loop       src/models/common/paged.rs:192-202 (literal loop, :196 quirk)
  paged_attention               src/backend/cpu.rs:57-112
  dense_attention_f64           src/backend/cpu.rs:24-42, :148-165 (in fp64)
  rope_kv_write                 src/models/common/attention.rs:96-104 (rope(q), rope(k) as
                                candle_nn::rotary_emb::rope, then the write_kv scatter)
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

F32, BF16, F16 = 0, 1, 2
_NP_CODE = {np.dtype(np.float32): F32}

MUT_NONE, MUT_MASK_OFF_BY_ONE, MUT_NO_CORRECTION, MUT_WRONG_KV_HEAD = 0, 1, 2, 3
MUT_NO_SCALE, MUT_OFFSET_ZERO, MUT_SLOT_SWAP = 4, 5, 6
MUT_ROPE_INTERLEAVED, MUT_ROPE_SIGN = 7, 8

_lib = None
_vp, _i64, _int, _f = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.oracle_slot.restype = _i64
        L.oracle_slot.argtypes = [_vp, _int, _i64]
        L.oracle_slots.argtypes = [_vp, _int, _i64, _i64, _vp]
        L.oracle_kv_write_scatter.restype = _i64
        L.oracle_kv_write_scatter.argtypes = [_vp, _vp, _i64, _i64, _vp, _vp, _vp, _int, _int, _int,
                                              _i64, _int]
        L.oracle_kv_write_reference_loop.restype = _int
        L.oracle_kv_write_reference_loop.argtypes = [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _i64,
                                                     _int]
        L.oracle_kv_write_quirk_index.restype = _int
        L.oracle_kv_write_quirk_index.argtypes = [_vp, _int]
        L.oracle_rope_kv_write.argtypes = [_vp, _vp, _i64, _i64, _int, _vp, _vp, _i64, _i64, _vp,
                                           _vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _i64,
                                           _int]
        L.oracle_rope_kv_write.restype = _i64
        L.oracle_paged_attention.restype = _int
        L.oracle_paged_attention.argtypes = [_vp, _int, _i64, _i64, _vp, _int, _i64, _i64, _vp, _vp,
                                             _int, _i64, _vp, _int, _vp, _vp, _int, _int, _int, _int,
                                             _int, _f, _int]
        L.oracle_dense_attention_f64.restype = _int
        L.oracle_dense_attention_f64.argtypes = [_vp, _vp, _int, _i64, _i64, _vp, _vp, _int, _i64,
                                                 _vp, _int, _vp, _vp, _int, _int, _int, _int, _int,
                                                 ctypes.c_double]
        L.oracle_set_mutation.argtypes = [_int]
        L.oracle_num_threads.restype = _int
        for n in ("oracle_f32_to_bf16", "oracle_bf16_to_f32", "oracle_f32_to_f16",
                  "oracle_f16_to_f32"):
            getattr(L, n).argtypes = [_vp, _vp, _i64]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def _code(a: np.ndarray, bf16: bool) -> int:
    """uint16 arrays are bf16 (or f16 when bf16=False); float32 is F32."""
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.uint16:
        return BF16 if bf16 else F16
    raise TypeError(f"oracle takes float32 or uint16 storage, got {a.dtype}")


# ------------------------------------------------------------------ conversions
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_bf16(_p(x), _p(y), x.size)
    return y


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    y = np.empty(x.shape, np.float32)
    lib().oracle_bf16_to_f32(_p(x), _p(y), x.size)
    return y


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_f16(_p(x), _p(y), x.size)
    return y


def f16_to_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    y = np.empty(x.shape, np.float32)
    lib().oracle_f16_to_f32(_p(x), _p(y), x.size)
    return y


# ------------------------------------------------------------------ paged.rs
def slot(blocks, block_size: int, pos: int) -> int:
    b = np.ascontiguousarray(blocks, dtype=np.int32)
    return int(lib().oracle_slot(_p(b), block_size, pos))


def slots(blocks, block_size: int, start: int, end: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.int32)
    out = np.empty(max(end - start, 0), np.uint32)
    lib().oracle_slots(_p(b), block_size, start, end, _p(out))
    return out


def kv_write_scatter(k: np.ndarray, v: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray,
                     slot_mapping: np.ndarray, bf16: bool = True) -> int:
    """In place: pool[h, slot[t], :] = k[t, h, :]; k/v (T, G, D) contiguous. Returns #skipped."""
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    T, G, D = k.shape
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int32)
    assert k_pool.flags.c_contiguous and v_pool.flags.c_contiguous
    return int(lib().oracle_kv_write_scatter(_p(k), _p(v), G * D, D, _p(k_pool), _p(v_pool), _p(sm),
                                             T, G, D, k_pool.shape[1], _code(k, bf16)))


def kv_write_reference_loop(k_ref: np.ndarray, v_ref: np.ndarray, k_pool: np.ndarray,
                            v_pool: np.ndarray, slots_u32: np.ndarray, bf16: bool = True) -> int:
    """Literal paged.rs:192-202 loop; k_ref/v_ref in the reference layout (G, seq, D)."""
    k_ref = np.ascontiguousarray(k_ref)
    v_ref = np.ascontiguousarray(v_ref)
    G, S, D = k_ref.shape
    s = np.ascontiguousarray(slots_u32, dtype=np.uint32)
    return int(lib().oracle_kv_write_reference_loop(_p(k_ref), _p(v_ref), _p(k_pool), _p(v_pool),
                                                    _p(s), S, G, D, k_pool.shape[1],
                                                    _code(k_ref, bf16)))


def kv_write_quirk_index(slots_u32: np.ndarray) -> int:
    s = np.ascontiguousarray(slots_u32, dtype=np.uint32)
    return int(lib().oracle_kv_write_quirk_index(_p(s), s.size))


def rope_kv_write(q: np.ndarray, k: np.ndarray, v: np.ndarray, k_pool: np.ndarray,
                  v_pool: np.ndarray, slot_mapping: np.ndarray, positions: np.ndarray,
                  cos: np.ndarray, sin: np.ndarray, bf16: bool = True,
                  q_out: np.ndarray | None = None) -> tuple[np.ndarray, int]:
    """RoPE on q (T, H, D) and k (T, G, D), then the scatter of rope(k) and v into the pools
    (in place). Returns (rope(q), tokens skipped for their position); rows of skipped tokens
    keep what ``q_out`` held (a new uninitialised array by default). Tables (max_pos, D/2)."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    cos = np.ascontiguousarray(cos)
    sin = np.ascontiguousarray(sin)
    T, H, D = q.shape
    G = k.shape[1]
    assert k_pool.flags.c_contiguous and v_pool.flags.c_contiguous
    sm = np.ascontiguousarray(slot_mapping, dtype=np.int32)
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    if q_out is None:
        q_out = np.empty_like(q)
    assert q_out.shape == q.shape and q_out.dtype == q.dtype and q_out.flags.c_contiguous
    n = lib().oracle_rope_kv_write(_p(q_out), _p(q), H * D, D, H, _p(k), _p(v), G * D, D,
                                   _p(k_pool), _p(v_pool), _p(sm), _p(pos), _p(cos), _p(sin),
                                   cos.shape[0], T, G, D, k_pool.shape[1], _code(q, bf16))
    return q_out, int(n)


# ------------------------------------------------------------------ cpu.rs
def paged_attention(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray,
                    block_tables: np.ndarray, cu_seqlens_q: np.ndarray, kv_lens: np.ndarray,
                    block_size: int, scale: float, out_dtype=np.float32, bf16: bool = True,
                    threads: int = 0) -> np.ndarray:
    """Batched restatement of paged_attention. q (total_q, H, D); pools (G, num_slots, D).

    Storage: float32 or uint16 (bf16 when bf16=True, else f16). Returns (total_q, H, D) in
    float32 (out_dtype=np.float32) or uint16 (out_dtype=np.uint16, same 16-bit format).
    """
    q = np.ascontiguousarray(q)
    T, H, D = q.shape
    G, num_slots, _ = k_pool.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cu = np.ascontiguousarray(cu_seqlens_q, dtype=np.int32)
    kl = np.ascontiguousarray(kv_lens, dtype=np.int32)
    out = np.empty((T, H, D), dtype=out_dtype)
    oc = F32 if out.dtype == np.float32 else (BF16 if bf16 else F16)
    rc = lib().oracle_paged_attention(_p(out), oc, H * D, D, _p(q), _code(q, bf16), H * D, D,
                                      _p(np.ascontiguousarray(k_pool)),
                                      _p(np.ascontiguousarray(v_pool)), _code(k_pool, bf16),
                                      num_slots, _p(bt), bt.shape[1], _p(cu), _p(kl), cu.size - 1,
                                      H, G, D, block_size, float(scale), threads)
    if rc != 0:
        raise ValueError("oracle_paged_attention: bad arguments")
    return out


def dense_attention_f64(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray,
                        block_tables: np.ndarray, cu_seqlens_q: np.ndarray, kv_lens: np.ndarray,
                        block_size: int, scale: float, bf16: bool = True) -> np.ndarray:
    q = np.ascontiguousarray(q)
    T, H, D = q.shape
    G, num_slots, _ = k_pool.shape
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cu = np.ascontiguousarray(cu_seqlens_q, dtype=np.int32)
    kl = np.ascontiguousarray(kv_lens, dtype=np.int32)
    out = np.empty((T, H, D), dtype=np.float64)
    rc = lib().oracle_dense_attention_f64(_p(out), _p(q), _code(q, bf16), H * D, D,
                                          _p(np.ascontiguousarray(k_pool)),
                                          _p(np.ascontiguousarray(v_pool)), _code(k_pool, bf16),
                                          num_slots, _p(bt), bt.shape[1], _p(cu), _p(kl),
                                          cu.size - 1, H, G, D, block_size, float(scale))
    if rc != 0:
        raise ValueError("oracle_dense_attention_f64: bad arguments")
    return out


def set_mutation(code: int) -> None:
    lib().oracle_set_mutation(code)


def num_threads() -> int:
    return int(lib().oracle_num_threads())
