"""Host-side KV cache over a device pool: the Python face of include/flour_cache.h.

Mirrors the reference's per-sequence cache (src/models/common/cache.rs, paged.rs, prefix.rs)
with the same method names and meaning:

* ``BlockAllocator``  <- paged.rs:7-54   (LIFO free list, refcounts; allocate() -> id or None)
* ``BlockTable``      <- paged.rs:57-121 (slot(pos) = blocks[pos // bs] * bs + pos % bs)
* ``KvBatch``         <- many sequences over one pool (continuous batching; the reference's
  engine is batch-1, engine.rs:88, :219-263), one plan per forward step
* ``KvCache``         <- cache.rs KvCache + Cache: allocate_kv, write_kv, attention
  (= kv_blocks + paged_attention), reset_sequence, match_prefix, register_prefix,
  clear_prefix_cache, free_blocks, export_prefix_bundle / import_prefix_bundle (the FLKV
  frame of src/kv_cache/bundle.rs), with the per-layer pools of PagedKvPool::new on the device.

Every operation is one call into libflour_hip.so; errors raise ``FlourError`` with the
library's message (the reference's ``candle_core::Error::Msg``).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib


def _i32(n: int):
    return (ctypes.c_int32 * max(n, 1))()


def _tokens(tokens) -> tuple:
    arr = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
    return arr, arr.ctypes.data_as(ctypes.c_void_p), int(arr.size)


class BlockAllocator:
    def __init__(self, num_blocks: int):
        self._h = ctypes.c_void_p()
        check(lib().flour_block_allocator_create(num_blocks, ctypes.byref(self._h)))

    def __del__(self):
        if getattr(self, "_h", None):
            lib().flour_block_allocator_destroy(self._h)
            self._h = None

    def allocate(self):
        i = lib().flour_block_allocator_allocate(self._h)
        return None if i < 0 else i

    def incref(self, block_id: int) -> None:
        check(lib().flour_block_allocator_incref(self._h, block_id))

    def decref(self, block_id: int) -> bool:
        r = lib().flour_block_allocator_decref(self._h, block_id)
        if r < 0:
            check(r)
        return bool(r)

    def ref_count(self, block_id: int) -> int:
        r = lib().flour_block_allocator_ref_count(self._h, block_id)
        if r < 0:
            check(r)
        return r

    def num_free(self) -> int:
        return lib().flour_block_allocator_num_free(self._h)


class BlockTable:
    def __init__(self, block_size: int):
        self._h = ctypes.c_void_p()
        check(lib().flour_block_table_create(block_size, ctypes.byref(self._h)))

    def __del__(self):
        if getattr(self, "_h", None):
            lib().flour_block_table_destroy(self._h)
            self._h = None

    def push_block(self, block_id: int) -> None:
        check(lib().flour_block_table_push_block(self._h, block_id))

    def advance(self, n: int) -> None:
        check(lib().flour_block_table_advance(self._h, n))

    def clear(self) -> None:
        check(lib().flour_block_table_clear(self._h))

    def len(self) -> int:
        return lib().flour_block_table_len(self._h)

    def is_empty(self) -> bool:
        return self.len() == 0

    def capacity(self) -> int:
        return lib().flour_block_table_capacity(self._h)

    def block_size(self) -> int:
        return lib().flour_block_table_block_size(self._h)

    def blocks(self) -> list[int]:
        n = ctypes.c_int(0)
        check(lib().flour_block_table_blocks(self._h, None, 0, ctypes.byref(n)))
        out = _i32(n.value)
        check(lib().flour_block_table_blocks(self._h, out, n.value, ctypes.byref(n)))
        return list(out[: n.value])

    def block_at(self, i: int) -> int:
        return self.blocks()[i]

    def slot(self, pos: int) -> int:
        r = lib().flour_block_table_slot(self._h, pos)
        if r < 0:
            check(int(r))
        return int(r)

    def slots(self, start: int, end: int) -> list[int]:
        out = _i32(end - start)
        check(lib().flour_block_table_slots(self._h, start, end, out))
        return list(out[: end - start])


class KvCache:
    """One sequence's paged KV cache (the reference's Cache / KvCache pair).

    ``device_pool=False`` keeps only the bookkeeping (tests without a GPU)."""

    def __init__(self, num_layers: int, max_seq_len: int, num_heads: int, kv_heads: int,
                 head_dim: int, dtype=None, block_size: int = 16, device_pool: bool = True):
        import torch

        dtype = dtype or torch.bfloat16
        self.num_layers, self.max_seq_len = num_layers, max_seq_len
        self.num_heads, self.kv_heads, self.head_dim = num_heads, kv_heads, head_dim
        self.block_size, self.dtype = block_size, dtype
        self.device_pool = bool(device_pool)
        self._h = ctypes.c_void_p()
        from .ops import dtype_code

        check(lib().flour_kv_cache_create(num_layers, max_seq_len, num_heads, kv_heads, head_dim,
                                          block_size, dtype_code(dtype), int(device_pool),
                                          ctypes.byref(self._h)))

    def __del__(self):
        if getattr(self, "_h", None):
            lib().flour_kv_cache_destroy(self._h)
            self._h = None

    # ---- bookkeeping (cache.rs)
    def allocate_kv(self, seq_len: int) -> None:
        check(lib().flour_kv_cache_allocate_kv(self._h, seq_len))

    def len(self) -> int:
        return lib().flour_kv_cache_len(self._h)

    def capacity(self) -> int:
        return lib().flour_kv_cache_capacity(self._h)

    def free_blocks(self) -> int:
        return lib().flour_kv_cache_free_blocks(self._h)

    def ref_count(self, block_id: int) -> int:
        r = lib().flour_kv_cache_ref_count(self._h, block_id)
        if r < 0:
            check(r)
        return r

    def blocks(self) -> list[int]:
        n = ctypes.c_int(0)
        check(lib().flour_kv_cache_blocks(self._h, None, 0, ctypes.byref(n)))
        out = _i32(n.value)
        check(lib().flour_kv_cache_blocks(self._h, out, n.value, ctypes.byref(n)))
        return list(out[: n.value])

    def slots(self, start: int, end: int) -> list[int]:
        out = _i32(end - start)
        check(lib().flour_kv_cache_slots(self._h, start, end, out))
        return list(out[: end - start])

    def reset_sequence(self) -> None:
        check(lib().flour_kv_cache_reset_sequence(self._h))

    def match_prefix(self, token_ids) -> int:
        arr, ptr, n = _tokens(token_ids)
        r = lib().flour_kv_cache_match_prefix(self._h, ptr, n)
        if r < 0:
            check(r)
        return r

    def register_prefix(self, token_ids) -> None:
        arr, ptr, n = _tokens(token_ids)
        check(lib().flour_kv_cache_register_prefix(self._h, ptr, n))

    def clear_prefix_cache(self) -> None:
        check(lib().flour_kv_cache_clear_prefix_cache(self._h))

    # ---- FLKV bundles (cache.rs:166-340, src/kv_cache/bundle.rs)
    def export_prefix_bundle(self, model_id: str, token_ids, token_count: int, out=None):
        """Cache::export_prefix_bundle + KvBundleCodec::encode: the FLKV frame of the first
        token_count live tokens, read from the device pools. Returns ``bytes``; with ``out`` (a
        CPU uint8 tensor, pinned for full copy speed, at least bundle_size() bytes) the frame
        is written there and its length returned."""
        arr, ptr, n = _tokens(token_ids)
        mid = model_id.encode("utf-8")
        stream = self._bundle_stream()
        size = ctypes.c_size_t(0)
        check(lib().flour_kv_cache_export_bundle(self._h, mid, ptr, n, token_count, None, 0,
                                                 ctypes.byref(size), stream))
        if out is None:
            buf = ctypes.create_string_buffer(size.value)
            check(lib().flour_kv_cache_export_bundle(self._h, mid, ptr, n, token_count, buf,
                                                     size.value, ctypes.byref(size), stream))
            return buf.raw[:size.value]
        check(lib().flour_kv_cache_export_bundle(self._h, mid, ptr, n, token_count,
                                                 ctypes.c_void_p(out.data_ptr()), out.numel(),
                                                 ctypes.byref(size), stream))
        return size.value

    def bundle_size(self, model_id: str, token_ids, token_count: int) -> int:
        """Length of the frame export_prefix_bundle would produce."""
        arr, ptr, n = _tokens(token_ids)
        size = ctypes.c_size_t(0)
        check(lib().flour_kv_cache_export_bundle(self._h, model_id.encode("utf-8"), ptr, n,
                                                 token_count, None, 0, ctypes.byref(size), None))
        return size.value

    def import_prefix_bundle(self, bundle, prompt_tokens) -> int:
        """KvBundleCodec::decode + Cache::import_prefix_bundle; ``bundle`` is ``bytes`` or a CPU
        uint8 tensor (the first ``numel`` bytes). Returns the imported token count."""
        arr, ptr, n = _tokens(prompt_tokens)
        got = ctypes.c_int(0)
        if isinstance(bundle, (bytes, bytearray)):
            data, size = bundle, len(bundle)
        else:
            data, size = ctypes.c_void_p(bundle.data_ptr()), bundle.numel()
        check(lib().flour_kv_cache_import_bundle(self._h, data, size, ptr, n,
                                                 ctypes.byref(got), self._bundle_stream()))
        return got.value

    def _bundle_stream(self):
        """torch's current stream for a device pool; none for bookkeeping-only caches."""
        if not self.device_pool:
            return None
        from .ops import _stream

        return _stream()

    # ---- device side
    def pool(self, layer: int):
        """(k_pool, v_pool) of a layer as torch views of shape (kv_heads, num_slots, head_dim)."""
        import torch

        k, v, ns = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int64()
        check(lib().flour_kv_cache_pool(self._h, layer, ctypes.byref(k), ctypes.byref(v),
                                        ctypes.byref(ns)))
        n = self.kv_heads * ns.value * self.head_dim
        return tuple(_device_view(p.value, n, self.dtype).view(self.kv_heads, ns.value,
                                                                self.head_dim) for p in (k, v))

    def write_kv(self, layer: int, k, v) -> None:
        """Cache::write_kv: k, v of shape (1, kv_heads, seq, head_dim) (the reference layout)
        or (seq, kv_heads, head_dim); the trailing seq live positions take them."""
        from .ops import _ptr, _stream

        if k.dim() == 4:
            seq = k.shape[2]
            st, sh = k.stride(2), k.stride(1)
        else:
            seq = k.shape[0]
            st, sh = k.stride(0), k.stride(1)
        assert k.stride() == v.stride() and k.dtype == v.dtype == self.dtype
        check(lib().flour_kv_cache_write_kv(self._h, layer, _ptr(k), _ptr(v), seq, st, sh,
                                            _stream()))

    def attention(self, layer: int, q, scale: float, out=None, out_dtype=None):
        """Cache::kv_blocks + paged_attention: q of shape (1, num_heads, seq_q, head_dim)
        (post-RoPE) attends causally to every live position; returns the same shape."""
        import torch
        from .ops import _ptr, _stream, dtype_code

        assert q.dim() == 4 and q.shape[0] == 1
        H, S, D = q.shape[1], q.shape[2], q.shape[3]
        out_dtype = out_dtype or q.dtype
        if out is None:
            out = torch.empty((1, H, S, D), dtype=out_dtype, device=q.device)
        check(lib().flour_kv_cache_attention(self._h, layer, _ptr(q), H, S, q.stride(2),
                                             q.stride(1), _ptr(out), dtype_code(out.dtype),
                                             out.stride(2), out.stride(1), float(scale),
                                             _stream()))
        return out


class KvBatch:
    """Many sequences over one device pool (the flour_kv_batch_* calls): a shared
    BlockAllocator and prefix registry, one BlockTable per sequence, and one plan per forward
    step that every layer's write_kv / attention uses."""

    def __init__(self, num_layers: int, num_blocks: int, max_seqs: int, max_seq_len: int,
                 max_batch_tokens: int, num_heads: int, kv_heads: int, head_dim: int, dtype=None,
                 block_size: int = 16, device_pool: bool = True):
        import torch

        from .ops import dtype_code

        self.dtype = dtype or torch.bfloat16
        self.num_layers, self.num_heads, self.kv_heads = num_layers, num_heads, kv_heads
        self.head_dim, self.block_size = head_dim, block_size
        self.device_pool = bool(device_pool)
        self._h = ctypes.c_void_p()
        check(lib().flour_kv_batch_create(num_layers, num_blocks, max_seqs, max_seq_len,
                                          max_batch_tokens, num_heads, kv_heads, head_dim,
                                          block_size, dtype_code(self.dtype), int(device_pool),
                                          ctypes.byref(self._h)))

    def __del__(self):
        if getattr(self, "_h", None):
            lib().flour_kv_batch_destroy(self._h)
            self._h = None

    def _r(self, rc: int) -> int:
        if rc < 0:
            check(rc)
        return rc

    def add_sequence(self) -> int:
        sid = ctypes.c_int(-1)
        check(lib().flour_kv_batch_add_sequence(self._h, ctypes.byref(sid)))
        return sid.value

    def remove_sequence(self, sid: int) -> None:
        check(lib().flour_kv_batch_remove_sequence(self._h, sid))

    def reset_sequence(self, sid: int) -> None:
        check(lib().flour_kv_batch_reset_sequence(self._h, sid))

    def allocate_kv(self, sid: int, seq_len: int) -> None:
        check(lib().flour_kv_batch_allocate_kv(self._h, sid, seq_len))

    def len(self, sid: int) -> int:
        return self._r(lib().flour_kv_batch_len(self._h, sid))

    def free_blocks(self) -> int:
        return self._r(lib().flour_kv_batch_free_blocks(self._h))

    def ref_count(self, block_id: int) -> int:
        return self._r(lib().flour_kv_batch_ref_count(self._h, block_id))

    def blocks(self, sid: int) -> list[int]:
        n = ctypes.c_int(0)
        check(lib().flour_kv_batch_blocks(self._h, sid, None, 0, ctypes.byref(n)))
        buf = _i32(n.value)
        check(lib().flour_kv_batch_blocks(self._h, sid, buf, n.value, ctypes.byref(n)))
        return list(buf[:n.value])

    def match_prefix(self, sid: int, token_ids) -> int:
        arr, ptr, n = _tokens(token_ids)
        return self._r(lib().flour_kv_batch_match_prefix(self._h, sid, ptr, n))

    def register_prefix(self, sid: int, token_ids) -> None:
        arr, ptr, n = _tokens(token_ids)
        check(lib().flour_kv_batch_register_prefix(self._h, sid, ptr, n))

    def clear_prefix_cache(self) -> None:
        check(lib().flour_kv_batch_clear_prefix_cache(self._h))

    def plan(self, seq_ids, seq_q) -> None:
        """The step: sequence seq_ids[i] brings its last seq_q[i] live positions as new rows,
        packed in this order."""
        from .ops import _stream

        ids = np.ascontiguousarray(np.asarray(seq_ids, dtype=np.int32))
        q = np.ascontiguousarray(np.asarray(seq_q, dtype=np.int32))
        assert ids.size == q.size
        check(lib().flour_kv_batch_plan(self._h, ids.ctypes.data_as(ctypes.c_void_p),
                                        q.ctypes.data_as(ctypes.c_void_p), int(ids.size),
                                        _stream() if self.device_pool else None))

    def step(self, seq_ids, seq_q) -> None:
        """allocate_kv(seq_ids[i], seq_q[i]) for every sequence, then plan(), in one call; a
        refused step changes no sequence."""
        from .ops import _stream

        ids = np.ascontiguousarray(np.asarray(seq_ids, dtype=np.int32))
        q = np.ascontiguousarray(np.asarray(seq_q, dtype=np.int32))
        assert ids.size == q.size
        check(lib().flour_kv_batch_step(self._h, ids.ctypes.data_as(ctypes.c_void_p),
                                        q.ctypes.data_as(ctypes.c_void_p), int(ids.size),
                                        _stream() if self.device_pool else None))

    def write_kv(self, layer: int, k, v) -> None:
        """The planned new rows, packed (rows, kv_heads, head_dim) with a unit last stride."""
        from .ops import _ptr, _stream

        assert k.stride() == v.stride() and k.dtype == v.dtype == self.dtype and k.stride(2) == 1
        check(lib().flour_kv_batch_write_kv(self._h, layer, _ptr(k), _ptr(v), k.stride(0),
                                            k.stride(1), _stream()))

    def rope_write_kv(self, layer: int, q, k, v, cos, sin, q_out=None):
        """RoPE on the planned rows' q and k at their positions in their sequences, rotated k
        and v into the layer's pools, in one kernel; returns rope(q) (``q_out=q`` rotates in
        place). q (rows, num_heads, head_dim), k / v (rows, kv_heads, head_dim), tables from
        ``ops.rope_tables`` covering max_seq_len positions."""
        import torch
        from .ops import _ptr, _stream

        assert k.stride() == v.stride() and k.stride(2) == 1 and q.stride(2) == 1
        assert q.dtype == k.dtype == v.dtype == cos.dtype == sin.dtype == self.dtype
        if q_out is None:
            q_out = torch.empty_strided(q.shape, q.stride(), dtype=q.dtype, device=q.device)
        assert q_out.shape == q.shape and q_out.stride() == q.stride()
        check(lib().flour_kv_batch_rope_write_kv(self._h, layer, _ptr(q_out), _ptr(q), q.stride(0),
                                                 q.stride(1), q.shape[1], _ptr(k), _ptr(v),
                                                 k.stride(0), k.stride(1), _ptr(cos), _ptr(sin),
                                                 cos.shape[0], _stream()))
        return q_out

    def attention(self, layer: int, q, scale: float, out=None, out_dtype=None):
        """Attention of the planned rows: q packed (rows, num_heads, head_dim); returns the
        same shape (decode when every sequence brings one row, varlen prefill otherwise)."""
        import torch
        from .ops import _ptr, _stream, dtype_code

        T, H, D = q.shape
        if out is None:
            out = torch.empty((T, H, D), dtype=out_dtype or q.dtype, device=q.device)
        check(lib().flour_kv_batch_attention(self._h, layer, _ptr(q), H, q.stride(0), q.stride(1),
                                             _ptr(out), dtype_code(out.dtype), out.stride(0),
                                             out.stride(1), float(scale), _stream()))
        return out

    def write_kv_attention(self, layer: int, k, v, q, scale: float, out=None, out_dtype=None):
        """``write_kv(layer, k, v)`` then ``attention(layer, q, scale)`` in one call; a decode
        step over private tail blocks runs as one launch (the decode kernel writes the new rows
        before it reads them). k / v packed (rows, kv_heads, head_dim) with a unit last stride,
        q (rows, num_heads, head_dim); returns the attention output."""
        import torch
        from .ops import _ptr, _stream, dtype_code

        assert k.stride() == v.stride() and k.dtype == v.dtype == self.dtype and k.stride(2) == 1
        T, H, D = q.shape
        if out is None:
            out = torch.empty((T, H, D), dtype=out_dtype or q.dtype, device=q.device)
        check(lib().flour_kv_batch_write_kv_attention(
            self._h, layer, _ptr(k), _ptr(v), k.stride(0), k.stride(1), _ptr(q), H, q.stride(0),
            q.stride(1), _ptr(out), dtype_code(out.dtype), out.stride(0), out.stride(1),
            float(scale), _stream()))
        return out

    def pool(self, layer: int):
        """(k_pool, v_pool) of a layer as torch views (kv_heads, num_slots, head_dim)."""
        k, v, ns = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int64()
        check(lib().flour_kv_batch_pool(self._h, layer, ctypes.byref(k), ctypes.byref(v),
                                        ctypes.byref(ns)))
        n = self.kv_heads * ns.value * self.head_dim
        return tuple(_device_view(p.value, n, self.dtype).view(self.kv_heads, ns.value,
                                                                self.head_dim) for p in (k, v))


def _device_view(addr: int, numel: int, dtype):
    """A torch tensor over device memory owned by the library (no copy, no ownership)."""
    import torch

    class _Holder:
        pass

    h = _Holder()
    h.__cuda_array_interface__ = {
        "shape": (numel,), "typestr": "<u2" if dtype in (torch.bfloat16, torch.float16) else "<f4",
        "data": (addr, False), "version": 3, "strides": None,
    }
    t = torch.as_tensor(h, device="cuda")
    return t.view(dtype)
