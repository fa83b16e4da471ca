"""Tensor-level entry points of the three kernels (device tensors in, device tensors out).

PyTorch only supplies device memory and the current HIP stream; every operation here is one
call into libflour_hip.so. Shapes follow the C-ABI (include/flour_hip.h):

* KV pool of one layer: ``k_pool``/``v_pool`` of shape (kv_heads, num_slots, head_dim),
  exactly PagedKvPool::new (src/models/common/paged.rs:124-167).
* ``kv_write``        <- PagedKvPool::write (paged.rs:186-204), scatter semantics.
* ``paged_decode``    <- paged_attention (src/backend/cpu.rs:57-112) for seq_q == 1, batched.
* ``varlen_prefill``  <- paged_attention for seq_q >= 1, batched over packed sequences.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import check, lib

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DT[dt]
    except KeyError:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, f"unsupported dtype {dt}") from None


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _need_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT,
                                  "flour_amd ops take device tensors (got a CPU tensor)")


def _need_i32(*ts: torch.Tensor) -> None:
    for t in ts:
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT,
                                  "index tensors must be contiguous int32")


def kv_write(k: torch.Tensor, v: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
             slot_mapping: torch.Tensor) -> None:
    """pool[h, slot_mapping[t], :] = k[t, h, :] for every token t with slot >= 0.

    ``k``/``v`` are (num_tokens, kv_heads, head_dim) views with a unit last stride (the
    reference's (kv_heads, seq, head_dim) is ``k.transpose(0, 1)`` of that). The pools are
    contiguous (kv_heads, num_slots, head_dim).
    """
    _need_cuda(k, v, k_pool, v_pool, slot_mapping)
    _need_i32(slot_mapping)
    T, G, D = k.shape
    if v.shape != k.shape or v.stride() != k.stride() or k.stride(2) != 1:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "k/v must share shape and strides, unit last stride")
    if k_pool.shape != v_pool.shape or k_pool.shape[0] != G or k_pool.shape[2] != D or \
            not k_pool.is_contiguous() or not v_pool.is_contiguous():
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "pools must be contiguous (kv_heads, num_slots, head_dim)")
    if k.dtype != k_pool.dtype or v.dtype != k_pool.dtype or v_pool.dtype != k_pool.dtype:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "k/v and pools must share a dtype")
    if slot_mapping.numel() != T:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "slot_mapping needs one slot per token")
    check(lib().flour_hip_kv_write(_ptr(k), _ptr(v), k.stride(0), k.stride(1), _ptr(k_pool),
                                   _ptr(v_pool), _ptr(slot_mapping), T, G, D, k_pool.shape[1],
                                   dtype_code(k.dtype), _stream()))


def rope_tables(max_pos: int, head_dim: int, rope_theta: float, dtype: torch.dtype,
                device: torch.device | str = "cpu") -> tuple[torch.Tensor, torch.Tensor]:
    """The cos / sin tables of Cache::new (src/models/common/cache.rs:377-393), each
    (max_pos, head_dim / 2): theta_i = 1 / rope_theta^(2i / head_dim) and angle = pos * theta_i
    in fp32, cos / sin in fp32, then cast to ``dtype``. Computed with torch's fp32 CPU math
    (the reference uses Rust's f32 powf / cos / sin, which may differ in the last fp32 bit)."""
    half = head_dim // 2
    i = torch.arange(half, dtype=torch.float32)
    theta = 1.0 / torch.pow(torch.tensor(rope_theta, dtype=torch.float32), (2 * i) / head_dim)
    pos = torch.arange(max_pos, dtype=torch.float32).reshape(max_pos, 1)
    ang = pos * theta.reshape(1, half)
    return (ang.cos().to(dtype).contiguous().to(device),
            ang.sin().to(dtype).contiguous().to(device))


def rope_kv_write(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_pool: torch.Tensor,
                  v_pool: torch.Tensor, slot_mapping: torch.Tensor, positions: torch.Tensor,
                  cos: torch.Tensor, sin: torch.Tensor, q_out: torch.Tensor | None = None
                  ) -> torch.Tensor:
    """RoPE on q and k (rotate-half form, each product and sum in the tensor dtype), then
    k_pool[h, slot_mapping[t], :] = rope(k[t, h, :]) and v_pool[h, slot_mapping[t], :] =
    v[t, h, :]; returns rope(q) in ``q_out`` (default: a new tensor; ``q_out=q`` rotates in
    place). ``q`` is (num_tokens, num_heads, head_dim), ``k``/``v`` (num_tokens, kv_heads,
    head_dim), all with a unit last stride; ``positions`` holds each token's table row."""
    _need_cuda(q, k, v, k_pool, v_pool, slot_mapping, positions, cos, sin)
    _need_i32(slot_mapping, positions)
    T, H, D = q.shape
    if k.dim() != 3 or k.shape[0] != T or k.shape[2] != D or v.shape != k.shape or \
            v.stride() != k.stride() or k.stride(2) != 1 or q.stride(2) != 1:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT,
                              "q (T, H, D), k/v (T, G, D) sharing strides, unit last strides")
    G = k.shape[1]
    if q_out is None:
        q_out = torch.empty_strided(q.shape, q.stride(), dtype=q.dtype, device=q.device)
    if q_out.shape != q.shape or q_out.stride() != q.stride() or q_out.dtype != q.dtype:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "q_out must match q's shape and strides")
    if k_pool.shape != v_pool.shape or k_pool.shape[0] != G or k_pool.shape[2] != D or \
            not k_pool.is_contiguous() or not v_pool.is_contiguous():
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "pools must be contiguous (kv_heads, num_slots, head_dim)")
    dts = {q.dtype, k.dtype, v.dtype, k_pool.dtype, v_pool.dtype, cos.dtype, sin.dtype}
    if len(dts) != 1:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "q, k, v, pools and tables must share a dtype")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != D // 2 or \
            not cos.is_contiguous() or not sin.is_contiguous():
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "tables must be contiguous (max_pos, head_dim / 2)")
    if slot_mapping.numel() != T or positions.numel() != T:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "one slot and one position per token")
    check(lib().flour_hip_rope_kv_write(_ptr(q_out), _ptr(q), q.stride(0), q.stride(1), H,
                                        _ptr(k), _ptr(v), k.stride(0), k.stride(1),
                                        _ptr(k_pool), _ptr(v_pool), _ptr(slot_mapping),
                                        _ptr(positions), _ptr(cos), _ptr(sin), cos.shape[0], T,
                                        G, D, k_pool.shape[1], dtype_code(q.dtype), _stream()))
    return q_out


def decode_workspace_bytes(batch: int, num_heads: int, kv_heads: int, head_dim: int,
                           max_context_len: int) -> int:
    n = ctypes.c_size_t(0)
    check(lib().flour_hip_paged_decode_workspace_size(batch, num_heads, kv_heads, head_dim,
                                                      max_context_len, ctypes.byref(n)))
    return n.value


class Workspace:
    """Device scratch for the kernels that take a workspace (split-context decode partials,
    the prefill V staging copy); grows on demand and is reused.

    Calls sharing one workspace must not overlap in time (one stream, or explicit ordering).
    """

    def __init__(self, device: torch.device | str = "cuda"):
        self.device = torch.device(device)
        self.buf: torch.Tensor | None = None

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=self.device)
        return self.buf


DecodeWorkspace = Workspace


_default_ws: dict[int, DecodeWorkspace] = {}


def paged_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                 block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
                 max_context_len: int, block_size: int = 16,
                 out_dtype: torch.dtype | None = None, out: torch.Tensor | None = None,
                 workspace: DecodeWorkspace | None = None) -> torch.Tensor:
    """One decode step for a batch: q (batch, num_heads, head_dim) -> (batch, num_heads, head_dim).

    ``block_tables`` is (batch, max_blocks_per_seq) int32, ``context_lens`` (batch,) int32;
    ``max_context_len`` bounds context_lens (it sizes the split-context grid); block_size is
    the cache's page size (BLOCK_SIZE = 16 in the reference, cache.rs:10).
    """
    _need_cuda(q, k_pool, v_pool, block_tables, context_lens)
    _need_i32(block_tables, context_lens)
    B, H, D = q.shape
    G, num_slots, Dk = k_pool.shape
    if Dk != D or not q.is_contiguous() or not k_pool.is_contiguous() or not v_pool.is_contiguous():
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "q and pools must be contiguous with matching head_dim")
    if q.dtype != k_pool.dtype:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "q and pools must share a dtype")
    _check_block_size(num_slots, block_size)
    out_dtype = out_dtype or q.dtype
    if out is None:
        out = torch.empty((B, H, D), dtype=out_dtype, device=q.device)
    if workspace is None:
        workspace = _default_ws.setdefault(q.device.index or 0, DecodeWorkspace(q.device))
    nbytes = decode_workspace_bytes(B, H, G, D, max_context_len)
    ws = workspace.get(nbytes)
    check(lib().flour_hip_paged_decode(_ptr(out), dtype_code(out.dtype), _ptr(q), _ptr(k_pool),
                                       _ptr(v_pool), _ptr(block_tables), block_tables.shape[1],
                                       _ptr(context_lens), B, H, G, D, block_size, num_slots,
                                       max_context_len, float(scale), dtype_code(q.dtype),
                                       _ptr(ws), ws.numel(), _stream()))
    return out


def prepare_paged_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                         block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
                         max_context_len: int, out: torch.Tensor, workspace: DecodeWorkspace,
                         block_size: int = 16):
    """Validates the arguments of paged_decode once and returns a callable that relaunches the
    same decode step (same tensors, current stream at preparation time) with no per-call
    Python work beyond the C call, as a serving loop that reuses its buffers would."""
    _need_cuda(q, k_pool, v_pool, block_tables, context_lens, out)
    _need_i32(block_tables, context_lens)
    B, H, D = q.shape
    G, num_slots, Dk = k_pool.shape
    if Dk != D or not q.is_contiguous() or not k_pool.is_contiguous() or not v_pool.is_contiguous():
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "q and pools must be contiguous with matching head_dim")
    if q.dtype != k_pool.dtype or out.shape != q.shape or not out.is_contiguous():
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "q, pools and out must agree")
    _check_block_size(num_slots, block_size)
    ws = workspace.get(decode_workspace_bytes(B, H, G, D, max_context_len))
    args = (_ptr(out), dtype_code(out.dtype), _ptr(q), _ptr(k_pool), _ptr(v_pool),
            _ptr(block_tables), block_tables.shape[1], _ptr(context_lens), B, H, G, D,
            block_size, num_slots, max_context_len, float(scale), dtype_code(q.dtype), _ptr(ws),
            ws.numel(), _stream())
    fn = lib().flour_hip_paged_decode

    def run() -> None:
        rc = fn(*args)
        if rc:
            check(rc)

    return run


def prefill_workspace_bytes(num_seqs: int, max_blocks_per_seq: int, block_size: int,
                            kv_heads: int, head_dim: int, dtype: torch.dtype) -> int:
    """Bytes of the V staging copy that varlen_prefill's long-prompt path reads (0 when no
    call of this shape can take that path)."""
    n = ctypes.c_size_t(0)
    check(lib().flour_hip_varlen_prefill_workspace_size(num_seqs, max_blocks_per_seq, block_size,
                                                        kv_heads, head_dim, dtype_code(dtype),
                                                        ctypes.byref(n)))
    return n.value


def varlen_prefill(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                   cu_seqlens_q: torch.Tensor, kv_lens: torch.Tensor, block_tables: torch.Tensor,
                   max_seqlen_q: int, scale: float, block_size: int = 16,
                   out_dtype: torch.dtype | None = None,
                   out: torch.Tensor | None = None,
                   workspace: Workspace | None = None) -> torch.Tensor:
    """Causal attention of packed query rows q (total_q, num_heads, head_dim) over the cache.

    Sequence s owns rows cu_seqlens_q[s]:cu_seqlens_q[s+1] and kv_lens[s] cached positions
    (its own new rows last). q may be any view with a unit last stride, e.g. the reference's
    head-major (num_heads, seq, head_dim) transposed to (seq, num_heads, head_dim).

    Without ``workspace`` the call goes to flour_hip_varlen_prefill, which needs no device
    memory beyond its arguments. With one, flour_hip_varlen_prefill_ws may stage V in it for
    long prompts (the workspace grows to the size the call needs).
    """
    _need_cuda(q, k_pool, v_pool, cu_seqlens_q, kv_lens, block_tables)
    _need_i32(cu_seqlens_q, kv_lens, block_tables)
    T, H, D = q.shape
    G, num_slots, Dk = k_pool.shape
    if Dk != D or q.stride(2) != 1 or not k_pool.is_contiguous() or not v_pool.is_contiguous():
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "bad q / pool layout")
    if q.dtype != k_pool.dtype:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT, "q and pools must share a dtype")
    _check_block_size(num_slots, block_size)
    out_dtype = out_dtype or q.dtype
    if out is None:
        out = torch.empty((T, H, D), dtype=out_dtype, device=q.device)
    num_seqs = cu_seqlens_q.numel() - 1
    args = (_ptr(out), dtype_code(out.dtype), out.stride(0), out.stride(1), _ptr(q), q.stride(0),
            q.stride(1), _ptr(k_pool), _ptr(v_pool), _ptr(cu_seqlens_q), _ptr(kv_lens),
            _ptr(block_tables), block_tables.shape[1], num_seqs, max_seqlen_q, T, H, G, D,
            block_size, num_slots, float(scale), dtype_code(q.dtype))
    if workspace is None:
        check(lib().flour_hip_varlen_prefill(*args, _stream()))
    else:
        nbytes = prefill_workspace_bytes(num_seqs, block_tables.shape[1], block_size, G, D,
                                         q.dtype)
        ws = workspace.get(nbytes)
        check(lib().flour_hip_varlen_prefill_ws(*args, _ptr(ws), ws.numel(), _stream()))
    return out


def _check_block_size(num_slots: int, block_size: int) -> None:
    """Pools hold whole blocks: num_slots is a multiple of block_size (cache.rs:21-23)."""
    if block_size <= 0 or num_slots % block_size != 0:
        raise _lib.FlourError(_lib.ERR_INVALID_ARGUMENT,
                              f"num_slots {num_slots} is not a multiple of block_size {block_size}")
