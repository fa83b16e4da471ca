//! Raw FFI bindings of `libflour_hip.so`: the C-ABI declared in `include/flour_hip.h` (the
//! attention hot path: KV-cache write, fused RoPE + KV write, paged decode, causal varlen
//! prefill) and `include/flour_cache.h` (block allocator, block table, per-sequence cache and
//! many sequences over one device pool).
//!
//! These replace, in the flour crate, `paged_attention` (`src/backend/cpu.rs:57-112`),
//! `PagedKvPool::write` (`src/models/common/paged.rs:186-204`) and the `Cache` calls of
//! `CausalSelfAttention::forward` (`src/models/common/attention.rs:104-109`). Every function
//! returns 0 on success or a negative `FLOUR_ERR_*` code; [`check`] turns a code into the
//! message the library recorded on the calling thread. Device pointers are the caller's;
//! launches are asynchronous on the `stream` argument (a `hipStream_t`, null for the default
//! stream).
#![allow(non_camel_case_types)]

use std::ffi::CStr;
use std::os::raw::{c_char, c_int, c_void};

pub const FLOUR_DTYPE_F32: c_int = 0;
pub const FLOUR_DTYPE_BF16: c_int = 1;
pub const FLOUR_DTYPE_F16: c_int = 2;

pub const FLOUR_OK: c_int = 0;
pub const FLOUR_ERR_INVALID_ARGUMENT: c_int = -1;
pub const FLOUR_ERR_UNSUPPORTED: c_int = -2;
pub const FLOUR_ERR_WORKSPACE: c_int = -3;
pub const FLOUR_ERR_HIP: c_int = -4;
pub const FLOUR_ERR_OUT_OF_BLOCKS: c_int = -5;
pub const FLOUR_ERR_CAPACITY: c_int = -6;

/// Opaque handles of `include/flour_cache.h`.
#[repr(C)]
pub struct FlourBlockAllocator {
    _private: [u8; 0],
}
#[repr(C)]
pub struct FlourBlockTable {
    _private: [u8; 0],
}
#[repr(C)]
pub struct FlourKvCache {
    _private: [u8; 0],
}
#[repr(C)]
pub struct FlourKvBatch {
    _private: [u8; 0],
}

// include/flour_hip.h
#[link(name = "flour_hip")]
extern "C" {
    pub fn flour_hip_last_error() -> *const c_char;
    pub fn flour_hip_version() -> *const c_char;
    pub fn flour_hip_kv_write(k: *const c_void, v: *const c_void, stride_tok: i64,
        stride_head: i64, k_pool: *mut c_void, v_pool: *mut c_void, slot_mapping: *const i32,
        num_tokens: c_int, kv_heads: c_int, head_dim: c_int, num_slots: i64, dtype: c_int,
        stream: *mut c_void) -> c_int;
    pub fn flour_hip_rope_kv_write(q_out: *mut c_void, q: *const c_void, q_stride_tok: i64,
        q_stride_head: i64, num_heads: c_int, k: *const c_void, v: *const c_void,
        kv_stride_tok: i64, kv_stride_head: i64, k_pool: *mut c_void, v_pool: *mut c_void,
        slot_mapping: *const i32, positions: *const i32, cos_table: *const c_void,
        sin_table: *const c_void, max_pos: c_int, num_tokens: c_int, kv_heads: c_int,
        head_dim: c_int, num_slots: i64, dtype: c_int, stream: *mut c_void) -> c_int;
    pub fn flour_hip_paged_decode_workspace_size(batch: c_int, num_heads: c_int, kv_heads: c_int,
        head_dim: c_int, max_context_len: c_int, bytes: *mut usize) -> c_int;
    pub fn flour_hip_paged_decode(out: *mut c_void, out_dtype: c_int, q: *const c_void,
        k_pool: *const c_void, v_pool: *const c_void, block_tables: *const i32,
        max_blocks_per_seq: c_int, context_lens: *const i32, batch: c_int, num_heads: c_int,
        kv_heads: c_int, head_dim: c_int, block_size: c_int, num_slots: i64,
        max_context_len: c_int, scale: f32, dtype: c_int, workspace: *mut c_void,
        workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn flour_hip_paged_decode_noalloc_max_workspace() -> usize;
    pub fn flour_hip_paged_decode_noalloc(out: *mut c_void, out_dtype: c_int, q: *const c_void,
        k_pool: *const c_void, v_pool: *const c_void, block_tables: *const i32,
        max_blocks_per_seq: c_int, context_lens: *const i32, batch: c_int, num_heads: c_int,
        kv_heads: c_int, head_dim: c_int, block_size: c_int, num_slots: i64,
        max_context_len: c_int, scale: f32, dtype: c_int, stream: *mut c_void) -> c_int;
    pub fn flour_hip_varlen_prefill(out: *mut c_void, out_dtype: c_int, o_stride_tok: i64,
        o_stride_head: i64, q: *const c_void, q_stride_tok: i64, q_stride_head: i64,
        k_pool: *const c_void, v_pool: *const c_void, cu_seqlens_q: *const i32,
        kv_lens: *const i32, block_tables: *const i32, max_blocks_per_seq: c_int, num_seqs: c_int,
        max_seqlen_q: c_int, total_q: c_int, num_heads: c_int, kv_heads: c_int, head_dim: c_int,
        block_size: c_int, num_slots: i64, scale: f32, dtype: c_int,
        stream: *mut c_void) -> c_int;
    pub fn flour_hip_varlen_prefill_workspace_size(num_seqs: c_int, max_blocks_per_seq: c_int,
        block_size: c_int, kv_heads: c_int, head_dim: c_int, dtype: c_int,
        bytes: *mut usize) -> c_int;
    pub fn flour_hip_varlen_prefill_ws(out: *mut c_void, out_dtype: c_int, o_stride_tok: i64,
        o_stride_head: i64, q: *const c_void, q_stride_tok: i64, q_stride_head: i64,
        k_pool: *const c_void, v_pool: *const c_void, cu_seqlens_q: *const i32,
        kv_lens: *const i32, block_tables: *const i32, max_blocks_per_seq: c_int, num_seqs: c_int,
        max_seqlen_q: c_int, total_q: c_int, num_heads: c_int, kv_heads: c_int, head_dim: c_int,
        block_size: c_int, num_slots: i64, scale: f32, dtype: c_int, workspace: *mut c_void,
        workspace_bytes: usize, stream: *mut c_void) -> c_int;
}

// include/flour_cache.h
#[link(name = "flour_hip")]
extern "C" {
    pub fn flour_block_allocator_create(num_blocks: c_int,
        out: *mut *mut FlourBlockAllocator) -> c_int;
    pub fn flour_block_allocator_destroy(a: *mut FlourBlockAllocator);
    pub fn flour_block_allocator_allocate(a: *mut FlourBlockAllocator) -> c_int;
    pub fn flour_block_allocator_incref(a: *mut FlourBlockAllocator, block_id: c_int) -> c_int;
    pub fn flour_block_allocator_decref(a: *mut FlourBlockAllocator, block_id: c_int) -> c_int;
    pub fn flour_block_allocator_ref_count(a: *const FlourBlockAllocator,
        block_id: c_int) -> c_int;
    pub fn flour_block_allocator_num_free(a: *const FlourBlockAllocator) -> c_int;
    pub fn flour_block_table_create(block_size: c_int, out: *mut *mut FlourBlockTable) -> c_int;
    pub fn flour_block_table_destroy(t: *mut FlourBlockTable);
    pub fn flour_block_table_push_block(t: *mut FlourBlockTable, block_id: c_int) -> c_int;
    pub fn flour_block_table_advance(t: *mut FlourBlockTable, n: c_int) -> c_int;
    pub fn flour_block_table_clear(t: *mut FlourBlockTable) -> c_int;
    pub fn flour_block_table_len(t: *const FlourBlockTable) -> c_int;
    pub fn flour_block_table_capacity(t: *const FlourBlockTable) -> c_int;
    pub fn flour_block_table_block_size(t: *const FlourBlockTable) -> c_int;
    pub fn flour_block_table_blocks(t: *const FlourBlockTable, out: *mut i32, cap: c_int,
        n: *mut c_int) -> c_int;
    pub fn flour_block_table_slot(t: *const FlourBlockTable, pos: c_int) -> i64;
    pub fn flour_block_table_slots(t: *const FlourBlockTable, start: c_int, end: c_int,
        out: *mut i32) -> c_int;
    pub fn flour_kv_cache_create(num_layers: c_int, max_seq_len: c_int, num_heads: c_int,
        kv_heads: c_int, head_dim: c_int, block_size: c_int, dtype: c_int, device_pool: c_int,
        out: *mut *mut FlourKvCache) -> c_int;
    pub fn flour_kv_cache_destroy(c: *mut FlourKvCache);
    pub fn flour_kv_cache_allocate_kv(c: *mut FlourKvCache, seq_len: c_int) -> c_int;
    pub fn flour_kv_cache_len(c: *const FlourKvCache) -> c_int;
    pub fn flour_kv_cache_capacity(c: *const FlourKvCache) -> c_int;
    pub fn flour_kv_cache_free_blocks(c: *const FlourKvCache) -> c_int;
    pub fn flour_kv_cache_ref_count(c: *const FlourKvCache, block_id: c_int) -> c_int;
    pub fn flour_kv_cache_blocks(c: *const FlourKvCache, out: *mut i32, cap: c_int,
        n: *mut c_int) -> c_int;
    pub fn flour_kv_cache_slots(c: *const FlourKvCache, start: c_int, end: c_int,
        out: *mut i32) -> c_int;
    pub fn flour_kv_cache_write_kv(c: *mut FlourKvCache, layer: c_int, k: *const c_void,
        v: *const c_void, seq_len: c_int, stride_tok: i64, stride_head: i64,
        stream: *mut c_void) -> c_int;
    pub fn flour_kv_cache_attention(c: *mut FlourKvCache, layer: c_int, q: *const c_void,
        num_heads: c_int, seq_q: c_int, q_stride_tok: i64, q_stride_head: i64, out: *mut c_void,
        out_dtype: c_int, o_stride_tok: i64, o_stride_head: i64, scale: f32,
        stream: *mut c_void) -> c_int;
    pub fn flour_kv_cache_reset_sequence(c: *mut FlourKvCache) -> c_int;
    pub fn flour_kv_cache_match_prefix(c: *mut FlourKvCache, tokens: *const u32,
        n: c_int) -> c_int;
    pub fn flour_kv_cache_register_prefix(c: *mut FlourKvCache, tokens: *const u32,
        n: c_int) -> c_int;
    pub fn flour_kv_cache_clear_prefix_cache(c: *mut FlourKvCache) -> c_int;
    pub fn flour_kv_cache_export_bundle(c: *mut FlourKvCache, model_id: *const c_char,
        token_ids: *const u32, n_ids: c_int, token_count: c_int, out: *mut c_void, cap: usize,
        len: *mut usize, stream: *mut c_void) -> c_int;
    pub fn flour_kv_cache_import_bundle(c: *mut FlourKvCache, bytes: *const c_void, len: usize,
        prompt_tokens: *const u32, n_prompt: c_int, imported: *mut c_int,
        stream: *mut c_void) -> c_int;
    pub fn flour_kv_cache_pool(c: *const FlourKvCache, layer: c_int, k_pool: *mut *mut c_void,
        v_pool: *mut *mut c_void, num_slots: *mut i64) -> c_int;
    pub fn flour_kv_batch_create(num_layers: c_int, num_blocks: c_int, max_seqs: c_int,
        max_seq_len: c_int, max_batch_tokens: c_int, num_heads: c_int, kv_heads: c_int,
        head_dim: c_int, block_size: c_int, dtype: c_int, device_pool: c_int,
        out: *mut *mut FlourKvBatch) -> c_int;
    pub fn flour_kv_batch_destroy(b: *mut FlourKvBatch);
    pub fn flour_kv_batch_add_sequence(b: *mut FlourKvBatch, seq_id: *mut c_int) -> c_int;
    pub fn flour_kv_batch_remove_sequence(b: *mut FlourKvBatch, seq_id: c_int) -> c_int;
    pub fn flour_kv_batch_reset_sequence(b: *mut FlourKvBatch, seq_id: c_int) -> c_int;
    pub fn flour_kv_batch_allocate_kv(b: *mut FlourKvBatch, seq_id: c_int,
        seq_len: c_int) -> c_int;
    pub fn flour_kv_batch_len(b: *const FlourKvBatch, seq_id: c_int) -> c_int;
    pub fn flour_kv_batch_free_blocks(b: *const FlourKvBatch) -> c_int;
    pub fn flour_kv_batch_ref_count(b: *const FlourKvBatch, block_id: c_int) -> c_int;
    pub fn flour_kv_batch_blocks(b: *const FlourKvBatch, seq_id: c_int, out: *mut i32, cap: c_int,
        n: *mut c_int) -> c_int;
    pub fn flour_kv_batch_match_prefix(b: *mut FlourKvBatch, seq_id: c_int, tokens: *const u32,
        n: c_int) -> c_int;
    pub fn flour_kv_batch_register_prefix(b: *mut FlourKvBatch, seq_id: c_int, tokens: *const u32,
        n: c_int) -> c_int;
    pub fn flour_kv_batch_clear_prefix_cache(b: *mut FlourKvBatch) -> c_int;
    pub fn flour_kv_batch_plan(b: *mut FlourKvBatch, seq_ids: *const c_int, seq_q: *const c_int,
        n_seqs: c_int, stream: *mut c_void) -> c_int;
    pub fn flour_kv_batch_step(b: *mut FlourKvBatch, seq_ids: *const c_int, seq_q: *const c_int,
        n_seqs: c_int, stream: *mut c_void) -> c_int;
    pub fn flour_kv_batch_write_kv(b: *mut FlourKvBatch, layer: c_int, k: *const c_void,
        v: *const c_void, stride_tok: i64, stride_head: i64, stream: *mut c_void) -> c_int;
    pub fn flour_kv_batch_rope_write_kv(b: *mut FlourKvBatch, layer: c_int, q_out: *mut c_void,
        q: *const c_void, q_stride_tok: i64, q_stride_head: i64, num_heads: c_int,
        k: *const c_void, v: *const c_void, kv_stride_tok: i64, kv_stride_head: i64,
        cos_table: *const c_void, sin_table: *const c_void, max_pos: c_int,
        stream: *mut c_void) -> c_int;
    pub fn flour_kv_batch_attention(b: *mut FlourKvBatch, layer: c_int, q: *const c_void,
        num_heads: c_int, q_stride_tok: i64, q_stride_head: i64, out: *mut c_void,
        out_dtype: c_int, o_stride_tok: i64, o_stride_head: i64, scale: f32,
        stream: *mut c_void) -> c_int;
    pub fn flour_kv_batch_write_kv_attention(b: *mut FlourKvBatch, layer: c_int,
        k: *const c_void, v: *const c_void, kv_stride_tok: i64, kv_stride_head: i64,
        q: *const c_void, num_heads: c_int, q_stride_tok: i64, q_stride_head: i64,
        out: *mut c_void, out_dtype: c_int, o_stride_tok: i64, o_stride_head: i64, scale: f32,
        stream: *mut c_void) -> c_int;
    pub fn flour_kv_batch_pool(b: *const FlourKvBatch, layer: c_int, k_pool: *mut *mut c_void,
        v_pool: *mut *mut c_void, num_slots: *mut i64) -> c_int;
}

/// An error returned by the library: the negative code and the message of
/// `flour_hip_last_error()` on the calling thread.
#[derive(Debug, Clone)]
pub struct FlourError {
    pub code: c_int,
    pub message: String,
}

impl std::fmt::Display for FlourError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "flour_hip error {}: {}", self.code, self.message)
    }
}

impl std::error::Error for FlourError {}

/// Maps a return code to `Ok(())` or the library's message for this thread, for the
/// reference's `candle_core::Error::Msg` mapping (`bail!` paths propagated with `?` into
/// `anyhow` at `engine.rs:194`, `:260-262`).
pub fn check(code: c_int) -> Result<(), FlourError> {
    if code == FLOUR_OK {
        return Ok(());
    }
    // SAFETY: the library returns a pointer to a NUL-terminated thread-local string.
    let message = unsafe { CStr::from_ptr(flour_hip_last_error()) }.to_string_lossy().into_owned();
    Err(FlourError { code, message })
}
