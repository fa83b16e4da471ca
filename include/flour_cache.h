/*
 * flour_cache.h — host-side KV-cache bookkeeping over a device pool, the C-ABI of the layer
 * that sits directly above the kernels of flour_hip.h in libflour_hip.so.
 *
 * It restates the reference's per-sequence cache (reference files cited as path:line,
 * relative to the lltsdyp/flour checkout):
 *
 *   src/models/common/paged.rs:7-54     BlockAllocator (LIFO free list, per-block refcounts)
 *   src/models/common/paged.rs:57-121   BlockTable (logical position -> physical slot)
 *   src/models/common/prefix.rs:1-60    block_hash / PrefixRegistry (chained full-block hashes)
 *   src/models/common/paged.rs:138-167  PagedKvPool::new (here: device arrays, zero-filled)
 *   src/models/common/cache.rs:13-165   KvCache (allocate, write_current, gather_blocks,
 *                                       reset_sequence, match_prefix, register_prefix)
 *   src/models/common/cache.rs:429-505  Cache::allocate_kv / write_kv / kv_blocks / ...
 *   src/models/common/cache.rs:166-340  export_prefix_bundle / import_prefix_bundle, with the
 *   src/kv_cache/bundle.rs:1-214        FLKV frame of KvBundleCodec::encode / decode
 *
 * and replaces the `kv_blocks` + `paged_attention` pair of the attention layer
 * (src/models/common/attention.rs:104-109) by one call that marshals the block table to the
 * device and launches the decode (seq_q == 1) or prefill kernel.
 *
 * Conventions are those of flour_hip.h: FLOUR_OK or a negative FLOUR_ERR_* code, with the
 * message in flour_hip_last_error(). Functions of one cache must not be called concurrently.
 * Block ids and slots are int32 (the pool holds fewer than 2^31 slots).
 */
#ifndef FLOUR_CACHE_H
#define FLOUR_CACHE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- BlockAllocator (paged.rs:7-54) --------------------------------------------------- */
typedef struct flour_block_allocator flour_block_allocator;

/* BlockAllocator::new: every block free; the first allocate returns block 0 (paged.rs:13-19). */
int flour_block_allocator_create(int num_blocks, flour_block_allocator** out);
void flour_block_allocator_destroy(flour_block_allocator* a);
/* BlockAllocator::allocate: a block id with refcount 1, or -1 when none is free (None). */
int flour_block_allocator_allocate(flour_block_allocator* a);
/* BlockAllocator::incref. */
int flour_block_allocator_incref(flour_block_allocator* a, int block_id);
/* BlockAllocator::decref: 1 when the block reached zero references and was freed, else 0;
 * FLOUR_ERR_INVALID_ARGUMENT for an unreferenced or unknown block (a debug_assert there). */
int flour_block_allocator_decref(flour_block_allocator* a, int block_id);
int flour_block_allocator_ref_count(const flour_block_allocator* a, int block_id);
int flour_block_allocator_num_free(const flour_block_allocator* a);

/* ---- BlockTable (paged.rs:57-121) ----------------------------------------------------- */
typedef struct flour_block_table flour_block_table;

int flour_block_table_create(int block_size, flour_block_table** out);
void flour_block_table_destroy(flour_block_table* t);
int flour_block_table_push_block(flour_block_table* t, int block_id);
int flour_block_table_advance(flour_block_table* t, int n);
int flour_block_table_clear(flour_block_table* t);
int flour_block_table_len(const flour_block_table* t);
int flour_block_table_capacity(const flour_block_table* t);
int flour_block_table_block_size(const flour_block_table* t);
/* BlockTable::blocks: copies up to `cap` ids to `out`, stores the count in *n. */
int flour_block_table_blocks(const flour_block_table* t, int32_t* out, int cap, int* n);
/* BlockTable::slot / slots(start, end): blocks[pos / bs] * bs + pos % bs. Positions must be
 * backed by a pushed block. */
int64_t flour_block_table_slot(const flour_block_table* t, int pos);
int flour_block_table_slots(const flour_block_table* t, int start, int end, int32_t* out);

/* ---- KvCache + Cache (cache.rs) -------------------------------------------------------- */
typedef struct flour_kv_cache flour_kv_cache;

/* KvCache::new (cache.rs:21-41): ceil(max_seq_len / block_size) blocks. With device_pool != 0
 * the per-layer K and V pools (kv_heads, num_slots, head_dim) are allocated zero-filled on the
 * current HIP device, together with the small device buffers the kernels read (block table,
 * slot mapping, lengths, decode workspace for up to num_heads query heads); with
 * device_pool == 0 only the bookkeeping exists (write_kv / attention then fail). */
int flour_kv_cache_create(int num_layers, int max_seq_len, int num_heads, int kv_heads,
                          int head_dim, int block_size, int dtype, int device_pool,
                          flour_kv_cache** out);
void flour_kv_cache_destroy(flour_kv_cache* c);

/* Cache::allocate_kv (cache.rs:429-447): reserve blocks for seq_len more tokens and advance
 * the live length. Errors: "paged kv cache overflow" past max_seq_len (FLOUR_ERR_CAPACITY),
 * "out of kv blocks" (FLOUR_ERR_OUT_OF_BLOCKS). */
int flour_kv_cache_allocate_kv(flour_kv_cache* c, int seq_len);
int flour_kv_cache_len(const flour_kv_cache* c);
int flour_kv_cache_capacity(const flour_kv_cache* c);
/* KvCache::free_blocks (cache.rs:361-363). */
int flour_kv_cache_free_blocks(const flour_kv_cache* c);
int flour_kv_cache_ref_count(const flour_kv_cache* c, int block_id);
/* The live block table (BlockTable::blocks) and KvCache::slots(start, end). */
int flour_kv_cache_blocks(const flour_kv_cache* c, int32_t* out, int cap, int* n);
int flour_kv_cache_slots(const flour_kv_cache* c, int start, int end, int32_t* out);

/* Cache::write_kv -> KvCache::write_current (cache.rs:71-77): the trailing seq_len tokens of
 * the live sequence take k/v element (t, h, d) at t*stride_tok + h*stride_head + d
 * (device memory; the reference's (1, kv_heads, seq, head_dim) is stride_tok = head_dim,
 * stride_head = seq_len * head_dim). Launches flour_hip_kv_write on `stream`. */
int flour_kv_cache_write_kv(flour_kv_cache* c, int layer, const void* k, const void* v,
                            int seq_len, int64_t stride_tok, int64_t stride_head, void* stream);

/* Cache::kv_blocks + paged_attention (cache.rs:456-458, cpu.rs:57-112) in one call: the
 * last seq_q rows of the live sequence attend causally to all live positions. q element
 * (row, head, d) at row*q_stride_tok + head*q_stride_head + d, out likewise with the o_
 * strides ((1, num_heads, seq_q, head_dim) is stride_tok = head_dim, stride_head =
 * seq_q * head_dim). seq_q == 1 runs the decode kernel, which requires out to be
 * (num_heads, head_dim) contiguous. The block table is copied to the device on `stream` when
 * it changed since the last call. */
int flour_kv_cache_attention(flour_kv_cache* c, int layer, const void* q, int num_heads,
                             int seq_q, int64_t q_stride_tok, int64_t q_stride_head, void* out,
                             int out_dtype, int64_t o_stride_tok, int64_t o_stride_head,
                             float scale, void* stream);

/* KvCache::reset_sequence (cache.rs:100-108). */
int flour_kv_cache_reset_sequence(flour_kv_cache* c);
/* KvCache::match_prefix (cache.rs:112-143): tokens served from cached full blocks (a multiple
 * of block_size; never the whole prompt). */
int flour_kv_cache_match_prefix(flour_kv_cache* c, const uint32_t* tokens, int n);
/* KvCache::register_prefix (cache.rs:145-159). */
int flour_kv_cache_register_prefix(flour_kv_cache* c, const uint32_t* tokens, int n);
/* KvCache::clear_prefix_cache (cache.rs:354-359). */
int flour_kv_cache_clear_prefix_cache(flour_kv_cache* c);

/* ---- FLKV bundles (src/kv_cache/bundle.rs:1-22, cache.rs:166-340) ----------------------
 * Frame: "FLKV", version u16 LE = 1, header_len u32 LE, the KvBundleMeta header as serde_json
 * writes it (fields model_id, token_count, token_ids, block_size, num_layers, num_kv_heads,
 * head_dim, dtype "F32"/"F16"/"BF16"), then per logical block, per layer, the K block and the V
 * block, each (kv_heads, block_size, head_dim) little-endian in the pool dtype. */

/* Cache::export_prefix_bundle (cache.rs:166-229) + KvBundleCodec::encode (bundle.rs:108-143):
 * the frame of the first token_count live tokens, read from the device pools on `stream`.
 * token_count must be a positive multiple of block_size and at most the live length, and
 * token_ids must hold at least token_count ids (the reference's error messages, as
 * FLOUR_ERR_INVALID_ARGUMENT). *len receives the frame size; with out == NULL nothing else
 * is done (size query), otherwise out (host memory) must hold cap >= *len bytes
 * (FLOUR_ERR_CAPACITY) and the call returns once it is filled. */
int flour_kv_cache_export_bundle(flour_kv_cache* c, const char* model_id,
                                 const uint32_t* token_ids, int n_ids, int token_count, void* out,
                                 size_t cap, size_t* len, void* stream);

/* KvBundleCodec::decode (bundle.rs:145-214) + Cache::import_prefix_bundle (cache.rs:238-340):
 * validates the frame (magic, version, header, block alignment, payload length) and the bundle
 * against this cache (block size, layers, kv heads, head_dim, dtype) and the prompt (it must
 * start with the bundle's token ids), then resets the sequence, allocates one block per bundle
 * block, copies the payload into the device pools on `stream`, sets the live length to the
 * bundle's token count and registers the blocks as a cached prefix. *imported receives the
 * token count. Rejections leave no partial state; "not enough free kv blocks to import" is
 * FLOUR_ERR_OUT_OF_BLOCKS (the sequence has been reset, as in the reference). */
int flour_kv_cache_import_bundle(flour_kv_cache* c, const void* bytes, size_t len,
                                 const uint32_t* prompt_tokens, int n_prompt, int* imported,
                                 void* stream);

/* Device pools of one layer (PagedKvPool::block_view, paged.rs:266-279: slot s of kv head h is
 * row h * num_slots + s of each array). */
int flour_kv_cache_pool(const flour_kv_cache* c, int layer, void** k_pool, void** v_pool,
                        int64_t* num_slots);

/* ---- Many sequences over one pool (continuous batching) ------------------------------------
 * The reference engine serves one sequence at a time (one Mutex<Cache>, src/engine.rs:88, and
 * the batch-1 loop of engine.rs:219-263). A flour_kv_batch shares one device pool of num_blocks
 * blocks, one BlockAllocator and one prefix registry among up to max_seqs sequences, each with
 * its own BlockTable and KvCache's per-sequence operations (cache.rs:13-165, :429-505); a
 * sequence can reuse the full prefix blocks that another registered. A forward step is planned
 * once (flour_kv_batch_plan uploads the step's block tables, kv lengths, cu_seqlens and the
 * slot mapping of the new rows); each layer then calls write_kv and attention on that plan.
 * Any change to a sequence invalidates the plan. Functions of one batch must not be called
 * concurrently. */
typedef struct flour_kv_batch flour_kv_batch;

/* Pools (kv_heads, num_blocks * block_size, head_dim) per layer, zero-filled; table rows of
 * ceil(max_seq_len / block_size) blocks; up to max_batch_tokens new rows per step; a decode
 * workspace for max_seqs sequences. device_pool == 0 keeps only the bookkeeping. */
int flour_kv_batch_create(int num_layers, int num_blocks, int max_seqs, int max_seq_len,
                          int max_batch_tokens, int num_heads, int kv_heads, int head_dim,
                          int block_size, int dtype, int device_pool, flour_kv_batch** out);
void flour_kv_batch_destroy(flour_kv_batch* b);
/* A new empty sequence (FLOUR_ERR_CAPACITY when max_seqs are live). */
int flour_kv_batch_add_sequence(flour_kv_batch* b, int* seq_id);
/* Releases the sequence's blocks (KvCache::reset_sequence) and frees its slot. */
int flour_kv_batch_remove_sequence(flour_kv_batch* b, int seq_id);
int flour_kv_batch_reset_sequence(flour_kv_batch* b, int seq_id);
/* Cache::allocate_kv for one sequence ("paged kv cache overflow", "out of kv blocks"). */
int flour_kv_batch_allocate_kv(flour_kv_batch* b, int seq_id, int seq_len);
int flour_kv_batch_len(const flour_kv_batch* b, int seq_id);
int flour_kv_batch_free_blocks(const flour_kv_batch* b);
int flour_kv_batch_ref_count(const flour_kv_batch* b, int block_id);
int flour_kv_batch_blocks(const flour_kv_batch* b, int seq_id, int32_t* out, int cap, int* n);
/* KvCache::match_prefix into an empty sequence, over the shared registry; returns the matched
 * token count. */
int flour_kv_batch_match_prefix(flour_kv_batch* b, int seq_id, const uint32_t* tokens, int n);
int flour_kv_batch_register_prefix(flour_kv_batch* b, int seq_id, const uint32_t* tokens, int n);
int flour_kv_batch_clear_prefix_cache(flour_kv_batch* b);
/* The step: sequence seq_ids[i] brings its last seq_q[i] live positions as new rows (already
 * allocated), packed in this order (cu_seqlens). Sequences must be distinct. */
int flour_kv_batch_plan(flour_kv_batch* b, const int* seq_ids, const int* seq_q, int n_seqs,
                        void* stream);
/* allocate_kv(seq_ids[i], seq_q[i]) for every listed sequence, then plan: one call per forward
 * step (a decode step passes seq_q[i] = 1). Every check (live and distinct sequences,
 * max_seq_len, max_batch_tokens, free blocks, the device pool) runs before any allocation, so
 * a refused step leaves every sequence as it was. */
int flour_kv_batch_step(flour_kv_batch* b, const int* seq_ids, const int* seq_q, int n_seqs,
                        void* stream);
/* The KV write of the planned new rows: k/v element (t, h, d) of packed row t at
 * t*stride_tok + h*stride_head + d (flour_hip_kv_write). */
int flour_kv_batch_write_kv(flour_kv_batch* b, int layer, const void* k, const void* v,
                            int64_t stride_tok, int64_t stride_head, void* stream);
/* The fused RoPE + KV write of the planned new rows (flour_hip_rope_kv_write with the plan's
 * slot mapping and positions: row t of sequence s sits at position len(s) - seq_q(s) + t, the
 * table row the reference's rope_for_cache uses, attention.rs:96-99 then :104). q is rotated
 * into q_out (q_out == q rotates in place); rotated k and v go to the layer's pools. The
 * cos / sin tables ((max_pos, head_dim / 2), storage dtype) must cover max_seq_len positions. */
int flour_kv_batch_rope_write_kv(flour_kv_batch* b, int layer, void* q_out, const void* q,
                                 int64_t q_stride_tok, int64_t q_stride_head, int num_heads,
                                 const void* k, const void* v, int64_t kv_stride_tok,
                                 int64_t kv_stride_head, const void* cos_table,
                                 const void* sin_table, int max_pos, void* stream);
/* Attention of the planned rows: paged decode when every sequence brings one row (q and out
 * (n_seqs, num_heads, head_dim) contiguous), varlen prefill otherwise (strided packed rows).
 * A mixed step (some sequences bring one row, others more) with packed contiguous q and out
 * (row stride num_heads * head_dim, head stride head_dim) over 16-bit pools at head_dim 128
 * runs its one-row sequences as one paged-decode launch and the others as one prefill launch,
 * each over its rows of the packed layout; other mixed steps run every row on the prefill
 * kernel. */
int flour_kv_batch_attention(flour_kv_batch* b, int layer, const void* q, int num_heads,
                             int64_t q_stride_tok, int64_t q_stride_head, void* out,
                             int out_dtype, int64_t o_stride_tok, int64_t o_stride_head,
                             float scale, void* stream);
/* flour_kv_batch_write_kv followed by flour_kv_batch_attention, as one call: the order of the
 * reference's layer (Cache::write_kv, cache.rs:451-453, then paged_attention, cpu.rs:57-112).
 * A decode step (every sequence brings one row) with packed contiguous q and out over 16-bit
 * pools of 16-token blocks at head_dim 128 or 64, whose new positions sit in blocks no other
 * sequence or the prefix registry holds, runs as ONE launch: the decode kernel writes each new K / V row into
 * the pool before it attends to it (the same pools and output as the two calls, bit for bit).
 * Every other step runs the two calls. This entry point has no counterpart in the reference; it
 * is for the per-layer loop of a continuous-batching server, where the KV write of a decode
 * step's few rows costs a whole launch. */
int flour_kv_batch_write_kv_attention(flour_kv_batch* b, int layer, const void* k,
                                      const void* v, int64_t kv_stride_tok,
                                      int64_t kv_stride_head, const void* q, int num_heads,
                                      int64_t q_stride_tok, int64_t q_stride_head, void* out,
                                      int out_dtype, int64_t o_stride_tok, int64_t o_stride_head,
                                      float scale, void* stream);
int flour_kv_batch_pool(const flour_kv_batch* b, int layer, void** k_pool, void** v_pool,
                        int64_t* num_slots);

#ifdef __cplusplus
}
#endif

#endif /* FLOUR_CACHE_H */
