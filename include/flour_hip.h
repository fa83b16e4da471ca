/*
 * flour_hip.h — C-ABI of libflour_hip.so, the MI355X (gfx950) attention hot path of flour.
 *
 * The library replaces the reference's CPU attention seam (reference files cited as path:line,
 * relative to the lltsdyp/flour checkout):
 *
 *   src/backend/cpu.rs:57-112          paged_attention(q, blocks, n_rep, scale)
 *   src/models/common/paged.rs:186-204 PagedKvPool::write(layer, slots, k, v)
 *   src/models/common/paged.rs:114-121 BlockTable::slot / slots
 *   src/models/common/paged.rs:7-54    BlockAllocator
 *   src/models/common/paged.rs:138-167 PagedKvPool::new (device KV layout)
 *   src/models/common/cache.rs:429-458 Cache::allocate_kv / write_kv / kv_blocks
 *   src/models/common/cache.rs:112-159 KvCache::match_prefix / register_prefix
 *
 * Conventions
 *   - Every function returns FLOUR_OK (0) on success or a negative FLOUR_ERR_* code;
 *     flour_hip_last_error() then holds a message (per calling thread).
 *   - Device pointers are owned by the caller. Kernel launches are asynchronous and ordered on
 *     `stream` (a hipStream_t passed as void*; NULL = the default stream).
 *   - The KV pool of one layer is two device arrays, K and V, each laid out
 *     (kv_heads, num_slots, head_dim) row-major, exactly as PagedKvPool::new builds them
 *     (paged.rs:124-167). Slot s of physical block b is b * block_size + s % block_size
 *     (paged.rs:114-116), so the 16 rows of one (head, block) pair are contiguous.
 *   - Element types are given by the flour_dtype codes below. Scores, softmax and accumulators
 *     are fp32 and outputs are rounded to nearest-even. The matrix products take bf16/f16
 *     inputs exactly, with one exception: prefill over bf16 pools runs P.V on fp16 matrix
 *     cores with V converted to fp16 (exact for 2^-17 <= |v| <= 65504) and P rounded to fp16;
 *     a work item whose output is not finite or whose output block has a root mean square
 *     below 2^-25 / 5e-4 (~6e-5) is recomputed with bf16 V and P split into two bf16 parts.
 *     Decode splits P into two 16-bit parts. fp32 pools stay fp32 throughout: prefill at
 *     head_dim 64 / 128 runs on the fp32 matrix cores, every other fp32 shape on the vector
 *     ALUs.
 */
#ifndef FLOUR_HIP_H
#define FLOUR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum flour_dtype {
    FLOUR_DTYPE_F32 = 0,
    FLOUR_DTYPE_BF16 = 1,
    FLOUR_DTYPE_F16 = 2,
};

#define FLOUR_OK 0
#define FLOUR_ERR_INVALID_ARGUMENT (-1)
#define FLOUR_ERR_UNSUPPORTED (-2)
#define FLOUR_ERR_WORKSPACE (-3)
#define FLOUR_ERR_HIP (-4)
#define FLOUR_ERR_OUT_OF_BLOCKS (-5)
#define FLOUR_ERR_CAPACITY (-6)

/* Message describing the last error on the calling thread ("" if none). */
const char* flour_hip_last_error(void);

/* Library version string. */
const char* flour_hip_version(void);

/* ------------------------------------------------------------------------------------------
 * Kernel (1): KV-cache write.
 * Replaces PagedKvPool::write (src/models/common/paged.rs:186-204) as called through
 * KvCache::write_current (src/models/common/cache.rs:71-77).
 *
 * For every token t with slot_mapping[t] >= 0 and every kv head h:
 *     k_pool[h, slot_mapping[t], :] = k[t, h, :]     (and the same for v)
 * where element (t, h, d) of k / v sits at t*stride_tok + h*stride_head + d (elements).
 * The reference layout (1, kv_heads, seq, head_dim) is stride_tok = head_dim,
 * stride_head = seq*head_dim; a packed (tokens, kv_heads, head_dim) batch is
 * stride_tok = kv_heads*head_dim, stride_head = head_dim.
 * A negative slot marks a padding token and is skipped; a slot >= num_slots is never written.
 * The copy is bit-exact (no conversion): k/v and the pools share `dtype`.
 * Each non-negative slot may appear at most once per call (BlockTable::slots, paged.rs:118-121,
 * never repeats one): tokens are written in parallel, so for a repeated slot the stored row is
 * one of the repeating tokens' rows, chosen 16 bytes at a time, not the last token's. The cache
 * layers of flour_cache.h only build mappings without repeats.
 * ---------------------------------------------------------------------------------------- */
int flour_hip_kv_write(const void* k, const void* v, int64_t stride_tok, int64_t stride_head,
                       void* k_pool, void* v_pool, const int32_t* slot_mapping, int num_tokens,
                       int kv_heads, int head_dim, int64_t num_slots, int dtype, void* stream);

/* ------------------------------------------------------------------------------------------
 * RoPE + KV-cache write, fused (the step before kernel (1) in the reference, now one pass).
 * Replaces, at src/models/common/attention.rs:96-104, rope(q) and rope(k)
 * (candle_nn::rotary_emb::rope: the non-interleaved "rotate half" form) with the cos / sin
 * tables of Cache::new (cache.rs:377-393) read at the token's position (Cache::rope_cos /
 * rope_sin narrow them to index_pos.., cache.rs:404-410), then Cache::write_kv
 * (cache.rs:451-453 -> PagedKvPool::write's scatter, paged.rs:186-187).
 *
 * For token t with table row p = positions[t] and i < head_dim / 2, c = cos[p][i],
 * s = sin[p][i], a row x is rotated to
 *   y[i] = x[i]·c - x[i + head_dim/2]·s,   y[i + head_dim/2] = x[i]·s + x[i + head_dim/2]·c
 * with every product and sum rounded to `dtype` (fp32: no contraction). Then
 *   q_out[t, h, :] = rope(q[t, h, :])                               h < num_heads
 *   k_pool[h, slot_mapping[t], :] = rope(k[t, h, :]),  v_pool[h, slot_mapping[t], :] = v[t, h, :]
 * q and q_out share the strides (q_out may be q: in place); k and v share kv_stride_*.
 * cos_table / sin_table: (max_pos, head_dim / 2) row-major in `dtype`. head_dim must be even.
 * A token whose slot is outside [0, num_slots) writes no K/V (its q row is still rotated);
 * one whose position is outside [0, max_pos) writes nothing.
 * ---------------------------------------------------------------------------------------- */
int flour_hip_rope_kv_write(void* q_out, const void* q, int64_t q_stride_tok,
                            int64_t q_stride_head, int num_heads, const void* k, const void* v,
                            int64_t kv_stride_tok, int64_t kv_stride_head, void* k_pool,
                            void* v_pool, const int32_t* slot_mapping, const int32_t* positions,
                            const void* cos_table, const void* sin_table, int max_pos,
                            int num_tokens, int kv_heads, int head_dim, int64_t num_slots,
                            int dtype, void* stream);

/* ------------------------------------------------------------------------------------------
 * Kernel (2): paged decode attention (one new query token per sequence).
 * Replaces paged_attention (src/backend/cpu.rs:57-112) for seq_q == 1, batched over sequences,
 * with the block list of Cache::kv_blocks (cache.rs:456-458 -> KvCache::gather_blocks
 * cache.rs:83-96) given as a block table.
 *
 *   q            (batch, num_heads, head_dim) contiguous, post-RoPE
 *   out          (batch, num_heads, head_dim) contiguous, element type out_dtype
 *   block_tables [batch, max_blocks_per_seq] int32 physical block ids, logical order
 *   context_lens [batch] int32 kv length of each sequence (>= 1; 0 gives a zero row; a
 *                length above max_context_len attends the first max_context_len positions)
 *   Query head h attends kv head h / (num_heads / kv_heads) (repeat_kv, cpu.rs:5-13).
 *   scale multiplies q.k before the softmax (attention.rs:108 passes 1/sqrt(head_dim)).
 *   max_context_len bounds context_lens[] and sizes the split-context grid.
 *
 * Long contexts are split across workgroups; partial (max, sum, acc) rows and the batch's
 * per-sequence chunk prefix sums go to `workspace` (device memory, 256-byte aligned, no
 * initialisation needed) and a second kernel on the same stream merges them.
 * flour_hip_paged_decode_workspace_size gives the bytes required; calls that share a
 * workspace must not overlap in time.
 * ---------------------------------------------------------------------------------------- */
int flour_hip_paged_decode_workspace_size(int batch, int num_heads, int kv_heads, int head_dim,
                                          int max_context_len, size_t* bytes);

int flour_hip_paged_decode(void* out, int out_dtype, const void* q, const void* k_pool,
                           const void* v_pool, const int32_t* block_tables,
                           int max_blocks_per_seq, const int32_t* context_lens, int batch,
                           int num_heads, int kv_heads, int head_dim, int block_size,
                           int64_t num_slots, int max_context_len, float scale, int dtype,
                           void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * Paged decode with no allocation anywhere: flour_hip_paged_decode without the workspace
 * arguments. This entry point has no counterpart in the reference; it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). The split-context workspace comes from a device array inside the
 * library, one per GPU (flour_hip_paged_decode_noalloc_max_workspace() bytes, 40 MiB, held
 * until the process ends). Arguments, results and kernels are those of flour_hip_paged_decode.
 * A call whose workspace would exceed that size fails with FLOUR_ERR_WORKSPACE before any
 * launch (at 256 CUs every shape the MFMA path takes fits; larger GQA groups or batches than
 * that would need flour_hip_paged_decode). Every call on one GPU shares that GPU's array:
 * calls that overlap in time on one GPU (different streams, or threads without ordering) race
 * and give wrong results. Nothing needs to start at zero; the array keeps the last call's
 * contents.
 * ---------------------------------------------------------------------------------------- */
size_t flour_hip_paged_decode_noalloc_max_workspace(void);

int flour_hip_paged_decode_noalloc(void* out, int out_dtype, const void* q, const void* k_pool,
                                   const void* v_pool, const int32_t* block_tables,
                                   int max_blocks_per_seq, const int32_t* context_lens,
                                   int batch, int num_heads, int kv_heads, int head_dim,
                                   int block_size, int64_t num_slots, int max_context_len,
                                   float scale, int dtype, void* stream);

/* ------------------------------------------------------------------------------------------
 * Kernel (3): causal varlen prefill attention over the paged cache.
 * Replaces paged_attention (src/backend/cpu.rs:57-112) for seq_q >= 1, batched over packed
 * sequences. Sequence s owns query rows cu_seqlens_q[s] .. cu_seqlens_q[s+1]-1 and attends
 * kv_lens[s] cached positions (its suffix plus any prefix-cached shared blocks), with the
 * reference's causal rule (cpu.rs:68, :88-95): query i of a sequence with q_len rows sees kv
 * position j iff j <= kv_len - q_len + i.
 *
 *   q    row r, head h at r*q_stride_tok + h*q_stride_head (elements), head_dim contiguous
 *   out  row r, head h at r*o_stride_tok + h*o_stride_head, element type out_dtype
 *   cu_seqlens_q [num_seqs+1] int32, kv_lens [num_seqs] int32 (kv_len >= q_len; a sequence
 *                with kv_len < q_len attends nothing and its rows are written as zeros)
 *   block_tables [num_seqs, max_blocks_per_seq] int32
 *   max_seqlen_q bounds the per-sequence query count; total_q = cu_seqlens_q[num_seqs].
 * The K/V of the new rows must already be in the pool (flour_hip_kv_write).
 * This entry point allocates nothing and needs no workspace: the kernel gathers every K/V
 * tile through registers into LDS.
 * ---------------------------------------------------------------------------------------- */
int flour_hip_varlen_prefill(void* out, int out_dtype, int64_t o_stride_tok,
                             int64_t o_stride_head, const void* q, int64_t q_stride_tok,
                             int64_t q_stride_head, const void* k_pool, const void* v_pool,
                             const int32_t* cu_seqlens_q, const int32_t* kv_lens,
                             const int32_t* block_tables, int max_blocks_per_seq, int num_seqs,
                             int max_seqlen_q, int total_q, int num_heads, int kv_heads,
                             int head_dim, int block_size, int64_t num_slots, float scale,
                             int dtype, void* stream);

/* ------------------------------------------------------------------------------------------
 * Kernel (3) with a caller-owned workspace: flour_hip_varlen_prefill plus `workspace` (device
 * memory, 256-byte aligned, no initialisation needed). Same arguments, results and
 * replacement of paged_attention (cpu.rs:57-112, seq_q >= 1) as flour_hip_varlen_prefill.
 *
 * With long prompts (at least 1,536 new rows per sequence on average) over 16-bit pools at
 * head_dim 128 the call stages V once into the workspace (every 16-token page of each
 * sequence, widened to fp16 and transposed, by a pre-pass kernel on `stream`) and the
 * attention kernel then loads both K and V tiles straight into LDS. Otherwise, or when
 * workspace_bytes is below flour_hip_varlen_prefill_workspace_size() for the call's
 * num_seqs and max_blocks_per_seq, the call runs exactly as flour_hip_varlen_prefill (the
 * workspace is not touched). Nothing is allocated either way. Calls that share a workspace
 * must not overlap in time.
 * ---------------------------------------------------------------------------------------- */
int flour_hip_varlen_prefill_workspace_size(int num_seqs, int max_blocks_per_seq,
                                            int block_size, int kv_heads, int head_dim,
                                            int dtype, size_t* bytes);

int flour_hip_varlen_prefill_ws(void* out, int out_dtype, int64_t o_stride_tok,
                                int64_t o_stride_head, const void* q, int64_t q_stride_tok,
                                int64_t q_stride_head, const void* k_pool, const void* v_pool,
                                const int32_t* cu_seqlens_q, const int32_t* kv_lens,
                                const int32_t* block_tables, int max_blocks_per_seq,
                                int num_seqs, int max_seqlen_q, int total_q, int num_heads,
                                int kv_heads, int head_dim, int block_size, int64_t num_slots,
                                float scale, int dtype, void* workspace, size_t workspace_bytes,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLOUR_HIP_H */
