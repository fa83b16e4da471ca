// kv_write.hip — kernel (1): scatter new K/V rows into the paged pool through slot_mapping.
//
// Replaces PagedKvPool::write (src/models/common/paged.rs:186-204) with its documented
// semantics pool[h, slots[t], :] = k[t, h, :] (paged.rs:186-187, test :287-306). The
// reference's run loop at paged.rs:192-202 has a run condition (:196) that reduces to
// `i == slots[i]`; for mappings without such a run start both agree bit for bit, and this
// kernel implements the scatter for every mapping (the quirk is a reference bug).
//
// Design: HBM-bound byte copy. A lane moves one 16-byte (or narrower, when alignment forbids)
// vector of K and the same of V for each of KW_ROUNDS tokens, so a 128-dim bf16 row (256 B) is
// 16 lanes and a wave moves 4 full rows per instruction. A lane reads its tokens' slots, then
// issues every load, then every store: one latency chain (slot, rows) per lane instead of one
// per token, and a grid small enough to be resident at once.
#include "flour_common.h"

namespace flour {

// Tokens per lane (a workgroup covers KW_ROUNDS groups). Measured on a 9.6K-token batch:
// 1 -> 18.8 us, 2 and 4 -> 17.8 us, 8 -> 19.5 us.
static constexpr int KW_ROUNDS = 4;

template <typename VecT>
__global__ __launch_bounds__(256) void kv_write_kernel(
    const char* __restrict__ k, const char* __restrict__ v, int64_t stride_tok_b,
    int64_t stride_head_b, char* __restrict__ k_pool, char* __restrict__ v_pool,
    const int32_t* __restrict__ slot_mapping, int num_tokens, int kv_heads, int vecs_per_row,
    int tokens_per_block, int64_t row_bytes, int64_t num_slots) {
    const int per_token = kv_heads * vecs_per_row;
    const int t_local = threadIdx.x / per_token;
    const int rem = threadIdx.x - t_local * per_token;
    if (t_local >= tokens_per_block) return;
    const int h = rem / vecs_per_row;
    const int c = rem - h * vecs_per_row;
    const int64_t src_lane = (int64_t)h * stride_head_b + (int64_t)c * sizeof(VecT);
    const int64_t dst_lane = (int64_t)h * num_slots * row_bytes + (int64_t)c * sizeof(VecT);
    // Token of round i: consecutive groups of tokens_per_block tokens. Loads are unconditional
    // (a token past the end reads the last token's row, a padding token its own row) so that the
    // compiler issues them back to back; only the stores are guarded.
    const int64_t t0 = (int64_t)blockIdx.x * tokens_per_block * KW_ROUNDS + t_local;
    int64_t slot[KW_ROUNDS];
#pragma unroll
    for (int i = 0; i < KW_ROUNDS; i++) {
        const int64_t t = t0 + (int64_t)i * tokens_per_block;
        slot[i] = slot_mapping[t < num_tokens ? t : num_tokens - 1];
    }
    VecT kv[KW_ROUNDS], vv[KW_ROUNDS];
#pragma unroll
    for (int i = 0; i < KW_ROUNDS; i++) {
        const int64_t t = t0 + (int64_t)i * tokens_per_block;
        const int64_t src = (t < num_tokens ? t : num_tokens - 1) * stride_tok_b + src_lane;
        kv[i] = *reinterpret_cast<const VecT*>(k + src);
        vv[i] = *reinterpret_cast<const VecT*>(v + src);
    }
    // keep the loads here (slots and rows): otherwise the compiler sinks each into its guarded
    // store, where it becomes a conditional load that is waited for before the next is issued
#pragma unroll
    for (int i = 0; i < KW_ROUNDS; i++) asm volatile("" ::"v"(kv[i]), "v"(vv[i]), "v"(slot[i]));
#pragma unroll
    for (int i = 0; i < KW_ROUNDS; i++) {
        const int64_t t = t0 + (int64_t)i * tokens_per_block;
        // tokens past the end, padding tokens (slot < 0) and slots outside the pool are skipped
        if (t < num_tokens && slot[i] >= 0 && slot[i] < num_slots) {
            const int64_t dst = slot[i] * row_bytes + dst_lane;
            *reinterpret_cast<VecT*>(k_pool + dst) = kv[i];
            *reinterpret_cast<VecT*>(v_pool + dst) = vv[i];
        }
    }
}

// Workgroup shape: enough whole tokens to fill up to 256 lanes, KW_ROUNDS groups of them.
template <typename VecT>
static int launch_kv_write(const void* k, const void* v, int64_t stride_tok, int64_t stride_head,
                           void* k_pool, void* v_pool, const int32_t* slots, int num_tokens,
                           int kv_heads, int64_t row_bytes, int64_t num_slots, int es,
                           hipStream_t stream) {
    const int vecs_per_row = (int)(row_bytes / (int64_t)sizeof(VecT));
    const int per_token = kv_heads * vecs_per_row;
    int tokens_per_block = per_token >= 256 ? 1 : 256 / per_token;
    int threads = per_token * tokens_per_block;
    if (threads > 1024) {
        set_error("kv_write: kv_heads*head_dim too large for one workgroup (%d vectors)",
                  per_token);
        return FLOUR_ERR_UNSUPPORTED;
    }
    threads = (threads + 63) / 64 * 64;
    const int64_t per_block = (int64_t)tokens_per_block * KW_ROUNDS;
    const int64_t blocks = ((int64_t)num_tokens + per_block - 1) / per_block;
    if (blocks > 0x7fffffff) {
        set_error("kv_write: too many tokens (%d)", num_tokens);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    kv_write_kernel<VecT><<<dim3((unsigned)blocks), dim3(threads), 0, stream>>>(
        static_cast<const char*>(k), static_cast<const char*>(v), stride_tok * es,
        stride_head * es, static_cast<char*>(k_pool), static_cast<char*>(v_pool), slots,
        num_tokens, kv_heads, vecs_per_row, tokens_per_block, row_bytes, num_slots);
    return check_hip(hipGetLastError(), "kv_write launch");
}

}  // namespace flour

using namespace flour;

extern "C" int flour_hip_kv_write(const void* k, const void* v, int64_t stride_tok,
                                  int64_t stride_head, void* k_pool, void* v_pool,
                                  const int32_t* slot_mapping, int num_tokens, int kv_heads,
                                  int head_dim, int64_t num_slots, int dtype, void* stream) {
    clear_error();
    if (!valid_dtype(dtype)) {
        set_error("kv_write: unknown dtype %d", dtype);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (num_tokens < 0 || kv_heads <= 0 || head_dim <= 0 || num_slots <= 0) {
        set_error("kv_write: bad shape (num_tokens=%d kv_heads=%d head_dim=%d num_slots=%lld)",
                  num_tokens, kv_heads, head_dim, (long long)num_slots);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (num_tokens == 0) return FLOUR_OK;
    if (!k || !v || !k_pool || !v_pool || !slot_mapping) {
        set_error("kv_write: null pointer");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    const int es = elem_bytes(dtype);
    const int64_t row_bytes = (int64_t)head_dim * es;
    // Widest vector that every address is aligned to.
    uint64_t align_bits = (uint64_t)row_bytes | (uint64_t)(stride_tok * es) |
                          (uint64_t)(stride_head * es) | (uint64_t)(uintptr_t)k |
                          (uint64_t)(uintptr_t)v | (uint64_t)(uintptr_t)k_pool |
                          (uint64_t)(uintptr_t)v_pool;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if ((align_bits & 15) == 0)
        return launch_kv_write<u32x4>(k, v, stride_tok, stride_head, k_pool, v_pool, slot_mapping,
                                      num_tokens, kv_heads, row_bytes, num_slots, es, s);
    if ((align_bits & 7) == 0)
        return launch_kv_write<u32x2>(k, v, stride_tok, stride_head, k_pool, v_pool, slot_mapping,
                                      num_tokens, kv_heads, row_bytes, num_slots, es, s);
    if ((align_bits & 3) == 0)
        return launch_kv_write<uint32_t>(k, v, stride_tok, stride_head, k_pool, v_pool,
                                         slot_mapping, num_tokens, kv_heads, row_bytes, num_slots,
                                         es, s);
    return launch_kv_write<uint16_t>(k, v, stride_tok, stride_head, k_pool, v_pool, slot_mapping,
                                     num_tokens, kv_heads, row_bytes, num_slots, es, s);
}
