// rope_kv_write.hip — rotary position embedding on the new q / k rows, fused with the KV-cache
// write.
//
// Replaces the steps of CausalSelfAttention::forward at src/models/common/attention.rs:96-104:
// rope(q) and rope(k) (candle_nn::rotary_emb::rope, the non-interleaved "rotate half" form, with
// the cos / sin tables of cache.rs:377-393 narrowed to index_pos .. index_pos + seq_len by
// Cache::rope_cos / rope_sin, cache.rs:404-410), then Cache::write_kv (the scatter of
// PagedKvPool::write, paged.rs:186-187). One pass over the new rows: q is rotated into q_out,
// k is rotated straight into its pool slot and v is copied there, so the rotated k never makes
// a round trip through HBM before the write.
//
// Numerics, for a row x of head_dim d at table row p and i < d/2, with c = cos[p][i] and
// s = sin[p][i]:
//   y[i]       = x[i]·c − x[i+d/2]·s
//   y[i+d/2]   = x[i]·s + x[i+d/2]·c
// every product and every sum rounded to the tensor dtype, as the CPU kernel of candle's rope
// evaluates them in the element type (bf16 / f16 operations go through f32 and round to nearest
// even; products of two 16-bit values are exact in f32, so the GPU reproduces each rounding).
// fp32 uses non-contracted multiplies and adds.
//
// Design: HBM-bound streaming. One lane per (token, row, chunk of P pairs), P = 16 bytes of
// elements: for a 16-bit head_dim-128 row, 8 lanes each read 16 B of x[i..], 16 B of x[i+64..]
// and 16 B of each table row (the tables stay in L2), and write 2 x 16 B. Rows are the
// num_heads q rows, the kv_heads k rows and the kv_heads v rows of a token; v lanes copy the
// same two 16 B chunks unchanged. Shapes whose addresses are not 16-byte aligned use one pair
// per lane.
#include "flour_common.h"

namespace flour {

template <typename T>
__device__ __forceinline__ float rnd(float x) {  // round to the storage type and back
    return to_f32(from_f32<T>(x));
}
template <>
__device__ __forceinline__ float rnd<float>(float x) {
    return x;
}

// One rotated pair in the element type's arithmetic.
template <typename T>
__device__ __forceinline__ void rope_pair(float x1, float x2, float c, float s, float& y1,
                                          float& y2) {
    // No contraction: fp32 products and sums round separately, and for fp16 the compiler
    // narrows round(x * c) to a native fp16 multiply (same result), which it would otherwise
    // fuse with the sum into an fma, skipping a rounding.
#pragma clang fp contract(off)
    if constexpr (std::is_same<T, float>::value) {
        y1 = x1 * c - x2 * s;
        y2 = x1 * s + x2 * c;
    } else {
        // products of two 16-bit values are exact in fp32; each is then rounded, as is the sum
        y1 = rnd<T>(rnd<T>(x1 * c) - rnd<T>(x2 * s));
        y2 = rnd<T>(rnd<T>(x1 * s) + rnd<T>(x2 * c));
    }
}

// P consecutive elements of storage type T (float / bf16_t / f16_t), moved as one access.
template <typename T, int P>
struct Chunk {
    T e[P];
};

template <typename T, int P>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(
    T* q_out, const T* q, int64_t q_st, int64_t q_sh, int num_heads,  // q_out may alias q
    const T* __restrict__ k, const T* __restrict__ v, int64_t kv_st, int64_t kv_sh,
    T* __restrict__ k_pool, T* __restrict__ v_pool, const int32_t* __restrict__ slot_mapping,
    const int32_t* __restrict__ positions, const T* __restrict__ cos_t,
    const T* __restrict__ sin_t, int max_pos, int num_tokens, int kv_heads, int head_dim,
    int64_t num_slots, int lanes_per_row, int per_token) {
    typedef Chunk<T, P> C;
    const int idx = (int)(blockIdx.x * blockDim.x + threadIdx.x);  // < 2^31 (checked on launch)
    const int t = idx / per_token;
    if (t >= num_tokens) return;
    const int u = idx - t * per_token;
    const int row = u / lanes_per_row;
    const int i0 = (u - row * lanes_per_row) * P;  // first pair of this lane
    const int half = head_dim >> 1;
    const int p = positions[t];
    if (p < 0 || p >= max_pos) return;  // no table row: the token is left unwritten
    const bool is_q = row < num_heads;
    const int h = is_q ? row : (row - num_heads) % kv_heads;
    const bool is_v = row >= num_heads + kv_heads;
    int64_t dst_off = 0;
    if (!is_q) {
        const int64_t slot = slot_mapping[t];
        if (slot < 0 || slot >= num_slots) return;  // padding token: no K/V write
        dst_off = ((int64_t)h * num_slots + slot) * head_dim;
    }
    const T* src = is_q ? q + (int64_t)t * q_st + (int64_t)h * q_sh
                        : (is_v ? v : k) + (int64_t)t * kv_st + (int64_t)h * kv_sh;
    T* dst = is_q ? q_out + (int64_t)t * q_st + (int64_t)h * q_sh
                  : (is_v ? v_pool : k_pool) + dst_off;
    const C a = *reinterpret_cast<const C*>(src + i0);
    const C b = *reinterpret_cast<const C*>(src + i0 + half);
    if (is_v) {
        *reinterpret_cast<C*>(dst + i0) = a;
        *reinterpret_cast<C*>(dst + i0 + half) = b;
        return;
    }
    const C cc = *reinterpret_cast<const C*>(cos_t + (int64_t)p * half + i0);
    const C ss = *reinterpret_cast<const C*>(sin_t + (int64_t)p * half + i0);
    C ya, yb;
#pragma unroll
    for (int j = 0; j < P; j++) {
        float y1, y2;
        rope_pair<T>(to_f32(a.e[j]), to_f32(b.e[j]), to_f32(cc.e[j]), to_f32(ss.e[j]), y1, y2);
        ya.e[j] = from_f32<T>(y1);
        yb.e[j] = from_f32<T>(y2);
    }
    *reinterpret_cast<C*>(dst + i0) = ya;
    *reinterpret_cast<C*>(dst + i0 + half) = yb;
}

template <typename T>
static int launch_rope_kv_write(void* q_out, const void* q, int64_t q_st, int64_t q_sh,
                                int num_heads, const void* k, const void* v, int64_t kv_st,
                                int64_t kv_sh, void* k_pool, void* v_pool, const int32_t* slots,
                                const int32_t* positions, const void* cos_t, const void* sin_t,
                                int max_pos, int num_tokens, int kv_heads, int head_dim,
                                int64_t num_slots, bool vec, hipStream_t stream) {
    constexpr int PV = 16 / (int)sizeof(T);
    const int P = vec ? PV : 1;
    const int lanes_per_row = (head_dim / 2) / P;
    const int64_t per_token = (int64_t)(num_heads + 2 * kv_heads) * lanes_per_row;
    const int64_t threads = per_token * num_tokens;
    if ((threads + 255) / 256 * 256 > 0x7fffffff) {
        set_error("rope_kv_write: %d tokens x %lld lanes exceed one launch", num_tokens,
                  (long long)per_token);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    const int64_t blocks = (threads + 255) / 256;
    auto go = [&](auto kern) {
        kern<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(
            static_cast<T*>(q_out), static_cast<const T*>(q), q_st, q_sh, num_heads,
            static_cast<const T*>(k), static_cast<const T*>(v), kv_st, kv_sh,
            static_cast<T*>(k_pool), static_cast<T*>(v_pool), slots, positions,
            static_cast<const T*>(cos_t), static_cast<const T*>(sin_t), max_pos, num_tokens,
            kv_heads, head_dim, num_slots, lanes_per_row, (int)per_token);
    };
    if (vec)
        go(rope_kv_write_kernel<T, PV>);
    else
        go(rope_kv_write_kernel<T, 1>);
    return check_hip(hipGetLastError(), "rope_kv_write launch");
}

}  // namespace flour

using namespace flour;

extern "C" int flour_hip_rope_kv_write(void* q_out, const void* q, int64_t q_stride_tok,
                                       int64_t q_stride_head, int num_heads, const void* k,
                                       const void* v, int64_t kv_stride_tok,
                                       int64_t kv_stride_head, void* k_pool, void* v_pool,
                                       const int32_t* slot_mapping, const int32_t* positions,
                                       const void* cos_table, const void* sin_table, int max_pos,
                                       int num_tokens, int kv_heads, int head_dim,
                                       int64_t num_slots, int dtype, void* stream) {
    clear_error();
    if (!valid_dtype(dtype)) {
        set_error("rope_kv_write: unknown dtype %d", dtype);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (num_tokens < 0 || num_heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
        (head_dim & 1) != 0 || num_slots <= 0 || max_pos <= 0) {
        set_error("rope_kv_write: bad shape (num_tokens=%d num_heads=%d kv_heads=%d "
                  "head_dim=%d num_slots=%lld max_pos=%d; head_dim must be even)",
                  num_tokens, num_heads, kv_heads, head_dim, (long long)num_slots, max_pos);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (num_tokens == 0) return FLOUR_OK;
    if (!q_out || !q || !k || !v || !k_pool || !v_pool || !slot_mapping || !positions ||
        !cos_table || !sin_table) {
        set_error("rope_kv_write: null pointer");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    const int64_t es = elem_bytes(dtype);
    // 16-byte chunks need every row start, half-row offset and table row 16-byte aligned.
    const uint64_t align_bits =
        (uint64_t)(q_stride_tok * es) | (uint64_t)(q_stride_head * es) |
        (uint64_t)(kv_stride_tok * es) | (uint64_t)(kv_stride_head * es) |
        (uint64_t)(head_dim / 2 * es) | (uint64_t)(uintptr_t)q_out | (uint64_t)(uintptr_t)q |
        (uint64_t)(uintptr_t)k | (uint64_t)(uintptr_t)v | (uint64_t)(uintptr_t)k_pool |
        (uint64_t)(uintptr_t)v_pool | (uint64_t)(uintptr_t)cos_table |
        (uint64_t)(uintptr_t)sin_table;
    const bool vec = (align_bits & 15) == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case FLOUR_DTYPE_F32:
            return launch_rope_kv_write<float>(q_out, q, q_stride_tok, q_stride_head, num_heads,
                                               k, v, kv_stride_tok, kv_stride_head, k_pool,
                                               v_pool, slot_mapping, positions, cos_table,
                                               sin_table, max_pos, num_tokens, kv_heads,
                                               head_dim, num_slots, vec, s);
        case FLOUR_DTYPE_BF16:
            return launch_rope_kv_write<bf16_t>(q_out, q, q_stride_tok, q_stride_head,
                                                num_heads, k, v, kv_stride_tok, kv_stride_head,
                                                k_pool, v_pool, slot_mapping, positions,
                                                cos_table, sin_table, max_pos, num_tokens,
                                                kv_heads, head_dim, num_slots, vec, s);
        default:
            return launch_rope_kv_write<f16_t>(q_out, q, q_stride_tok, q_stride_head, num_heads,
                                               k, v, kv_stride_tok, kv_stride_head, k_pool,
                                               v_pool, slot_mapping, positions, cos_table,
                                               sin_table, max_pos, num_tokens, kv_heads,
                                               head_dim, num_slots, vec, s);
    }
}
