// flour_common.h — shared device helpers and host error plumbing for libflour_hip.so (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <exception>
#include <new>
#include <string>

#include "flour_hip.h"

namespace flour {

// ------------------------------------------------------------------ vector types
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(2))) uint16_t u16x2;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

// Tag types for the 16-bit storage formats.
struct bf16_t {
    uint16_t bits;
};
struct f16_t {
    uint16_t bits;
};

// ------------------------------------------------------------------ scalar conversions
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float((uint32_t)x.bits << 16); }
__device__ __forceinline__ float to_f32(f16_t x) {
    return (float)__builtin_bit_cast(_Float16, x.bits);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) {
    return x;
}
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
    // v_cvt_pk_bf16_f32 rounds to nearest even.
    f32x2 v = {x, 0.0f};
    bf16x2 h = __builtin_convertvector(v, bf16x2);
    bf16_t r;
    r.bits = __builtin_bit_cast(uint32_t, h) & 0xffffu;
    return r;
}
template <>
__device__ __forceinline__ f16_t from_f32<f16_t>(float x) {
    f16_t r;
    r.bits = __builtin_bit_cast(uint16_t, (_Float16)x);
    return r;
}

// Two floats -> one dword of two 16-bit values (lo = a, hi = b), round to nearest even.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<bf16_t>(float a, float b) {
    f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
template <>
__device__ __forceinline__ uint32_t pack2<f16_t>(float a, float b) {
    f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// The low / high 16-bit element of a dword, widened to fp32.
template <typename T>
__device__ __forceinline__ float lo_f32(uint32_t w);
template <typename T>
__device__ __forceinline__ float hi_f32(uint32_t w);
template <>
__device__ __forceinline__ float lo_f32<bf16_t>(uint32_t w) {
    return __uint_as_float(w << 16);
}
template <>
__device__ __forceinline__ float hi_f32<bf16_t>(uint32_t w) {
    return __uint_as_float(w & 0xffff0000u);
}
template <>
__device__ __forceinline__ float lo_f32<f16_t>(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
template <>
__device__ __forceinline__ float hi_f32<f16_t>(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// ------------------------------------------------------------------ MFMA wrappers
// 16x16x32 (A: 16 x 32, B: 32 x 16, 8 elements per lane), fp32 accumulate.
template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<bf16_t>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<f16_t>(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
// 16x16x16 (4 elements per lane).
template <typename T>
__device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma16x16x16<bf16_t>(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, a),
                                                     __builtin_bit_cast(bf16x4, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16x16x16<f16_t>(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}
// 32x32x16 (A: 32 x 16, B: 16 x 32, 8 elements per lane), 16 fp32 per lane.
template <typename T>
__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c);
template <>
__device__ __forceinline__ f32x16 mfma32x32x16<bf16_t>(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32x32x16<f16_t>(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// ------------------------------------------------------------------ buffer loads
// Dword 3 of a raw buffer resource (untyped 32-bit data format) and the cache-policy bits of
// a non-temporal load.
static constexpr int BUF_DWORD3 = 0x00020000;
static constexpr int BUF_NT = 2;

// ------------------------------------------------------------------ misc device helpers
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// dword v_perm_b32 select: bytes 0-3 come from `lo_src`, 4-7 from `hi_src`.
__device__ __forceinline__ uint32_t perm_lo16(uint32_t lo_src, uint32_t hi_src) {
    // result = (hi_src.lo16 << 16) | lo_src.lo16
    return __builtin_amdgcn_perm(hi_src, lo_src, 0x05040100u);
}
__device__ __forceinline__ uint32_t perm_hi16(uint32_t lo_src, uint32_t hi_src) {
    // result = (hi_src.hi16 << 16) | lo_src.hi16
    return __builtin_amdgcn_perm(hi_src, lo_src, 0x07060302u);
}

// IEEE maximum (NaN-propagating): lowers to v_maximum3_f32 chains with no canonicalising moves,
// unlike fmaxf, whose NaN-quieting rule costs one extra instruction per MFMA-produced operand.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// max(x, x of lane l^32): one row-swap (VALU) instead of an LDS permute.
__device__ __forceinline__ float max_across_halves(float x) {
    const uint32_t u = __float_as_uint(x);
    auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return vmax(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float wave_shfl_xor(float x, int mask) {
    return __shfl_xor(x, mask, 64);
}

// Inclusive prefix sum over the 64 lanes of a wave without the LDS crossbar: a scan within each
// 16-lane row from DPP row shifts (lanes shifted in from outside the row read 0), then each row
// adds the totals of the rows before it (lanes 15, 31, 47, read into scalars).
__device__ __forceinline__ int wave_incl_sum(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(x, 15);
    const int r1 = __builtin_amdgcn_readlane(x, 31);
    const int r2 = __builtin_amdgcn_readlane(x, 47);
    const int row = (int)(__lane_id() >> 4);
    return x + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// Reductions over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48) with the gfx950
// row-swap instructions (plain VALU ops, no LDS crossbar): permlane16_swap pairs lane l with
// l^16, permlane32_swap pairs l with l^32.
__device__ __forceinline__ float max_across_rows(float x) {
    const uint32_t u = __float_as_uint(x);
    auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const uint32_t v = __float_as_uint(x);
    auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_across_rows(float x) {
    const uint32_t u = __float_as_uint(x);
    auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const uint32_t v = __float_as_uint(x);
    auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
// Sum over all 64 lanes, in every lane: DPP row rotations by 8, 4, 2, 1 sum each 16-lane row,
// then the rows are summed with the row swaps.
__device__ __forceinline__ float wave_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xf, 0xf, false));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf, false));
    return sum_across_rows(x);
}
// Maximum over all 64 lanes (fmaxf: a NaN lane is ignored), in every lane, the same way.
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xf, 0xf, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf, false)));
    return max_across_rows(x);
}
// x + x of lane l^32 with one row swap (VALU) instead of an LDS permute.
__device__ __forceinline__ float sum_across_halves(float x) {
    const uint32_t u = __float_as_uint(x);
    auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// ------------------------------------------------------------------ host-side error state
// Both are noexcept: the message lives in a fixed per-thread buffer.
void set_error(const char* fmt, ...) noexcept __attribute__((format(printf, 1, 2)));
void clear_error() noexcept;

// Runs the body of a C entry point so that no C++ exception crosses the C ABI (the caller may
// be C, ctypes or another language's FFI): a failed host allocation in a container or `new`
// becomes FLOUR_ERR_CAPACITY with a message, any other exception FLOUR_ERR_INVALID_ARGUMENT.
template <typename F>
int abi_guard(const char* what, F&& body) noexcept {
    try {
        return body();
    } catch (const std::bad_alloc&) {
        set_error("%s: out of host memory", what);
        return FLOUR_ERR_CAPACITY;
    } catch (const std::exception& e) {
        set_error("%s: %s", what, e.what());
        return FLOUR_ERR_INVALID_ARGUMENT;
    } catch (...) {
        set_error("%s: unexpected exception", what);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
}

inline int elem_bytes(int dtype) { return dtype == FLOUR_DTYPE_F32 ? 4 : 2; }
inline bool valid_dtype(int dtype) {
    return dtype == FLOUR_DTYPE_F32 || dtype == FLOUR_DTYPE_BF16 || dtype == FLOUR_DTYPE_F16;
}

// Check a HIP launch/runtime status; record an error and return FLOUR_ERR_HIP on failure.
int check_hip(hipError_t e, const char* what);

// Library-internal launchers with per-sequence row indices, for a mixed continuous-batching
// step (kv_batch.cpp): its one-row sequences run as one paged-decode batch whose entry b reads
// and writes packed row rows[b], and its longer sequences as one varlen prefill whose sequence
// s starts at packed row q_rows[s]. Both need the matrix-core path and return
// FLOUR_ERR_UNSUPPORTED before any launch otherwise.
// Whether the matrix-core decode / prefill kernels take a shape (alignment of q / out / strides
// aside for prefill, which the entry point checks with the pointers).
bool decode_mfma_supported(int dtype, int head_dim, int block_size, int n_rep, int batch,
                           int num_heads, int64_t num_slots, const void* q, const void* k_pool,
                           const void* v_pool);
bool prefill_mfma_supported(int dtype, int head_dim, int block_size, int64_t num_slots,
                            float scale, int64_t q_stride_tok);
int paged_decode_rows(void* out, int out_dtype, const void* q, const void* k_pool,
                      const void* v_pool, const int32_t* block_tables, int max_blocks_per_seq,
                      const int32_t* context_lens, const int32_t* rows, int batch, int num_heads,
                      int kv_heads, int head_dim, int block_size, int64_t num_slots,
                      int max_context_len, float scale, int dtype, void* workspace,
                      size_t workspace_bytes, void* stream);
// Decode step of a batch (one new row per sequence) with the step's KV write fused into the
// decode launch (kv_batch.cpp): the new K / V row of entry b and kv head g, at k_new / v_new +
// b * new_stride_tok + g * new_stride_head elements, goes to pool slot new_slots[b] (none outside
// [0, num_slots)) and is attended as position context_lens[b] - 1. The result equals
// flour_hip_kv_write followed by flour_hip_paged_decode when every new_slots[b] is the block
// table's slot of position context_lens[b] - 1 and no other entry's blocks hold it.
// FLOUR_ERR_UNSUPPORTED before any launch when the matrix-core decode does not take the shape,
// the pages are not 16 tokens, or the new rows are not aligned to a lane's share of a row (16
// bytes at head_dim 128, 8 at 64).
int paged_decode_write_kv(void* out, int out_dtype, const void* q, void* k_pool, void* v_pool,
                          const int32_t* block_tables, int max_blocks_per_seq,
                          const int32_t* context_lens, int batch, int num_heads, int kv_heads,
                          int head_dim, int block_size, int64_t num_slots, int max_context_len,
                          float scale, int dtype, void* workspace, size_t workspace_bytes,
                          const void* k_new, const void* v_new, int64_t new_stride_tok,
                          int64_t new_stride_head, const int32_t* new_slots, void* stream);
int varlen_prefill_rows(void* out, int out_dtype, int64_t o_stride_tok, int64_t o_stride_head,
                        const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                        const void* k_pool, const void* v_pool, const int32_t* cu_seqlens_q,
                        const int32_t* q_rows, const int32_t* kv_lens,
                        const int32_t* block_tables, int max_blocks_per_seq, int num_seqs,
                        int max_seqlen_q, int total_q, int num_heads, int kv_heads, int head_dim,
                        int block_size, int64_t num_slots, float scale, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream);

}  // namespace flour
