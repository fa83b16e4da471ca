// attn_generic.hip — paged attention for any head_dim <= 512, block size and GQA ratio, in
// fp32 / bf16 / f16 storage. It serves the shapes the MFMA kernels do not (fp32 pools,
// head_dim != 128, block sizes that are not a multiple of 16), e.g. the fp32 decode
// configuration (head_dim 64) and the tiny shapes of the reference's own tests.
//
// Semantics follow paged_attention (src/backend/cpu.rs:57-112): query row i of a sequence
// with q_len rows and kv_len cached positions sees kv position j iff j <= kv_len - q_len + i
// (cpu.rs:68, :88-95), query head h reads kv head h / n_rep (repeat_kv, cpu.rs:5-13), scores
// are q.k * scale in fp32, the softmax is folded online over chunks with the running max /
// running sum / rescaled accumulator of cpu.rs:96-105, and out = acc / sum (cpu.rs:111).
//
// Layout of work: one 256-lane workgroup per (query row, head). Each chunk of 256 kv
// positions gives one score per lane; the workgroup reduces max and sum in LDS, then each lane
// owns output dims d = lane, lane + 256 and folds p_j * v[j][d] over the chunk.
#include <math.h>

#include "flour_common.h"

namespace flour {

static constexpr int GEN_THREADS = 256;

__device__ __forceinline__ float block_reduce_max(float x, float* red) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = x;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < GEN_THREADS / 64; i++) r = fmaxf(r, red[i]);
    return r;
}

__device__ __forceinline__ float block_reduce_sum(float x, float* red) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = x;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < GEN_THREADS / 64; i++) r += red[i];
    return r;
}

template <typename TQ, typename TKV, typename TO>
__global__ __launch_bounds__(GEN_THREADS) void attn_generic_kernel(
    TO* __restrict__ out, int64_t o_st, int64_t o_sh, const TQ* __restrict__ q, int64_t q_st,
    int64_t q_sh, const TKV* __restrict__ k_pool, const TKV* __restrict__ v_pool,
    const int32_t* __restrict__ cu_seqlens_q, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ block_tables, int max_blocks, int num_seqs, int n_rep,
    int head_dim, int block_size, int64_t num_slots, int max_kv, float scale) {
    __shared__ float qs[512];
    __shared__ float ps[GEN_THREADS];
    __shared__ int64_t rows[GEN_THREADS];
    __shared__ float red[GEN_THREADS / 64];

    const int64_t r = blockIdx.x;  // packed query row
    const int h = blockIdx.y;
    const int tid = threadIdx.x;

    // Sequence of this row: cu_seqlens_q == nullptr means one query row per sequence.
    int s, i, q_len;
    if (cu_seqlens_q) {
        int lo = 0, hi = num_seqs;  // find s with cu[s] <= r < cu[s+1]
        while (hi - lo > 1) {
            int mid = (lo + hi) >> 1;
            if (cu_seqlens_q[mid] <= r)
                lo = mid;
            else
                hi = mid;
        }
        s = lo;
        i = (int)(r - cu_seqlens_q[s]);
        q_len = cu_seqlens_q[s + 1] - cu_seqlens_q[s];
    } else {
        s = (int)r;
        i = 0;
        q_len = 1;
    }
    // never read past the table; decode also clamps to max_context_len, as the MFMA path does
    const int kv_len = min(min(kv_lens[s], max_blocks * block_size), max_kv);
    const int64_t n_vis = (kv_len >= q_len) ? (int64_t)kv_len - q_len + i + 1 : 0;
    const int kvh = h / n_rep;
    const int32_t* bt = block_tables + (int64_t)s * max_blocks;

    for (int d = tid; d < head_dim; d += GEN_THREADS) qs[d] = to_f32(q[r * q_st + h * q_sh + d]);
    __syncthreads();

    float m = -INFINITY, l = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
    const int64_t head_base = (int64_t)kvh * num_slots;
    const int64_t max_phys = num_slots / block_size - 1;
    for (int64_t c0 = 0; c0 < n_vis; c0 += GEN_THREADS) {
        const int64_t j = c0 + tid;
        float sc = -INFINITY;
        int64_t row = 0;
        if (j < n_vis) {
            const int64_t lb = j / block_size;
            int64_t phys = bt[lb];  // clamped: a bad block id never leaves the pool
            phys = phys < 0 ? 0 : (phys > max_phys ? max_phys : phys);
            row = (head_base + phys * block_size + (j - lb * block_size)) * head_dim;
            float dot = 0.0f;
            for (int d = 0; d < head_dim; d++) dot = fmaf(qs[d], to_f32(k_pool[row + d]), dot);
            sc = dot * scale;
        }
        rows[tid] = row;
        const float cmax = block_reduce_max(sc, red);
        const float m_new = fmaxf(m, cmax);
        const float corr = (m == -INFINITY) ? 0.0f : expf(m - m_new);
        const float p = (j < n_vis) ? expf(sc - m_new) : 0.0f;
        ps[tid] = p;
        const float psum = block_reduce_sum(p, red);  // its barriers also publish ps / rows
        l = l * corr + psum;
        const int nj = (n_vis - c0) < GEN_THREADS ? (int)(n_vis - c0) : GEN_THREADS;
        if (tid < head_dim) {
            float pv = 0.0f;
            for (int jj = 0; jj < nj; jj++) pv = fmaf(ps[jj], to_f32(v_pool[rows[jj] + tid]), pv);
            acc0 = acc0 * corr + pv;
        }
        if (tid + GEN_THREADS < head_dim) {
            float pv = 0.0f;
            for (int jj = 0; jj < nj; jj++)
                pv = fmaf(ps[jj], to_f32(v_pool[rows[jj] + tid + GEN_THREADS]), pv);
            acc1 = acc1 * corr + pv;
        }
        m = m_new;
        __syncthreads();  // ps / rows are rewritten by the next chunk
    }
    const float inv = (l > 0.0f) ? 1.0f / l : 0.0f;
    if (tid < head_dim) out[r * o_st + h * o_sh + tid] = from_f32<TO>(acc0 * inv);
    if (tid + GEN_THREADS < head_dim)
        out[r * o_st + h * o_sh + tid + GEN_THREADS] = from_f32<TO>(acc1 * inv);
}

template <typename TQ, typename TKV, typename TO>
static void launch_generic_t(void* out, int64_t o_st, int64_t o_sh, const void* q, int64_t q_st,
                             int64_t q_sh, const void* k_pool, const void* v_pool,
                             const int32_t* cu, const int32_t* kv_lens, const int32_t* bt,
                             int max_blocks, int num_seqs, int total_q, int num_heads, int n_rep,
                             int head_dim, int block_size, int64_t num_slots, int max_kv,
                             float scale, hipStream_t stream) {
    attn_generic_kernel<TQ, TKV, TO><<<dim3(total_q, num_heads), dim3(GEN_THREADS), 0, stream>>>(
        static_cast<TO*>(out), o_st, o_sh, static_cast<const TQ*>(q), q_st, q_sh,
        static_cast<const TKV*>(k_pool), static_cast<const TKV*>(v_pool), cu, kv_lens, bt,
        max_blocks, num_seqs, n_rep, head_dim, block_size, num_slots, max_kv, scale);
}

template <typename T>
static void launch_generic_in(int out_dtype, void* out, int64_t o_st, int64_t o_sh,
                              const void* q, int64_t q_st, int64_t q_sh, const void* k_pool,
                              const void* v_pool, const int32_t* cu, const int32_t* kv_lens,
                              const int32_t* bt, int max_blocks, int num_seqs, int total_q,
                              int num_heads, int n_rep, int head_dim, int block_size,
                              int64_t num_slots, int max_kv, float scale, hipStream_t stream) {
    if (out_dtype == FLOUR_DTYPE_F32)
        launch_generic_t<T, T, float>(out, o_st, o_sh, q, q_st, q_sh, k_pool, v_pool, cu, kv_lens,
                                      bt, max_blocks, num_seqs, total_q, num_heads, n_rep,
                                      head_dim, block_size, num_slots, max_kv, scale, stream);
    else if (out_dtype == FLOUR_DTYPE_BF16)
        launch_generic_t<T, T, bf16_t>(out, o_st, o_sh, q, q_st, q_sh, k_pool, v_pool, cu,
                                       kv_lens, bt, max_blocks, num_seqs, total_q, num_heads,
                                       n_rep, head_dim, block_size, num_slots, max_kv, scale, stream);
    else
        launch_generic_t<T, T, f16_t>(out, o_st, o_sh, q, q_st, q_sh, k_pool, v_pool, cu, kv_lens,
                                      bt, max_blocks, num_seqs, total_q, num_heads, n_rep,
                                      head_dim, block_size, num_slots, max_kv, scale, stream);
}

// Launch the generic kernel; dtype is the storage type of q and the pools.
int launch_attn_generic(int dtype, int out_dtype, void* out, int64_t o_st, int64_t o_sh,
                        const void* q, int64_t q_st, int64_t q_sh, const void* k_pool,
                        const void* v_pool, const int32_t* cu, const int32_t* kv_lens,
                        const int32_t* bt, int max_blocks, int num_seqs, int total_q,
                        int num_heads, int n_rep, int head_dim, int block_size, int64_t num_slots,
                        int max_kv, float scale, hipStream_t stream) {
    if (head_dim > 512) {
        set_error("attention: head_dim %d > 512 is not supported", head_dim);
        return FLOUR_ERR_UNSUPPORTED;
    }
    if (total_q == 0) return FLOUR_OK;
    if (num_heads > 65535) {
        set_error("attention: num_heads %d too large", num_heads);
        return FLOUR_ERR_UNSUPPORTED;
    }
    if (dtype == FLOUR_DTYPE_F32)
        launch_generic_in<float>(out_dtype, out, o_st, o_sh, q, q_st, q_sh, k_pool, v_pool, cu,
                                 kv_lens, bt, max_blocks, num_seqs, total_q, num_heads, n_rep,
                                 head_dim, block_size, num_slots, max_kv, scale, stream);
    else if (dtype == FLOUR_DTYPE_BF16)
        launch_generic_in<bf16_t>(out_dtype, out, o_st, o_sh, q, q_st, q_sh, k_pool, v_pool, cu,
                                  kv_lens, bt, max_blocks, num_seqs, total_q, num_heads, n_rep,
                                  head_dim, block_size, num_slots, max_kv, scale, stream);
    else
        launch_generic_in<f16_t>(out_dtype, out, o_st, o_sh, q, q_st, q_sh, k_pool, v_pool, cu,
                                 kv_lens, bt, max_blocks, num_seqs, total_q, num_heads, n_rep,
                                 head_dim, block_size, num_slots, max_kv, scale, stream);
    return check_hip(hipGetLastError(), "attention (generic) launch");
}

}  // namespace flour
