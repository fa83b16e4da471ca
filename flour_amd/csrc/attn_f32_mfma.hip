// attn_f32_mfma.hip — causal varlen prefill over fp32 pools on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32), head_dim 64 or 128. fp32 is the reference's model dtype when
// config.json names none (src/engine.rs:32-38); the arithmetic stays fp32 end to end: fp32
// products and sums in the matrix cores, fp32 softmax state.
//
// Semantics follow paged_attention (src/backend/cpu.rs:57-112): query row i of a sequence with
// q_len rows and kv_len cached positions sees kv position j iff j <= kv_len - q_len + i
// (cpu.rs:68, :88-95); query head h reads kv head h / n_rep (repeat_kv, cpu.rs:5-13); scores
// are q.k * scale; the softmax is folded online with a running max, sum and rescaled
// accumulator (cpu.rs:96-105); out = acc / sum (cpu.rs:111). A sequence with kv_len < q_len
// reads nothing and writes zero rows, as the other paths of this library do.
//
// Work: one workgroup per (query head, sequence, tile of 32 query rows), tiles of the highest
// index first (they read the longest kv ranges). Its W waves split the tile's causal kv range
// in steps of 32 positions (wave w takes steps w, w + W, ...) and fold their partial states
// together at the end through LDS, by log-sum-exp.
//
// Per step, with lane l holding query row r = l % 32 and half h = l / 32:
//  * S^T = K Q^T (32 positions x 32 rows) over D/2 products of k = 2: product s pairs head-dim
//    element D/2 h + s of the position (A, lane l: position l % 32) and of the row (B, lane l:
//    row l % 32), so each lane reads one contiguous half-row of K and of Q.
//  * The result leaves lane l with the scores of row r at positions 8 (e / 4) + 4 h + e % 4,
//    e = 0 .. 15: the row's max and sum need only the partner lane l ^ 32.
//  * O^T += V^T P^T over 16 products of k = 2, one per score register: product s takes the
//    lane's own score s as its B operand (position 8 (s / 4) + 4 h + s % 4, row r), and V at
//    that position as A, at head-dim element D/32 c + t of output tile t for lane row c = l % 32.
//    Each lane so reads D/32 contiguous elements of one V row per product; the positions' pool
//    slots come from the lanes that hold them for K (lane shuffles, no second table walk).
#include <math.h>

#include "flour_common.h"

namespace flour {

static constexpr int F32M_QT = 32;  // query rows per workgroup
static constexpr int F32M_KT = 32;  // kv positions per step
// Waves per workgroup: at head_dim 64 a wave holds 128 registers (two per SIMD, and two
// workgroups per CU); at 128 it holds 256, one per SIMD (8 waves of ~200 registers measured
// slower).
__host__ __device__ constexpr int f32m_waves(int d) { return d == 64 ? 8 : 4; }

__device__ __forceinline__ f32x16 mfma32x32x2_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Stores N consecutive outputs (N = 2 or 4) from fp32.
template <int N>
__device__ __forceinline__ void store_run(void* out, int out_dtype, int64_t idx, const float* v) {
    if (out_dtype == FLOUR_DTYPE_F32) {
        if constexpr (N == 4)
            *reinterpret_cast<f32x4*>(static_cast<float*>(out) + idx) = f32x4{v[0], v[1], v[2], v[3]};
        else
            *reinterpret_cast<f32x2*>(static_cast<float*>(out) + idx) = f32x2{v[0], v[1]};
    } else if (out_dtype == FLOUR_DTYPE_BF16) {
        if constexpr (N == 4)
            *reinterpret_cast<u32x2*>(static_cast<bf16_t*>(out) + idx) =
                u32x2{pack2<bf16_t>(v[0], v[1]), pack2<bf16_t>(v[2], v[3])};
        else
            *reinterpret_cast<uint32_t*>(static_cast<bf16_t*>(out) + idx) = pack2<bf16_t>(v[0], v[1]);
    } else {
        if constexpr (N == 4)
            *reinterpret_cast<u32x2*>(static_cast<f16_t*>(out) + idx) =
                u32x2{pack2<f16_t>(v[0], v[1]), pack2<f16_t>(v[2], v[3])};
        else
            *reinterpret_cast<uint32_t*>(static_cast<f16_t*>(out) + idx) = pack2<f16_t>(v[0], v[1]);
    }
}

template <int D>
__global__ __launch_bounds__(f32m_waves(D) * 64) void prefill_f32_mfma_kernel(
    void* __restrict__ out, int out_dtype, int64_t o_st, int64_t o_sh,
    const float* __restrict__ q, int64_t q_st, int64_t q_sh, const float* __restrict__ k_pool,
    const float* __restrict__ v_pool, const int32_t* __restrict__ cu_seqlens_q,
    const int32_t* __restrict__ q_rows, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ block_tables, int max_blocks, int n_rep, int block_size,
    int num_slots, int n_qt, float scale_log2) {
    constexpr int W = f32m_waves(D);
    constexpr int DH = D / 2;   // products of S^T per step
    constexpr int DT = D / 32;  // 32-row tiles of O^T
    constexpr int NS = 16 * DT + 2;  // a lane's state: O^T registers, max, sum
    // partial states of the upper half of the waves still merging, [wave][value][lane]
    __shared__ float red[(W / 2) * NS * 64];

    const int head = blockIdx.x, s = blockIdx.y, qt = n_qt - 1 - (int)blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int r = lane & 31, h = lane >> 5;
    const int c0 = cu_seqlens_q[s];
    const int q_len = cu_seqlens_q[s + 1] - c0;
    if (qt * F32M_QT >= q_len) return;  // uniform: no such tile in this sequence
    const int row0 = q_rows ? q_rows[s] : c0;  // the sequence's first packed row
    const int kv_len = min(kv_lens[s], max_blocks * block_size);
    const int off = kv_len - q_len;  // row i sees positions j <= off + i
    const int i = qt * F32M_QT + r;  // this lane's row in the sequence
    const int last = min(qt * F32M_QT + F32M_QT, q_len) - 1;
    const int kv_end = kv_len >= q_len ? off + last + 1 : 0;  // positions the tile reads
    const int lim = (i < q_len && kv_len >= q_len) ? off + i : -1;
    const int kvh = head / n_rep;
    const int32_t* bt = block_tables + (int64_t)s * max_blocks;
    const int max_phys = num_slots / block_size - 1;
    const float* kbase = k_pool + (int64_t)kvh * num_slots * D;
    const float* vbase = v_pool + (int64_t)kvh * num_slots * D;

    // this lane's half-row of Q (rows past the sequence read its last row; they are masked),
    // pre-scaled into the exp2 domain
    float qv[DH];
    {
        const float* qp = q + (int64_t)(row0 + min(i, q_len - 1)) * q_st + (int64_t)head * q_sh + DH * h;
#pragma unroll
        for (int x = 0; x < DH / 4; x++) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(qp + 4 * x);
#pragma unroll
            for (int e = 0; e < 4; e++) qv[4 * x + e] = v[e] * scale_log2;
        }
    }

    float m = -INFINITY, l = 0.0f;
    f32x16 o[DT];
#pragma unroll
    for (int t = 0; t < DT; t++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[t][e] = 0.0f;

    const int n_st = (kv_end + F32M_KT - 1) / F32M_KT;
    for (int st = w; st < n_st; st += W) {
        const int kv0 = st * F32M_KT;
        // pool slot of position kv0 + r (row 0 past the tile's range: those scores are masked);
        // a block id outside the pool is clamped into it
        int slot = 0;
        {
            const int j = kv0 + r;
            if (j < kv_end) {
                const int lb = j / block_size;
                const int id = bt[lb];
                const int phys = id < 0 ? 0 : (id > max_phys ? max_phys : id);
                slot = phys * block_size + (j - lb * block_size);
            }
        }
        float kx[DH];
        {
            const float* kp = kbase + (int64_t)slot * D + DH * h;
#pragma unroll
            for (int x = 0; x < DH / 4; x++) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(kp + 4 * x);
#pragma unroll
                for (int e = 0; e < 4; e++) kx[4 * x + e] = v[e];
            }
        }
        // V at the positions of this lane's scores; the slot of position 8 (e/4) + 4h + e%4 is
        // held by that lane
        float vx[16][DT];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int src = 8 * (e >> 2) + 4 * h + (e & 3);
            const int sl = __shfl(slot, src, 64);
            const float* vp = vbase + (int64_t)sl * D + DT * r;
            if constexpr (DT == 4) {
                const f32x4 v = *reinterpret_cast<const f32x4*>(vp);
#pragma unroll
                for (int t = 0; t < 4; t++) vx[e][t] = v[t];
            } else {
                const f32x2 v = *reinterpret_cast<const f32x2*>(vp);
                vx[e][0] = v[0];
                vx[e][1] = v[1];
            }
        }
        // S^T = K Q^T
        f32x16 sc;
#pragma unroll
        for (int e = 0; e < 16; e++) sc[e] = 0.0f;
#pragma unroll
        for (int x = 0; x < DH; x++) sc = mfma32x32x2_f32(kx[x], qv[x], sc);
        // causal mask and the row's max (lanes l and l ^ 32 hold the same row)
        float tm = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int j = kv0 + 8 * (e >> 2) + 4 * h + (e & 3);
            if (j > lim) sc[e] = -INFINITY;
            tm = fmaxf(tm, sc[e]);
        }
        tm = max_across_halves(tm);
        const float m_new = fmaxf(m, tm);
        const float mu = m_new == -INFINITY ? 0.0f : m_new;  // nothing visible yet: all p = 0
        const float alpha = fast_exp2(m - mu);
        m = m_new;
        float p[16], ps = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            p[e] = fast_exp2(sc[e] - mu);
            ps += p[e];
        }
        l = l * alpha + ps;
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int e = 0; e < 16; e++) o[t][e] *= alpha;
        // O^T += V^T P^T
#pragma unroll
        for (int e = 0; e < 16; e++)
#pragma unroll
            for (int t = 0; t < DT; t++) o[t] = mfma32x32x2_f32(vx[e][t], p[e], o[t]);
    }
    l = sum_across_halves(l);  // the row's sum over both halves of its positions

    // fold the waves' states pairwise: the upper half writes, the lower half merges
#pragma unroll
    for (int half = W / 2; half >= 1; half >>= 1) {
        if (w >= half && w < 2 * half) {
            float* dst = red + (w - half) * NS * 64 + lane;
#pragma unroll
            for (int t = 0; t < DT; t++)
#pragma unroll
                for (int e = 0; e < 16; e++) dst[(16 * t + e) * 64] = o[t][e];
            dst[16 * DT * 64] = m;
            dst[(16 * DT + 1) * 64] = l;
        }
        __syncthreads();
        if (w < half) {
            const float* src = red + w * NS * 64 + lane;
            const float mb = src[16 * DT * 64], lb = src[(16 * DT + 1) * 64];
            const float mm = fmaxf(m, mb);
            const float mz = mm == -INFINITY ? 0.0f : mm;
            const float fa = fast_exp2(m - mz), fb = fast_exp2(mb - mz);
            l = l * fa + lb * fb;
            m = mm;
#pragma unroll
            for (int t = 0; t < DT; t++)
#pragma unroll
                for (int e = 0; e < 16; e++) o[t][e] = o[t][e] * fa + src[(16 * t + e) * 64] * fb;
        }
        if (half > 1) __syncthreads();
    }
    if (w != 0 || i >= q_len) return;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;  // no visible position: a zero row
    const int64_t obase = (int64_t)(row0 + i) * o_st + (int64_t)head * o_sh;
#pragma unroll
    for (int e = 0; e < 16; e++) {
        float v[DT];
#pragma unroll
        for (int t = 0; t < DT; t++) v[t] = o[t][e] * inv;
        store_run<DT>(out, out_dtype, obase + DT * (8 * (e >> 2) + 4 * h + (e & 3)), v);
    }
}

static int g_prefill_f32_mfma = 1;  // a test / tuning switch

bool prefill_f32_mfma_supported(int dtype, int head_dim, int num_seqs, int max_seqlen_q,
                                int block_size, int64_t num_slots) {
    const int64_t n_qt = ((int64_t)max_seqlen_q + F32M_QT - 1) / F32M_QT;
    return g_prefill_f32_mfma && dtype == FLOUR_DTYPE_F32 && (head_dim == 64 || head_dim == 128) &&
           num_seqs <= 65535 && n_qt <= 65535 && block_size > 0 && num_slots <= 0x7fffffff &&
           num_slots % block_size == 0;
}

// The caller checks prefill_f32_mfma_supported, the 16-byte alignment of q, the pools and out
// and of their row and head strides.
int launch_prefill_f32_mfma(int out_dtype, void* out, int64_t o_st, int64_t o_sh, const void* q,
                            int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool,
                            const int32_t* cu_seqlens_q, const int32_t* q_rows,
                            const int32_t* kv_lens, const int32_t* block_tables, int max_blocks,
                            int num_seqs, int max_seqlen_q, int num_heads, int n_rep,
                            int head_dim, int block_size, int64_t num_slots, float scale,
                            hipStream_t stream) {
    const int n_qt = (max_seqlen_q + F32M_QT - 1) / F32M_QT;
    if (n_qt == 0 || num_seqs == 0) return FLOUR_OK;
    const dim3 grid((unsigned)num_heads, (unsigned)num_seqs, (unsigned)n_qt);
    const float sl2 = scale * 1.4426950408889634f;
#define FLOUR_F32M(D)                                                                            \
    prefill_f32_mfma_kernel<D><<<grid, dim3(f32m_waves(D) * 64), 0, stream>>>(                   \
        out, out_dtype, o_st, o_sh, static_cast<const float*>(q), q_st, q_sh,                    \
        static_cast<const float*>(k_pool), static_cast<const float*>(v_pool), cu_seqlens_q,      \
        q_rows, kv_lens, block_tables, max_blocks, n_rep, block_size, (int)num_slots, n_qt, sl2)
    if (head_dim == 64)
        FLOUR_F32M(64);
    else
        FLOUR_F32M(128);
#undef FLOUR_F32M
    return check_hip(hipGetLastError(), "varlen_prefill (fp32 matrix cores) launch");
}

}  // namespace flour

using namespace flour;

// 1 (the default): fp32 prefill at head_dim 64 / 128 on the fp32 matrix cores; 0: on the vector
// kernel. A test / tuning switch.
extern "C" int flour_hip_set_prefill_f32_mfma(int on) {
    g_prefill_f32_mfma = on ? 1 : 0;
    return FLOUR_OK;
}
