// attn_simt.hip — paged attention on the vector ALUs for the shapes the matrix-core kernels do
// not take: fp32 pools (the reference's dtype when config.json names none, engine.rs:32-38),
// head dims other than 128 (64 for Qwen2.5-0.5B-sized models) and page sizes that are not a
// multiple of 16. Decode (seq_q == 1) and causal varlen prefill share the kernel.
//
// Semantics follow paged_attention (src/backend/cpu.rs:57-112): query row i of a sequence with
// q_len rows and kv_len cached positions sees kv position j iff j <= kv_len - q_len + i
// (cpu.rs:68, :88-95); query head h reads kv head h / n_rep (repeat_kv, cpu.rs:5-13); scores
// are q.k * scale in fp32; the softmax is folded online with the running max, running sum and
// rescaled accumulator of cpu.rs:96-105; out = acc / sum (cpu.rs:111).
//
// Work decomposition: a workgroup of four waves owns one kv head of one sequence and up to
// SIMT_NQ queries that read it: the query heads of the kv head (GQA: each K/V row is loaded
// once for all of them) and, in prefill, as many consecutive query rows as fit. Every K and V
// row is read with 16-byte loads: a row of D elements spans LPR = D * sizeof(T) / 16 lanes, so
// one wave load covers 64 / LPR whole rows (coalesced runs of the (head, slot, dim) pool).
// Each lane group (the LPR lanes of one row) keeps its own running (max, sum, accumulator)
// per query over the rows it reads; the groups of a wave are merged with lane shuffles and the
// four waves through LDS, both by log-sum-exp.
#include <math.h>

#include <algorithm>

#include "flour_common.h"

namespace flour {

static constexpr int SIMT_MAX_WAVES = 16;  // waves per workgroup (split of the kv range)
// Waves per workgroup the register budget allows: the per-query state (query slice and
// accumulator, 2 x VEC per query) fits 128 VGPRs per lane for up to two queries (16 waves, four
// per SIMD), 256 otherwise (8 waves).
__host__ __device__ constexpr int simt_max_waves(int nq) { return nq <= 2 ? 16 : 8; }
static constexpr int SIMT_NQ_MAX = 8;      // queries (rows x heads) per workgroup
static constexpr int SIMT_UNROLL = 2;      // row loads per lane per chunk (two chunks in flight)
static constexpr int SIMT_MAX_D = 256;     // head_dim bound of the vector kernel

template <typename T>
struct Vec16;  // 16 bytes of T widened to fp32
template <>
struct Vec16<float> {
    static constexpr int N = 4;
    __device__ __forceinline__ static void widen(const u32x4& r, float* x) {
#pragma unroll
        for (int i = 0; i < 4; i++) x[i] = __uint_as_float(r[i]);
    }
};
template <>
struct Vec16<bf16_t> {
    static constexpr int N = 8;
    __device__ __forceinline__ static void widen(const u32x4& r, float* x) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[2 * i] = lo_f32<bf16_t>(r[i]);
            x[2 * i + 1] = hi_f32<bf16_t>(r[i]);
        }
    }
};
template <>
struct Vec16<f16_t> {
    static constexpr int N = 8;
    __device__ __forceinline__ static void widen(const u32x4& r, float* x) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            x[2 * i] = lo_f32<f16_t>(r[i]);
            x[2 * i + 1] = hi_f32<f16_t>(r[i]);
        }
    }
};

// Sum over the aligned group of `G` lanes holding one row (every lane receives the sum), with
// DPP lane moves inside 16-lane rows and row swaps beyond: xor 1 and xor 2 within quads, the
// mirrored half-row (lane i <-> 7 - i, quads already uniform), the mirrored row (i <-> 15 - i),
// then lanes l ^ 16 and l ^ 32.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                              0xf, 0xf, false));
}
template <int G>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (G >= 2) x += dpp_move<0xB1>(x);   // quad_perm [1, 0, 3, 2]
    if constexpr (G >= 4) x += dpp_move<0x4E>(x);   // quad_perm [2, 3, 0, 1]
    if constexpr (G >= 8) x += dpp_move<0x141>(x);  // row_half_mirror
    if constexpr (G >= 16) x += dpp_move<0x140>(x); // row_mirror
    if constexpr (G >= 32) {
        const uint32_t u = __float_as_uint(x);
        auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    }
    if constexpr (G >= 64) {
        const uint32_t u = __float_as_uint(x);
        auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        x = __uint_as_float(b[0]) + __uint_as_float(b[1]);
    }
    return x;
}

// Sum / maximum over the lanes that hold the same slice of a row (lanes li + LPR g, every
// lane receives the result): DPP rotations inside 16-lane rows by multiples of LPR, then the
// row swaps for lanes l ^ 16 and l ^ 32. No LDS crossbar.
template <int LPR, bool MAX>
__device__ __forceinline__ float across_groups(float x) {
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    if constexpr (LPR <= 8) x = op(x, dpp_move<0x128>(x));  // row_ror:8
    if constexpr (LPR <= 4) x = op(x, dpp_move<0x124>(x));  // row_ror:4
    if constexpr (LPR <= 2) x = op(x, dpp_move<0x122>(x));  // row_ror:2
    if constexpr (LPR <= 1) x = op(x, dpp_move<0x121>(x));  // row_ror:1
    if constexpr (LPR <= 16) {
        const uint32_t u = __float_as_uint(x);
        auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        x = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
    }
    if constexpr (LPR <= 32) {
        const uint32_t u = __float_as_uint(x);
        auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        x = op(__uint_as_float(b[0]), __uint_as_float(b[1]));
    }
    return x;
}

__device__ __forceinline__ void store_out(void* out, int out_dtype, int64_t idx, float v) {
    if (out_dtype == FLOUR_DTYPE_F32)
        static_cast<float*>(out)[idx] = v;
    else if (out_dtype == FLOUR_DTYPE_BF16)
        static_cast<bf16_t*>(out)[idx] = from_f32<bf16_t>(v);
    else
        static_cast<f16_t*>(out)[idx] = from_f32<f16_t>(v);
}

// One workgroup per (item, kv head, head group); its waves split the kv range. An item is one
// sequence of a decode batch (cu_seqlens_q == nullptr), or `rows` consecutive query rows of one
// prefill sequence: item x is the x-th row block in sequence order, found by scanning
// cu_seqlens_q. NQ (a power of two) bounds the queries of the workgroup: rows x heads of the
// group; the unused ones are masked.
template <typename T, int LPR, int NQ>
__global__ __launch_bounds__(simt_max_waves(NQ) * 64) void attn_simt_kernel(
    void* __restrict__ out, int out_dtype, int64_t o_st, int64_t o_sh, const T* __restrict__ q,
    int64_t q_st, int64_t q_sh, const T* __restrict__ k_pool, const T* __restrict__ v_pool,
    const int32_t* __restrict__ cu_seqlens_q, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ block_tables, int max_blocks, int num_seqs, int n_rep,
    int heads_per_group, int rows, int head_dim, int block_size, int64_t num_slots, int max_kv,
    float scale_log2) {
    constexpr int VEC = Vec16<T>::N;  // elements per lane per row
    constexpr int RPL = 64 / LPR;     // rows per wave load
    extern __shared__ float red[];    // [waves][NQ][2 + head_dim]: (max, sum, acc) per wave
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int waves = blockDim.x >> 6;
    const int grp = lane / LPR, li = lane % LPR;  // lane group (row of a load), lane in group
    const int kvh = blockIdx.y;
    const int h0 = kvh * n_rep + blockIdx.z * heads_per_group;  // first query head
    const int nh = min(heads_per_group, n_rep - blockIdx.z * heads_per_group);

    // ---- the item: sequence s, its first row r0 and row count nr
    int s = 0, r0 = 0, nr = 1, q_len = 1;
    if (cu_seqlens_q) {
        __shared__ int found[2];
        if (w == 0) {
            const int x = blockIdx.x;
            int base = 0, seq = -1, first = 0;
            for (int s0 = 0; s0 < num_seqs && seq < 0; s0 += 64) {
                const int sq = s0 + lane;
                const int n = sq < num_seqs ? (cu_seqlens_q[sq + 1] - cu_seqlens_q[sq] + rows - 1) / rows : 0;
                const int incl = wave_incl_sum(n);
                const int excl = base + incl - n;
                const uint64_t hit = __ballot(n > 0 && x >= excl && x < excl + n);
                if (hit) {
                    const int src = __ffsll((unsigned long long)hit) - 1;
                    seq = s0 + src;
                    first = __builtin_amdgcn_readlane(x - excl, src);
                }
                base += __builtin_amdgcn_readlane(incl, 63);
            }
            if (lane == 0) {
                found[0] = seq;
                found[1] = first;
            }
        }
        __syncthreads();
        s = found[0];
        if (s < 0) return;  // uniform: a block past the last one
        const int q0 = cu_seqlens_q[s];
        q_len = cu_seqlens_q[s + 1] - q0;
        r0 = q0 + found[1] * rows;
        nr = min(rows, q0 + q_len - r0);
    } else {
        s = blockIdx.x;
        r0 = s;
    }
    const int i0 = r0 - (cu_seqlens_q ? cu_seqlens_q[s] : s);  // row index in the sequence
    const int kv_len = min(min(kv_lens[s], max_blocks * block_size), max_kv);
    const int off = kv_len - q_len;  // row i sees kv j <= off + i (none when kv_len < q_len)
    const int nq = nr * nh;          // queries: (row rr, head hh) = (qi / nh, qi % nh)
    const int kv_end = kv_len >= q_len ? off + i0 + nr : 0;  // rows the block reads
    const int32_t* bt = block_tables + (int64_t)s * max_blocks;
    const int64_t max_phys = num_slots / block_size - 1;
    const T* kbase = k_pool + (int64_t)kvh * num_slots * head_dim + li * VEC;
    const T* vbase = v_pool + (int64_t)kvh * num_slots * head_dim + li * VEC;

    // this lane's slice of every query, pre-scaled into the exp2 domain
    float qv[NQ][VEC];
    int lim[NQ];  // causal limit of each query's row (-1: an unused query slot)
#pragma unroll
    for (int qi = 0; qi < NQ; qi++) {
        const int rr = min(qi / nh, nr - 1), hh = qi % nh;
        u32x4 raw = {0, 0, 0, 0};
        if (qi < nq)
            raw = *reinterpret_cast<const u32x4*>(q + (int64_t)(r0 + rr) * q_st + (int64_t)(h0 + hh) * q_sh + li * VEC);
        Vec16<T>::widen(raw, qv[qi]);
#pragma unroll
        for (int e = 0; e < VEC; e++) qv[qi][e] *= scale_log2;
        lim[qi] = qi < nq ? off + i0 + rr : -1;
    }
    float m[NQ], l[NQ], acc[NQ][VEC];
#pragma unroll
    for (int qi = 0; qi < NQ; qi++) {
        m[qi] = -INFINITY;
        l[qi] = 0.0f;
#pragma unroll
        for (int e = 0; e < VEC; e++) acc[qi][e] = 0.0f;
    }

    // ---- chunks of waves * RPL * SIMT_UNROLL rows: row j = c0 + (u * waves + w) * RPL + grp.
    // The next chunk's rows are loaded while this one is computed, and the block ids of the
    // chunk after it are fetched with those loads, so a chunk's K/V loads never wait for a
    // block-table read of their own. A block id is read whether or not its row is < kv_end
    // (the index is clamped into the table row), so that it does not wait for the kv length:
    // the first two chunks' K/V loads depend on one memory round trip (their block ids), not two.
    const int chunk = waves * RPL * SIMT_UNROLL;
    auto load_ids = [&](int c0, int* ids) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < SIMT_UNROLL; u++) {
            const int j = c0 + (u * waves + w) * RPL + grp;
            ids[u] = bt[min(j / block_size, max_blocks - 1)];
        }
    };
    auto load = [&](int c0, const int* ids, u32x4* kr, u32x4* vr, int* jr) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < SIMT_UNROLL; u++) {
            const int j = c0 + (u * waves + w) * RPL + grp;
            jr[u] = j;
            int64_t row = 0;  // rows past the end read row 0 of the pool (their scores are masked)
            if (j < kv_end) {
                const int lb = j / block_size;
                // clamped: a bad block id never leaves the pool
                const int64_t phys = ids[u] < 0 ? 0 : (ids[u] > max_phys ? max_phys : (int64_t)ids[u]);
                row = (phys * block_size + (j - lb * block_size)) * head_dim;
            }
            kr[u] = *reinterpret_cast<const u32x4*>(kbase + row);
            vr[u] = *reinterpret_cast<const u32x4*>(vbase + row);
        }
    };
    u32x4 ka[SIMT_UNROLL], va[SIMT_UNROLL], kb[SIMT_UNROLL], vb[SIMT_UNROLL];
    int ja[SIMT_UNROLL], jb[SIMT_UNROLL];
    auto compute = [&](const u32x4* kr, const u32x4* vr, const int* jr) __attribute__((always_inline)) {
        float sc[SIMT_UNROLL][NQ];
#pragma unroll
        for (int u = 0; u < SIMT_UNROLL; u++) {
            float kx[VEC];
            Vec16<T>::widen(kr[u], kx);
#pragma unroll
            for (int qi = 0; qi < NQ; qi++) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < VEC; e++) d = fmaf(qv[qi][e], kx[e], d);
                d = group_sum<LPR>(d);
                sc[u][qi] = jr[u] <= lim[qi] ? d : -INFINITY;  // causal limit / past the end
            }
        }
#pragma unroll
        for (int qi = 0; qi < NQ; qi++) {
            float cm = sc[0][qi];
#pragma unroll
            for (int u = 1; u < SIMT_UNROLL; u++) cm = fmaxf(cm, sc[u][qi]);
            const float m_new = fmaxf(m[qi], cm);
            if (m_new == -INFINITY) continue;  // nothing visible yet
            const float corr = exp2f(m[qi] - m_new);  // 0 for the first visible rows
            float p[SIMT_UNROLL], ps = 0.0f;
#pragma unroll
            for (int u = 0; u < SIMT_UNROLL; u++) {
                p[u] = exp2f(sc[u][qi] - m_new);
                ps += p[u];
            }
            l[qi] = l[qi] * corr + ps;
            m[qi] = m_new;
#pragma unroll
            for (int e = 0; e < VEC; e++) acc[qi][e] *= corr;
#pragma unroll
            for (int u = 0; u < SIMT_UNROLL; u++) {
                float vx[VEC];
                Vec16<T>::widen(vr[u], vx);
#pragma unroll
                for (int e = 0; e < VEC; e++) acc[qi][e] = fmaf(p[u], vx[e], acc[qi][e]);
            }
        }
    };
    // ids_a: block ids of the chunk that set A loads next, ids_b those of set B
    int ids_a[SIMT_UNROLL], ids_b[SIMT_UNROLL];
    load_ids(0, ids_a);  // unconditional, so that they need not wait for the kv length
    load_ids(chunk, ids_b);
    load(0, ids_a, ka, va, ja);
    for (int c0 = 0; c0 < kv_end; c0 += 2 * chunk) {
        const bool more = c0 + chunk < kv_end;
        if (more) {
            load(c0 + chunk, ids_b, kb, vb, jb);
            if (c0 + 2 * chunk < kv_end) load_ids(c0 + 2 * chunk, ids_a);
        }
        compute(ka, va, ja);
        if (!more) break;
        if (c0 + 2 * chunk < kv_end) {
            load(c0 + 2 * chunk, ids_a, ka, va, ja);
            if (c0 + 3 * chunk < kv_end) load_ids(c0 + 3 * chunk, ids_b);
        }
        compute(kb, vb, jb);
    }

    // ---- merge the lane groups of the wave (lanes li + LPR g), then the waves through LDS
    const int stride = 2 + head_dim;
#pragma unroll
    for (int qi = 0; qi < NQ; qi++) {
        if (qi >= nq) break;
        const float M = across_groups<LPR, true>(m[qi]);
        const float f = (M == -INFINITY) ? 0.0f : exp2f(m[qi] - M);
        const float L = across_groups<LPR, false>(l[qi] * f);
        float* r = red + ((int64_t)w * NQ + qi) * stride;
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            const float a = across_groups<LPR, false>(acc[qi][e] * f);
            if (grp == 0) r[2 + li * VEC + e] = a;
        }
        if (lane == 0) {
            r[0] = M;
            r[1] = L;
        }
    }
    __syncthreads();
    for (int x = tid; x < nq * head_dim; x += blockDim.x) {
        const int qi = x / head_dim, d = x - qi * head_dim;
        float M = -INFINITY;
        for (int ww = 0; ww < waves; ww++) M = fmaxf(M, red[((int64_t)ww * NQ + qi) * stride]);
        float L = 0.0f, A = 0.0f;
        if (M != -INFINITY) {
            for (int ww = 0; ww < waves; ww++) {
                const float* r = red + ((int64_t)ww * NQ + qi) * stride;
                const float f = exp2f(r[0] - M);
                L += r[1] * f;
                A += r[2 + d] * f;
            }
        }
        const int rr = qi / nh, hh = qi - rr * nh;
        store_out(out, out_dtype, (int64_t)(r0 + rr) * o_st + (int64_t)(h0 + hh) * o_sh + d,
                  L > 0.0f ? A / L : 0.0f);
    }
}

static int nq_pow2(int nq) { return nq <= 1 ? 1 : nq <= 2 ? 2 : nq <= 4 ? 4 : 8; }

static int device_cus_simt() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

template <typename T, int LPR, int NQ>
static void launch_simt_t(dim3 grid, int waves, size_t lds, void* out, int out_dtype,
                          int64_t o_st, int64_t o_sh, const void* q, int64_t q_st, int64_t q_sh,
                          const void* k_pool, const void* v_pool, const int32_t* cu,
                          const int32_t* kv_lens, const int32_t* bt, int max_blocks,
                          int num_seqs, int n_rep, int hpg, int rows, int head_dim,
                          int block_size, int64_t num_slots, int max_kv, float scale_log2,
                          hipStream_t stream) {
    attn_simt_kernel<T, LPR, NQ><<<grid, dim3(64 * waves), lds, stream>>>(
        out, out_dtype, o_st, o_sh, static_cast<const T*>(q), q_st, q_sh,
        static_cast<const T*>(k_pool), static_cast<const T*>(v_pool), cu, kv_lens, bt,
        max_blocks, num_seqs, n_rep, hpg, rows, head_dim, block_size, num_slots, max_kv,
        scale_log2);
}

template <typename T, int LPR>
static void launch_simt_nq(int nq, dim3 grid, int waves, size_t lds, void* out, int out_dtype,
                           int64_t o_st, int64_t o_sh, const void* q, int64_t q_st, int64_t q_sh,
                           const void* k_pool, const void* v_pool, const int32_t* cu,
                           const int32_t* kv_lens, const int32_t* bt, int max_blocks,
                           int num_seqs, int n_rep, int hpg, int rows, int head_dim,
                           int block_size, int64_t num_slots, int max_kv, float scale_log2,
                           hipStream_t stream) {
#define FLOUR_SIMT_NQ(N)                                                                      \
    launch_simt_t<T, LPR, N>(grid, waves, lds, out, out_dtype, o_st, o_sh, q, q_st, q_sh,      \
                             k_pool, v_pool, cu, kv_lens, bt, max_blocks, num_seqs, n_rep, hpg, \
                             rows, head_dim, block_size, num_slots, max_kv, scale_log2, stream)
    if (nq <= 1)
        FLOUR_SIMT_NQ(1);
    else if (nq <= 2)
        FLOUR_SIMT_NQ(2);
    else if (nq <= 4)
        FLOUR_SIMT_NQ(4);
    else
        FLOUR_SIMT_NQ(8);
#undef FLOUR_SIMT_NQ
}

// Whether the vector kernel takes a shape: a row of 16-byte chunks spread over 2 to 64 lanes
// (a power of two), head_dim <= 256, 16-byte aligned pointers and strides.
bool simt_supported(int dtype, int head_dim, const void* q, int64_t q_st, int64_t q_sh,
                    const void* k_pool, const void* v_pool) {
    const int es = dtype == FLOUR_DTYPE_F32 ? 4 : 2;
    const int row_bytes = head_dim * es;
    if (row_bytes % 16 != 0 || head_dim > SIMT_MAX_D) return false;
    const int lpr = row_bytes / 16;
    if (lpr < 2 || lpr > 64 || (lpr & (lpr - 1)) != 0) return false;
    return ((uintptr_t)q % 16 == 0) && ((uintptr_t)k_pool % 16 == 0) &&
           ((uintptr_t)v_pool % 16 == 0) && ((q_st * es) % 16 == 0) && ((q_sh * es) % 16 == 0);
}

template <typename T>
static void launch_simt_lpr(int lpr, int nq, dim3 grid, int waves, size_t lds, void* out,
                            int out_dtype, int64_t o_st, int64_t o_sh, const void* q,
                            int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool,
                            const int32_t* cu, const int32_t* kv_lens, const int32_t* bt,
                            int max_blocks, int num_seqs, int n_rep, int hpg, int rows,
                            int head_dim, int block_size, int64_t num_slots, int max_kv,
                            float scale_log2, hipStream_t stream) {
#define FLOUR_SIMT(L)                                                                          \
    launch_simt_nq<T, L>(nq, grid, waves, lds, out, out_dtype, o_st, o_sh, q, q_st, q_sh,     \
                         k_pool, v_pool, cu, kv_lens, bt, max_blocks, num_seqs, n_rep, hpg,    \
                         rows, head_dim, block_size, num_slots, max_kv, scale_log2, stream)
    switch (lpr) {
        case 2: FLOUR_SIMT(2); break;
        case 4: FLOUR_SIMT(4); break;
        case 8: FLOUR_SIMT(8); break;
        case 16: FLOUR_SIMT(16); break;
        case 32: FLOUR_SIMT(32); break;
        default: FLOUR_SIMT(64); break;
    }
#undef FLOUR_SIMT
}

// Launch the vector kernel (simt_supported must hold); dtype is the storage type of q and the
// pools; cu == nullptr means one query row per sequence (decode). `max_q` bounds the query rows
// of one sequence and `max_kv` its kv length (both size the launch).
int launch_attn_simt(int dtype, int out_dtype, void* out, int64_t o_st, int64_t o_sh,
                     const void* q, int64_t q_st, int64_t q_sh, const void* k_pool,
                     const void* v_pool, const int32_t* cu, const int32_t* kv_lens,
                     const int32_t* bt, int max_blocks, int num_seqs, int total_q, int num_heads,
                     int n_rep, int head_dim, int block_size, int64_t num_slots, int max_kv,
                     float scale, hipStream_t stream) {
    if (total_q == 0 || num_seqs == 0) return FLOUR_OK;
    const int kv_heads = num_heads / n_rep;
    const int es = dtype == FLOUR_DTYPE_F32 ? 4 : 2;
    const int lpr = head_dim * es / 16;
    const int hpg = n_rep < SIMT_NQ_MAX ? n_rep : SIMT_NQ_MAX;  // heads per group
    const int groups = (n_rep + hpg - 1) / hpg;
    const int rows = cu ? (SIMT_NQ_MAX / hpg) : 1;  // query rows per workgroup
    const int nq = rows * hpg;
    // prefill: row blocks per sequence are ceil(q_len / rows); their total is at most
    // total_q / rows + num_seqs (blocks past the last exit at once)
    const int64_t items = cu ? ((int64_t)total_q + rows - 1) / rows + num_seqs : num_seqs;
    if (items > 0x7fffffff || kv_heads > 65535 || groups > 65535) {
        set_error("attention (vector kernel): grid too large");
        return FLOUR_ERR_UNSUPPORTED;
    }
    // waves per workgroup: enough workgroups x waves for 8 waves per CU, no more waves than the
    // longest kv range has row loads for, and the merge buffer within 64 KiB of LDS
    const int64_t wgs = items * kv_heads * groups;
    const int64_t want = (8LL * device_cus_simt() + wgs - 1) / wgs;
    const int64_t kv_cap = std::min<int64_t>(max_kv, (int64_t)max_blocks * block_size);
    const int64_t loads = (kv_cap + (64 / lpr) * SIMT_UNROLL - 1) / ((64 / lpr) * SIMT_UNROLL);
    int waves = 1;
    const size_t per_wave = (size_t)nq_pow2(nq) * (2 + head_dim) * sizeof(float);
    while (waves < simt_max_waves(nq_pow2(nq)) && waves < want && waves < loads &&
           (size_t)(2 * waves) * per_wave <= (64u << 10))
        waves *= 2;
    const size_t lds = (size_t)waves * per_wave;
    const dim3 grid((unsigned)items, kv_heads, groups);
    const float sl2 = scale * 1.4426950408889634f;
    if (dtype == FLOUR_DTYPE_F32)
        launch_simt_lpr<float>(lpr, nq, grid, waves, lds, out, out_dtype, o_st, o_sh, q, q_st,
                               q_sh, k_pool, v_pool, cu, kv_lens, bt, max_blocks, num_seqs, n_rep,
                               hpg, rows, head_dim, block_size, num_slots, max_kv, sl2, stream);
    else if (dtype == FLOUR_DTYPE_BF16)
        launch_simt_lpr<bf16_t>(lpr, nq, grid, waves, lds, out, out_dtype, o_st, o_sh, q, q_st,
                                q_sh, k_pool, v_pool, cu, kv_lens, bt, max_blocks, num_seqs,
                                n_rep, hpg, rows, head_dim, block_size, num_slots, max_kv, sl2,
                                stream);
    else
        launch_simt_lpr<f16_t>(lpr, nq, grid, waves, lds, out, out_dtype, o_st, o_sh, q, q_st,
                               q_sh, k_pool, v_pool, cu, kv_lens, bt, max_blocks, num_seqs, n_rep,
                               hpg, rows, head_dim, block_size, num_slots, max_kv, sl2, stream);
    return check_hip(hipGetLastError(), "attention (vector kernel) launch");
}

}  // namespace flour
