// paged_decode.hip — kernel (2): paged decode attention on gfx950 matrix cores.
//
// Replaces paged_attention (src/backend/cpu.rs:57-112) for one new query per sequence
// (seq_q == 1, the decode step engine.rs:259-262), batched over sequences. The block list of
// Cache::kv_blocks (cache.rs:456-458, KvCache::gather_blocks cache.rs:83-96) arrives as a
// block table; query head h reads kv head h / n_rep (repeat_kv, cpu.rs:5-13); with seq_q == 1
// the causal mask of cpu.rs:88-95 admits every cached position, so only positions past the
// context length are masked.
//
// Design (bf16/f16 pools, head_dim 128, block_size a multiple of 16):
//  * One workgroup of 4 waves per (context split, kv head, sequence). Every wave handles
//    16-token tiles (one MFMA tile; one 4 KB (head, 16 slots) pool run of K and of V) with a
//    stride of 4 tiles, so the 4 waves stream adjacent pool memory. All n_rep query heads of
//    the kv head share each K/V load (GQA reuse: K/V are read from HBM once).
//  * Scores S = K Q^T on v_mfma_f32_16x16x32 (M = 16 tokens, N = 16 query-head columns, the
//    n_rep real heads padded with zero rows), so lane (g, c) = (lane/16, lane%16) holds the
//    scores of query head c for tokens 4g..4g+3.
//  * That register layout is exactly the B operand of v_mfma_f32_16x16x16 for O^T = V^T P^T
//    (K = the 16 tokens), so P never leaves the lane. The V^T A operand is built in-lane:
//    each lane loads V rows 4g..4g+3, dims 8c..8c+7 (four fully coalesced 16 B loads; a wave
//    reads 4 whole 256 B rows per instruction) and v_perm_b32 packs, per output dim 8c+n,
//    the four tokens' values. The O^T accumulator then holds, in lane (g, c), query head c at
//    dims 32g..32g+31.
//  * P is split into bf16 hi + lo parts (two MFMAs per product) so the P.V contraction keeps
//    ~16 mantissa bits of P; products are exact in fp32 and accumulate in fp32.
//  * Online softmax in the exp2 domain: the only cross-lane step per tile is the max over the
//    four 4-token row groups (two xor shuffles); running sums stay lane-partial until the
//    end, and the accumulator is rescaled only when some lane's max moved.
//  * Split-context: partial (max, sum, acc) rows go to the workspace; the last workgroup of a
//    (sequence, kv head) — elected with an atomic counter it resets — merges them (log-sum-
//    exp merge, as in the running update of cpu.rs:96-105) and writes the output.
#include <math.h>

#include "flour_common.h"

namespace flour {

int launch_attn_generic(int dtype, int out_dtype, void* out, int64_t o_st, int64_t o_sh,
                        const void* q, int64_t q_st, int64_t q_sh, const void* k_pool,
                        const void* v_pool, const int32_t* cu, const int32_t* kv_lens,
                        const int32_t* bt, int max_blocks, int num_seqs, int total_q,
                        int num_heads, int n_rep, int head_dim, int block_size, int64_t num_slots,
                        float scale, hipStream_t stream);

static constexpr int DEC_D = 128;
static constexpr int DEC_WAVES = 4;
static constexpr int DEC_THREADS = DEC_WAVES * 64;
static constexpr float LOG2E = 1.4426950408889634f;

struct DecodeWs {
    int* counters;  // [batch * kv_heads]
    float* ml;      // [batch * kv_heads * max_splits * n_rep][2] (max, sum), exp2 domain
    float* o;       // [batch * kv_heads * max_splits * n_rep * D]
};

// Tokens per context split: a multiple of 64 (4 waves x 16-token tiles). Long contexts use
// 512-token splits; short or few sequences use smaller splits so the grid fills the 256 CUs.
static int choose_split_tokens(int batch, int kv_heads, int max_context_len) {
    int split = 512;
    const int64_t units = (int64_t)batch * kv_heads;
    while (split > 64 && units * ((max_context_len + split - 1) / split) < 1024) split >>= 1;
    return split;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static size_t decode_ws_bytes(int batch, int kv_heads, int n_rep, int head_dim, int max_splits) {
    const size_t units = (size_t)batch * kv_heads;
    return align256(units * sizeof(int)) + align256(units * max_splits * n_rep * 2 * sizeof(float)) +
           align256(units * max_splits * n_rep * (size_t)head_dim * sizeof(float));
}

template <typename T, typename TO>
__global__ __launch_bounds__(DEC_THREADS) void paged_decode_mfma_kernel(
    TO* __restrict__ out, const T* __restrict__ q, const T* __restrict__ k_pool,
    const T* __restrict__ v_pool, const int32_t* __restrict__ block_tables, int max_blocks,
    const int32_t* __restrict__ context_lens, int num_heads, int kv_heads, int n_rep,
    int block_size, int64_t num_slots, int max_ctx, float scale_log2, int split_tokens,
    int max_splits, DecodeWs ws) {
    constexpr int D = DEC_D;
    extern __shared__ float smem[];  // [4 waves][n_rep][D] acc, then [4][n_rep] max, sum

    const int sp = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, lg = lane >> 4, lc = lane & 15;
    // Context lengths beyond the stated maximum are clamped, so a bad length can neither read
    // past the block table nor leave a split unmerged.
    const int ctx = min(context_lens[b], max_ctx);
    const int n_splits = ctx > 0 ? (ctx + split_tokens - 1) / split_tokens : 1;
    if (sp >= n_splits) return;

    TO* out_g = out + ((int64_t)b * num_heads + (int64_t)g * n_rep) * D;
    if (ctx <= 0) {  // empty context: the row is defined as zeros
        for (int idx = tid; idx < n_rep * D; idx += DEC_THREADS) out_g[idx] = from_f32<TO>(0.0f);
        return;
    }

    // Q^T as the B operand: lane (lg, lc) holds head lc, dims 32kk + 8lg .. +7.
    u32x4 qb[4];
    {
        const T* qh = q + ((int64_t)b * num_heads + (int64_t)g * n_rep + lc) * D + 8 * lg;
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            qb[kk] = (lc < n_rep) ? *reinterpret_cast<const u32x4*>(qh + 32 * kk) : u32x4{0, 0, 0, 0};
        }
    }

    const int tok_begin = sp * split_tokens;
    const int tok_end = min(ctx, tok_begin + split_tokens);
    const int ntiles = (tok_end - tok_begin + 15) >> 4;
    const int32_t* bt = block_tables + (int64_t)b * max_blocks;
    const T* k_head = k_pool + (int64_t)g * num_slots * D;
    const T* v_head = v_pool + (int64_t)g * num_slots * D;
    const int64_t max_phys = num_slots / block_size - 1;

    float m = -INFINITY, lsum = 0.0f;
    f32x4 acc[8];
#pragma unroll
    for (int nn = 0; nn < 8; nn++) acc[nn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    u32x4 ka[4], va[4];
    auto load_tile = [&](int it, u32x4* kd, u32x4* vd) {
        const int tok0 = tok_begin + it * 16;
        const int lb = tok0 / block_size;
        const int within = tok0 - lb * block_size;
        int64_t phys = bt[lb];  // clamped: a bad block id never leaves the pool
        phys = phys < 0 ? 0 : (phys > max_phys ? max_phys : phys);
        const int64_t slot0 = phys * block_size + within;
        const T* kp = k_head + slot0 * D;
        const T* vp = v_head + slot0 * D;
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
            kd[kk] = *reinterpret_cast<const u32x4*>(kp + lc * D + 32 * kk + 8 * lg);
#pragma unroll
        for (int j = 0; j < 4; j++)
            vd[j] = *reinterpret_cast<const u32x4*>(vp + (4 * lg + j) * D + 8 * lc);
    };

    int it = w;
    if (it < ntiles) load_tile(it, ka, va);
    for (; it < ntiles; it += DEC_WAVES) {
        u32x4 kn[4], vn[4];
        const int nxt = it + DEC_WAVES;
        if (nxt < ntiles) load_tile(nxt, kn, vn);

        const int tok0 = tok_begin + it * 16;
        const bool full = tok0 + 16 <= tok_end;
        if (!full) {  // tokens past the context: zero V so garbage pool bits cannot leak in
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (tok0 + 4 * lg + j >= tok_end) va[j] = u32x4{0, 0, 0, 0};
        }

        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < 4; kk++) s = mfma16x16x32<T>(ka[kk], qb[kk], s);

        float sv[4];
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const bool ok = full || (tok0 + 4 * lg + r < tok_end);
            sv[r] = ok ? s[r] * scale_log2 : -INFINITY;
            tmax = fmaxf(tmax, sv[r]);
        }
        tmax = fmaxf(tmax, wave_shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, wave_shfl_xor(tmax, 32));
        const float m_new = fmaxf(m, tmax);
        const float alpha = fast_exp2(m - m_new);
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; r++) p[r] = fast_exp2(sv[r] - m_new);
        lsum = lsum * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
        if (__builtin_amdgcn_ballot_w64(m_new > m) != 0) {
#pragma unroll
            for (int nn = 0; nn < 8; nn++) acc[nn] *= alpha;
        }
        m = m_new;

        // P^T as B operand, split hi + lo.
        const uint32_t ph0 = pack2<T>(p[0], p[1]), ph1 = pack2<T>(p[2], p[3]);
        const uint32_t pl0 = pack2<T>(p[0] - lo_f32<T>(ph0), p[1] - hi_f32<T>(ph0));
        const uint32_t pl1 = pack2<T>(p[2] - lo_f32<T>(ph1), p[3] - hi_f32<T>(ph1));
        const u32x2 PH = {ph0, ph1}, PL = {pl0, pl1};

#pragma unroll
        for (int nn = 0; nn < 8; nn++) {
            const int wd = nn >> 1;
            u32x2 A;
            if (nn & 1) {
                A[0] = perm_hi16(va[0][wd], va[1][wd]);
                A[1] = perm_hi16(va[2][wd], va[3][wd]);
            } else {
                A[0] = perm_lo16(va[0][wd], va[1][wd]);
                A[1] = perm_lo16(va[2][wd], va[3][wd]);
            }
            acc[nn] = mfma16x16x16<T>(A, PH, acc[nn]);
            acc[nn] = mfma16x16x16<T>(A, PL, acc[nn]);
        }

        if (nxt < ntiles) {
#pragma unroll
            for (int x = 0; x < 4; x++) {
                ka[x] = kn[x];
                va[x] = vn[x];
            }
        }
    }

    // Wave totals: the row sum over the four row groups (max is already shared).
    lsum += wave_shfl_xor(lsum, 16);
    lsum += wave_shfl_xor(lsum, 32);

    float* sm_o = smem;                                  // [4][n_rep][D]
    float* sm_m = smem + DEC_WAVES * n_rep * D;          // [4][n_rep]
    float* sm_l = sm_m + DEC_WAVES * n_rep;              // [4][n_rep]
    if (lc < n_rep) {
        float* o = sm_o + (w * n_rep + lc) * D + 32 * lg;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int nn = 0; nn < 8; nn++) o[8 * r + nn] = acc[nn][r];
        if (lg == 0) {
            sm_m[w * n_rep + lc] = m;
            sm_l[w * n_rep + lc] = lsum;
        }
    }
    __syncthreads();

    const int unit = b * kv_heads + g;
    for (int idx = tid; idx < n_rep * D; idx += DEC_THREADS) {
        const int hh = idx / D, d = idx - hh * D;
        float M = -INFINITY;
#pragma unroll
        for (int x = 0; x < DEC_WAVES; x++) M = fmaxf(M, sm_m[x * n_rep + hh]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int x = 0; x < DEC_WAVES; x++) {
            const float mx = sm_m[x * n_rep + hh];
            const float f = (mx == -INFINITY) ? 0.0f : fast_exp2(mx - M);
            L += f * sm_l[x * n_rep + hh];
            O += f * sm_o[(x * n_rep + hh) * D + d];
        }
        if (n_splits == 1) {
            out_g[idx] = from_f32<TO>(O / L);
        } else {
            const int64_t pidx = ((int64_t)unit * max_splits + sp) * n_rep + hh;
            ws.o[pidx * D + d] = O;
            if (d == 0) {
                ws.ml[2 * pidx] = M;
                ws.ml[2 * pidx + 1] = L;
            }
        }
    }
    if (n_splits == 1) return;

    // Split-context merge: the last workgroup of this (sequence, kv head) combines partials.
    __shared__ int sm_last;
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const int prev = atomicAdd(&ws.counters[unit], 1);
        sm_last = (prev == n_splits - 1);
    }
    __syncthreads();
    if (!sm_last) return;
    __threadfence();
    for (int idx = tid; idx < n_rep * D; idx += DEC_THREADS) {
        const int hh = idx / D, d = idx - hh * D;
        const int64_t base = (int64_t)unit * max_splits * n_rep + hh;
        float M = -INFINITY;
        for (int x = 0; x < n_splits; x++) M = fmaxf(M, ws.ml[2 * (base + (int64_t)x * n_rep)]);
        float L = 0.0f, O = 0.0f;
        for (int x = 0; x < n_splits; x++) {
            const int64_t pidx = base + (int64_t)x * n_rep;
            const float mx = ws.ml[2 * pidx];
            const float f = (mx == -INFINITY) ? 0.0f : fast_exp2(mx - M);
            L += f * ws.ml[2 * pidx + 1];
            O += f * ws.o[pidx * D + d];
        }
        out_g[idx] = from_f32<TO>(O / L);
    }
    if (tid == 0) ws.counters[unit] = 0;  // leave the counter ready for the next call
}

template <typename T, typename TO>
static int launch_decode_mfma(void* out, const void* q, const void* k_pool, const void* v_pool,
                              const int32_t* bt, int max_blocks, const int32_t* ctx_lens,
                              int batch, int num_heads, int kv_heads, int n_rep, int block_size,
                              int64_t num_slots, int max_ctx, float scale, int split_tokens,
                              int max_splits, DecodeWs ws, hipStream_t stream) {
    const size_t lds = (size_t)(DEC_WAVES * n_rep * DEC_D + 2 * DEC_WAVES * n_rep) * sizeof(float);
    dim3 grid(max_splits, kv_heads, batch);
    paged_decode_mfma_kernel<T, TO><<<grid, dim3(DEC_THREADS), lds, stream>>>(
        static_cast<TO*>(out), static_cast<const T*>(q), static_cast<const T*>(k_pool),
        static_cast<const T*>(v_pool), bt, max_blocks, ctx_lens, num_heads, kv_heads, n_rep,
        block_size, num_slots, max_ctx, scale * LOG2E, split_tokens, max_splits, ws);
    return check_hip(hipGetLastError(), "paged_decode launch");
}

}  // namespace flour

using namespace flour;

extern "C" int flour_hip_paged_decode_workspace_size(int batch, int num_heads, int kv_heads,
                                                     int head_dim, int max_context_len,
                                                     size_t* bytes) {
    clear_error();
    if (!bytes || batch < 0 || num_heads <= 0 || kv_heads <= 0 || num_heads % kv_heads != 0 ||
        head_dim <= 0 || max_context_len < 0) {
        set_error("paged_decode_workspace_size: bad arguments");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    const int split = choose_split_tokens(batch, kv_heads, max_context_len);
    const int max_splits = max_context_len > 0 ? (max_context_len + split - 1) / split : 1;
    *bytes = decode_ws_bytes(batch, kv_heads, num_heads / kv_heads, head_dim, max_splits);
    return FLOUR_OK;
}

extern "C" int flour_hip_paged_decode(void* out, int out_dtype, const void* q,
                                      const void* k_pool, const void* v_pool,
                                      const int32_t* block_tables, int max_blocks_per_seq,
                                      const int32_t* context_lens, int batch, int num_heads,
                                      int kv_heads, int head_dim, int block_size,
                                      int64_t num_slots, int max_context_len, float scale,
                                      int dtype, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    clear_error();
    if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) {
        set_error("paged_decode: unknown dtype (%d, out %d)", dtype, out_dtype);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (batch < 0 || num_heads <= 0 || kv_heads <= 0 || num_heads % kv_heads != 0 ||
        head_dim <= 0 || block_size <= 0 || num_slots <= 0 || max_blocks_per_seq <= 0 ||
        max_context_len < 0 || (int64_t)max_context_len > (int64_t)max_blocks_per_seq * block_size) {
        set_error("paged_decode: bad shape (batch=%d heads=%d kv_heads=%d head_dim=%d bs=%d "
                  "max_blocks=%d max_ctx=%d)",
                  batch, num_heads, kv_heads, head_dim, block_size, max_blocks_per_seq,
                  max_context_len);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (batch == 0) return FLOUR_OK;
    if (!out || !q || !k_pool || !v_pool || !block_tables || !context_lens) {
        set_error("paged_decode: null pointer");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int n_rep = num_heads / kv_heads;
    const bool mfma = (dtype == FLOUR_DTYPE_BF16 || dtype == FLOUR_DTYPE_F16) &&
                      head_dim == DEC_D && block_size % 16 == 0 && n_rep <= 16 &&
                      ((uintptr_t)q % 16 == 0) && ((uintptr_t)k_pool % 16 == 0) &&
                      ((uintptr_t)v_pool % 16 == 0);
    if (!mfma) {
        // one query row per sequence: cu_seqlens == nullptr
        return launch_attn_generic(dtype, out_dtype, out, (int64_t)num_heads * head_dim, head_dim,
                                   q, (int64_t)num_heads * head_dim, head_dim, k_pool, v_pool,
                                   nullptr, context_lens, block_tables, max_blocks_per_seq, batch,
                                   batch, num_heads, n_rep, head_dim, block_size, num_slots, scale,
                                   s);
    }
    if (batch > 65535 || kv_heads > 65535) {
        set_error("paged_decode: batch/kv_heads beyond grid limits");
        return FLOUR_ERR_UNSUPPORTED;
    }
    const int split = choose_split_tokens(batch, kv_heads, max_context_len);
    const int max_splits = max_context_len > 0 ? (max_context_len + split - 1) / split : 1;
    DecodeWs ws{nullptr, nullptr, nullptr};
    if (max_splits > 1) {
        const size_t need = decode_ws_bytes(batch, kv_heads, n_rep, head_dim, max_splits);
        if (!workspace || workspace_bytes < need || ((uintptr_t)workspace % 256) != 0) {
            set_error("paged_decode: workspace of %zu bytes (256-byte aligned, zero-filled once) "
                      "required, got %zu at %p",
                      need, workspace_bytes, workspace);
            return FLOUR_ERR_WORKSPACE;
        }
        const size_t units = (size_t)batch * kv_heads;
        char* p = static_cast<char*>(workspace);
        ws.counters = reinterpret_cast<int*>(p);
        p += align256(units * sizeof(int));
        ws.ml = reinterpret_cast<float*>(p);
        p += align256(units * max_splits * n_rep * 2 * sizeof(float));
        ws.o = reinterpret_cast<float*>(p);
    }
#define FLOUR_DEC(T)                                                                            \
    do {                                                                                        \
        if (out_dtype == FLOUR_DTYPE_F32)                                                       \
            return launch_decode_mfma<T, float>(out, q, k_pool, v_pool, block_tables,           \
                                                max_blocks_per_seq, context_lens, batch,        \
                                                num_heads, kv_heads, n_rep, block_size,         \
                                                num_slots, max_context_len, scale, split, max_splits, ws, s);    \
        if (out_dtype == FLOUR_DTYPE_BF16)                                                      \
            return launch_decode_mfma<T, bf16_t>(out, q, k_pool, v_pool, block_tables,          \
                                                 max_blocks_per_seq, context_lens, batch,       \
                                                 num_heads, kv_heads, n_rep, block_size,        \
                                                 num_slots, max_context_len, scale, split, max_splits, ws, s);   \
        return launch_decode_mfma<T, f16_t>(out, q, k_pool, v_pool, block_tables,               \
                                            max_blocks_per_seq, context_lens, batch, num_heads, \
                                            kv_heads, n_rep, block_size, num_slots,             \
                                            max_context_len, scale, split, max_splits, ws, s);                          \
    } while (0)
    if (dtype == FLOUR_DTYPE_BF16) FLOUR_DEC(bf16_t);
    FLOUR_DEC(f16_t);
#undef FLOUR_DEC
}
