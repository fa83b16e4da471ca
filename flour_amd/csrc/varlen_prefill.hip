// varlen_prefill.hip — kernel (3): causal varlen prefill attention over the paged cache, on
// gfx950 bf16/f16 matrix cores.
//
// Replaces paged_attention (src/backend/cpu.rs:57-112) for seq_q >= 1 (prefill,
// CausalLM::forward model.rs:43-59 and the suffix-only prefill_suffix model.rs:68-85),
// batched over packed sequences (cu_seqlens layout). Sequence s has q_len query rows and
// kv_len cached positions (its prefix-cached shared blocks, then its own new rows); query i
// sees kv position j iff j <= kv_len - q_len + i (cpu.rs:68, :88-95); query head h reads kv
// head h / n_rep (repeat_kv, cpu.rs:5-13).
//
// Design (head_dim 128, block_size a multiple of 16):
//  * One workgroup (4 waves) per (128-row query tile, query head, sequence); wave w owns 32
//    query rows. Tiles are issued heaviest first (last query tile of every sequence first),
//    and the (sequence, head) order inside one tile rank is permuted so that the heads that
//    share a kv head land on the same XCD (same L2) — the hardware deals workgroups to the 8
//    XCDs round-robin.
//  * 64-token K/V tiles are gathered page by page through the block table into LDS; the
//    global loads of tile t+1 are in flight while tile t is computed. K is stored row-major
//    (pitch 272 B, conflict-free 16 B reads); V is stored transposed (V^T, pitch 144 B) with the
//    tokens of each 16-token group permuted (bits 2 and 3 swapped), which is the order in which
//    the score registers feed the P.V product.
//  * S^T = K Q^T on v_mfma_f32_32x32x16 (M = 32 tokens, N = 32 queries, K = 16 dims): lane
//    (h, q) = (lane/32, lane%32) holds query q's scores for tokens 8i + 4h + j. Those registers
//    are, after bf16 packing, the B operand of O^T = V^T P^T (K = 16 tokens), so P never moves
//    between lanes; V^T rows come straight from LDS as 16 B reads.
//  * Online softmax in the exp2 domain, one max exchange between the two lane halves per tile;
//    the output accumulator is rescaled only when some lane's max moved. Fully masked tiles
//    are skipped per wave, masks are evaluated only on tiles that cross the diagonal.
//  * PRECISE_P: P is split into hi + lo 16-bit parts (two MFMAs per product), keeping ~16
//    mantissa bits of the softmax weights; otherwise P is rounded once to 16 bits.
#include <math.h>

#include "flour_common.h"

namespace flour {

int launch_attn_generic(int dtype, int out_dtype, void* out, int64_t o_st, int64_t o_sh,
                        const void* q, int64_t q_st, int64_t q_sh, const void* k_pool,
                        const void* v_pool, const int32_t* cu, const int32_t* kv_lens,
                        const int32_t* bt, int max_blocks, int num_seqs, int total_q,
                        int num_heads, int n_rep, int head_dim, int block_size, int64_t num_slots,
                        float scale, hipStream_t stream);

static constexpr int PF_D = 128;
static constexpr int PF_QT = 128;  // query rows per workgroup
static constexpr int PF_KT = 64;   // kv tokens per tile
static constexpr int PF_THREADS = 256;
static constexpr int PF_KPITCH = PF_D + 8;   // elements: 272 B rows
static constexpr int PF_VPITCH = PF_KT + 8;  // elements: 144 B rows
static constexpr float PF_LOG2E = 1.4426950408889634f;

__device__ __forceinline__ int swap_bits01(int x) {
    return (x & ~3) | ((x & 1) << 1) | ((x >> 1) & 1);
}

template <typename T, typename TO, bool PRECISE_P>
__global__ __launch_bounds__(PF_THREADS, 2) void varlen_prefill_mfma_kernel(
    TO* __restrict__ out, int64_t o_st, int64_t o_sh, const T* __restrict__ q, int64_t q_st,
    int64_t q_sh, const T* __restrict__ k_pool, const T* __restrict__ v_pool,
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ block_tables, int max_blocks, int num_seqs, int num_heads,
    int n_rep, int block_size, int64_t num_slots, float scale_log2) {
    constexpr int D = PF_D;
    __shared__ __attribute__((aligned(16))) uint16_t Ks[PF_KT * PF_KPITCH];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[PF_D * PF_VPITCH];

    // ---- work item: (query tile from the end, sequence, head)
    const int per_rank = num_seqs * num_heads;
    const int bid = blockIdx.x;
    const int tile_rev = bid / per_rank;
    int r = bid - tile_rev * per_rank;
    const int full8 = per_rank & ~7;
    if (r < full8) r = (r & 7) * (full8 >> 3) + (r >> 3);
    const int seq = r / num_heads;
    const int head = r - seq * num_heads;

    const int q0 = cu_seqlens[seq];
    const int ql = cu_seqlens[seq + 1] - q0;
    // kv lengths are clamped to what the block table can address (a bad length never reads
    // past the table).
    const int kv_len = min(kv_lens[seq], max_blocks * block_size);
    const int n_qt = (ql + PF_QT - 1) / PF_QT;
    const int qt = n_qt - 1 - tile_rev;
    if (qt < 0 || kv_len < ql) return;
    const int off = kv_len - ql;
    const int row_begin = qt * PF_QT;
    const int row_last = min(row_begin + PF_QT, ql) - 1;
    const int kv_end = off + row_last + 1;  // exclusive bound of visible kv for this tile
    const int n_kt = (kv_end + PF_KT - 1) / PF_KT;

    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int h2 = lane >> 5, ql32 = lane & 31;
    const int kvh = head / n_rep;
    const int32_t* bt = block_tables + (int64_t)seq * max_blocks;
    const T* k_head = k_pool + (int64_t)kvh * num_slots * D;
    const T* v_head = v_pool + (int64_t)kvh * num_slots * D;
    const int64_t max_phys = num_slots / block_size - 1;

    // ---- this lane's query row and its causal limit (padded rows copy the last valid row)
    const int wr0 = row_begin + 32 * w;
    const bool wave_active = wr0 < ql;
    const int qrow = min(wr0 + ql32, ql - 1);
    const int lim = off + qrow;                       // visible kv j <= lim
    const int wave_lim = off + min(wr0 + 31, ql - 1);  // largest limit in the wave
    const int wave_min_lim = off + wr0;                // smallest limit in the wave

    // Q^T as the B operand: lane (h2, q) holds row q, dims 16kk + 8h2 .. +7.
    u32x4 qb[8];
    {
        const T* qp = q + (int64_t)(q0 + qrow) * q_st + (int64_t)head * q_sh + 8 * h2;
#pragma unroll
        for (int kk = 0; kk < 8; kk++) qb[kk] = *reinterpret_cast<const u32x4*>(qp + 16 * kk);
    }

    // ---- staging assignment
    // K: 4 chunks of 16 B per thread: chunk c = tid + 256 i -> token c / 16, dims (c % 16) * 8.
    // V: token quad tq = tid % 16 (tokens 4tq..4tq+3), dims 8 dg .. 8 dg + 7 with dg = tid / 16.
    const int v_tq = tid & 15, v_dg = tid >> 4;
    u32x4 kst[4], vst[4];
    auto slot_of = [&](int tok) -> int64_t {
        const int lb = tok / block_size;
        int64_t phys = bt[lb];
        phys = phys < 0 ? 0 : (phys > max_phys ? max_phys : phys);
        return phys * block_size + (tok - lb * block_size);
    };
    auto gload = [&](int kt) {
        const int kv0 = kt * PF_KT;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + PF_THREADS * i;
            const int tok = kv0 + (c >> 4);
            if (tok < kv_len)
                kst[i] = *reinterpret_cast<const u32x4*>(k_head + slot_of(tok) * D + (c & 15) * 8);
            else
                kst[i] = u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int tok = kv0 + 4 * v_tq + j;
            if (tok < kv_len)
                vst[j] = *reinterpret_cast<const u32x4*>(v_head + slot_of(tok) * D + 8 * v_dg);
            else
                vst[j] = u32x4{0, 0, 0, 0};
        }
    };
    auto lds_store = [&]() {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int c = tid + PF_THREADS * i;
            *reinterpret_cast<u32x4*>(&Ks[(c >> 4) * PF_KPITCH + (c & 15) * 8]) = kst[i];
        }
        const int col = 4 * swap_bits01(v_tq);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int wd = e >> 1;
            u32x2 pr;
            if (e & 1) {
                pr[0] = perm_hi16(vst[0][wd], vst[1][wd]);
                pr[1] = perm_hi16(vst[2][wd], vst[3][wd]);
            } else {
                pr[0] = perm_lo16(vst[0][wd], vst[1][wd]);
                pr[1] = perm_lo16(vst[2][wd], vst[3][wd]);
            }
            *reinterpret_cast<u32x2*>(&Vt[(8 * v_dg + e) * PF_VPITCH + col]) = pr;
        }
    };

    float m = -INFINITY, lsum = 0.0f;
    f32x16 o[4];
#pragma unroll
    for (int x = 0; x < 4; x++)
#pragma unroll
        for (int y = 0; y < 16; y++) o[x][y] = 0.0f;

    gload(0);
    for (int kt = 0; kt < n_kt; kt++) {
        lds_store();
        __syncthreads();
        if (kt + 1 < n_kt) gload(kt + 1);

        const int kv0 = kt * PF_KT;
        if (wave_active && kv0 <= wave_lim) {
            // ---- S^T tile (64 tokens x 32 queries) in two 32-token halves
            f32x16 st[2];
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
#pragma unroll
                for (int y = 0; y < 16; y++) st[mt][y] = 0.0f;
                const uint16_t* kr = &Ks[(32 * mt + ql32) * PF_KPITCH + 8 * h2];
#pragma unroll
                for (int kk = 0; kk < 8; kk++) {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(kr + 16 * kk);
                    st[mt] = mfma32x32x16<T>(a, qb[kk], st[mt]);
                }
            }
            // ---- scale, mask, running max
            const bool need_mask = kv0 + PF_KT - 1 > wave_min_lim;
            const int tl = lim - kv0 - 4 * h2;  // token offset 32mt + 8i + j visible iff <= tl
            float tmax = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        float v = st[mt][4 * i + j] * scale_log2;
                        if (need_mask && (32 * mt + 8 * i + j > tl)) v = -INFINITY;
                        st[mt][4 * i + j] = v;
                        tmax = fmaxf(tmax, v);
                    }
            tmax = fmaxf(tmax, wave_shfl_xor(tmax, 32));
            const float m_new = fmaxf(m, tmax);
            const float alpha = fast_exp2(m - m_new);
            float psum = 0.0f;
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int y = 0; y < 16; y++) {
                    const float p = fast_exp2(st[mt][y] - m_new);
                    st[mt][y] = p;
                    psum += p;
                }
            lsum = lsum * alpha + psum;
            if (__builtin_amdgcn_ballot_w64(m_new > m) != 0) {
#pragma unroll
                for (int x = 0; x < 4; x++) o[x] *= alpha;
            }
            m = m_new;

            // ---- P^T B operands: kk2 covers tokens of half kk2/2, rows i = 2(kk2&1), +1
            u32x4 pb[4], pl[4];
#pragma unroll
            for (int kk2 = 0; kk2 < 4; kk2++) {
                const int mt = kk2 >> 1, y0 = 8 * (kk2 & 1);
#pragma unroll
                for (int x = 0; x < 4; x++) {
                    const float a0 = st[mt][y0 + 2 * x], a1 = st[mt][y0 + 2 * x + 1];
                    const uint32_t hi = pack2<T>(a0, a1);
                    pb[kk2][x] = hi;
                    if (PRECISE_P) pl[kk2][x] = pack2<T>(a0 - lo_f32<T>(hi), a1 - hi_f32<T>(hi));
                }
            }
            // ---- O^T += V^T P^T
#pragma unroll
            for (int mt2 = 0; mt2 < 4; mt2++) {
                const uint16_t* vr = &Vt[(32 * mt2 + ql32) * PF_VPITCH + 8 * h2];
#pragma unroll
                for (int kk2 = 0; kk2 < 4; kk2++) {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(vr + 16 * kk2);
                    o[mt2] = mfma32x32x16<T>(a, pb[kk2], o[mt2]);
                    if (PRECISE_P) o[mt2] = mfma32x32x16<T>(a, pl[kk2], o[mt2]);
                }
            }
        }
        __syncthreads();
    }

    // ---- epilogue: lane (h2, q) holds dims 32 mt2 + 8 i + 4 h2 + j of query row wr0 + q
    lsum += wave_shfl_xor(lsum, 32);
    const int orow = wr0 + ql32;
    if (!wave_active || orow >= ql) return;
    const float inv = 1.0f / lsum;
    TO* op = out + (int64_t)(q0 + orow) * o_st + (int64_t)head * o_sh + 4 * h2;
#pragma unroll
    for (int mt2 = 0; mt2 < 4; mt2++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            TO* dst = op + 32 * mt2 + 8 * i;
            const float a0 = o[mt2][4 * i] * inv, a1 = o[mt2][4 * i + 1] * inv;
            const float a2 = o[mt2][4 * i + 2] * inv, a3 = o[mt2][4 * i + 3] * inv;
            if constexpr (sizeof(TO) == 4) {
                *reinterpret_cast<f32x4*>(dst) = f32x4{a0, a1, a2, a3};
            } else {
                *reinterpret_cast<u32x2*>(dst) = u32x2{pack2<TO>(a0, a1), pack2<TO>(a2, a3)};
            }
        }
}

template <typename T, typename TO, bool PRECISE>
static int launch_prefill_mfma(void* out, int64_t o_st, int64_t o_sh, const void* q,
                               int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool,
                               const int32_t* cu, const int32_t* kv_lens, const int32_t* bt,
                               int max_blocks, int num_seqs, int max_seqlen_q, int num_heads,
                               int n_rep, int block_size, int64_t num_slots, float scale,
                               hipStream_t stream) {
    const int64_t n_qt = (max_seqlen_q + PF_QT - 1) / PF_QT;
    const int64_t grid = n_qt * num_seqs * num_heads;
    if (grid > 0x7fffffff) {
        set_error("varlen_prefill: grid too large");
        return FLOUR_ERR_UNSUPPORTED;
    }
    if (grid == 0) return FLOUR_OK;
    varlen_prefill_mfma_kernel<T, TO, PRECISE><<<dim3((unsigned)grid), dim3(PF_THREADS), 0, stream>>>(
        static_cast<TO*>(out), o_st, o_sh, static_cast<const T*>(q), q_st, q_sh,
        static_cast<const T*>(k_pool), static_cast<const T*>(v_pool), cu, kv_lens, bt, max_blocks,
        num_seqs, num_heads, n_rep, block_size, num_slots, scale * PF_LOG2E);
    return check_hip(hipGetLastError(), "varlen_prefill launch");
}

// Precision mode of the P.V product on the MFMA path (1 = hi + lo split, 0 = single rounding).
static int g_prefill_precise = 1;

}  // namespace flour

using namespace flour;

extern "C" int flour_hip_set_prefill_precise_p(int on) {
    g_prefill_precise = on ? 1 : 0;
    return FLOUR_OK;
}

extern "C" int flour_hip_varlen_prefill(void* out, int out_dtype, int64_t o_stride_tok,
                                        int64_t o_stride_head, const void* q,
                                        int64_t q_stride_tok, int64_t q_stride_head,
                                        const void* k_pool, const void* v_pool,
                                        const int32_t* cu_seqlens_q, const int32_t* kv_lens,
                                        const int32_t* block_tables, int max_blocks_per_seq,
                                        int num_seqs, int max_seqlen_q, int total_q,
                                        int num_heads, int kv_heads, int head_dim, int block_size,
                                        int64_t num_slots, float scale, int dtype, void* stream) {
    clear_error();
    if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) {
        set_error("varlen_prefill: unknown dtype (%d, out %d)", dtype, out_dtype);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (num_seqs < 0 || total_q < 0 || max_seqlen_q < 0 || num_heads <= 0 || kv_heads <= 0 ||
        num_heads % kv_heads != 0 || head_dim <= 0 || block_size <= 0 || num_slots <= 0 ||
        max_blocks_per_seq <= 0) {
        set_error("varlen_prefill: bad shape (seqs=%d total_q=%d max_q=%d heads=%d kv_heads=%d "
                  "head_dim=%d bs=%d max_blocks=%d)",
                  num_seqs, total_q, max_seqlen_q, num_heads, kv_heads, head_dim, block_size,
                  max_blocks_per_seq);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (num_seqs == 0 || total_q == 0) return FLOUR_OK;
    if (!out || !q || !k_pool || !v_pool || !cu_seqlens_q || !kv_lens || !block_tables) {
        set_error("varlen_prefill: null pointer");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int n_rep = num_heads / kv_heads;
    const int es = elem_bytes(dtype);
    const int oes = elem_bytes(out_dtype);
    const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)k_pool % 16 == 0) &&
                         ((uintptr_t)v_pool % 16 == 0) && ((q_stride_tok * es) % 16 == 0) &&
                         ((q_stride_head * es) % 16 == 0) && ((uintptr_t)out % 16 == 0) &&
                         ((o_stride_tok * oes) % 16 == 0) && ((o_stride_head * oes) % 16 == 0);
    const bool mfma = (dtype == FLOUR_DTYPE_BF16 || dtype == FLOUR_DTYPE_F16) &&
                      head_dim == PF_D && block_size % 16 == 0 && aligned;
    if (!mfma) {
        return launch_attn_generic(dtype, out_dtype, out, o_stride_tok, o_stride_head, q,
                                   q_stride_tok, q_stride_head, k_pool, v_pool, cu_seqlens_q,
                                   kv_lens, block_tables, max_blocks_per_seq, num_seqs, total_q,
                                   num_heads, n_rep, head_dim, block_size, num_slots, scale, s);
    }
#define FLOUR_PF(T, TO)                                                                          \
    return g_prefill_precise                                                                     \
               ? launch_prefill_mfma<T, TO, true>(out, o_stride_tok, o_stride_head, q,           \
                                                  q_stride_tok, q_stride_head, k_pool, v_pool,   \
                                                  cu_seqlens_q, kv_lens, block_tables,           \
                                                  max_blocks_per_seq, num_seqs, max_seqlen_q,    \
                                                  num_heads, n_rep, block_size, num_slots,       \
                                                  scale, s)                                      \
               : launch_prefill_mfma<T, TO, false>(out, o_stride_tok, o_stride_head, q,          \
                                                   q_stride_tok, q_stride_head, k_pool, v_pool,  \
                                                   cu_seqlens_q, kv_lens, block_tables,          \
                                                   max_blocks_per_seq, num_seqs, max_seqlen_q,   \
                                                   num_heads, n_rep, block_size, num_slots,      \
                                                   scale, s)
    if (dtype == FLOUR_DTYPE_BF16) {
        if (out_dtype == FLOUR_DTYPE_F32) FLOUR_PF(bf16_t, float);
        if (out_dtype == FLOUR_DTYPE_BF16) FLOUR_PF(bf16_t, bf16_t);
        FLOUR_PF(bf16_t, f16_t);
    }
    if (out_dtype == FLOUR_DTYPE_F32) FLOUR_PF(f16_t, float);
    if (out_dtype == FLOUR_DTYPE_BF16) FLOUR_PF(f16_t, bf16_t);
    FLOUR_PF(f16_t, f16_t);
#undef FLOUR_PF
}
