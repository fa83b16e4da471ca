// paged_decode.hip — kernel (2): paged decode attention on gfx950 matrix cores.
//
// Replaces paged_attention (src/backend/cpu.rs:57-112) for one new query per sequence
// (seq_q == 1, the decode step engine.rs:259-262), batched over sequences. The block list of
// Cache::kv_blocks (cache.rs:456-458, KvCache::gather_blocks cache.rs:83-96) arrives as a
// block table; query head h reads kv head h / n_rep (repeat_kv, cpu.rs:5-13); with seq_q == 1
// the causal mask of cpu.rs:88-95 admits every cached position, so only positions past the
// context length are masked.
//
// Work decomposition (stream-K at wave granularity): the K/V to read is the list of 32-token
// chunks of every (sequence, kv head) pair, laid end to end. One resident round of one-wave
// workgroups (3 per CU) each takes an equal contiguous range of that list, so every
// wave streams the same number of bytes whatever the spread of context lengths, and no wave
// pays a launch or a ramp-up twice. A pair wholly inside one range is finished by its wave; a
// pair cut by range ends leaves one partial (max, sum, acc) row per piece, and a small second
// kernel on the same stream merges those (log-sum-exp merge, as in the running update of
// cpu.rs:96-105). The kernel boundary orders partial writes before merge reads; an in-kernel
// "last workgroup merges" scheme would need an agent-scope release/acquire per workgroup,
// which on this multi-XCD part writes back and invalidates the XCD's L2 each time.
//
// Inside a piece (bf16/f16 pools, head_dim 128 or 64, block_size a multiple of 16; the
// figures below are for head_dim 128, and head_dim 64 halves every row: 8-byte lane loads, a
// 128-byte row per 16 lanes, 16 output dims per lane instead of 32):
//  * The wave walks its piece chunk by chunk. A chunk is two 16-token MFMA tiles, each one
//    4 KB (head, 16 slots) pool run of K and of V, read with buffer loads (per-pool resource,
//    loop-invariant lane offset, per-tile SGPR offset; non-temporal, whole rows per
//    instruction; K is turned into the MFMA layout through LDS); two register buffers
//    ping-pong so the next chunk's loads are in flight while one is computed, with the loop
//    peeled so that no load is conditional. Every query head of the kv head shares each K/V
//    load (GQA reuse: K/V leave HBM once).
//  * Scores S = K Q^T on v_mfma_f32_16x16x32 (M = 16 tokens, N = 16 query-head columns, the
//    n_rep real heads padded with zero rows): lane (g, c) = (lane/16, lane%16) holds head c's
//    scores for tokens 4g..4g+3 of each tile.
//  * Those registers, for the two tiles, are exactly the B operand of v_mfma_f32_16x16x32 for
//    O^T = V^T P^T (K = the 32 tokens), so P never leaves the lane. The V^T A operand is built
//    in-lane: each lane loads V rows 4g..4g+3, dims 8c..8c+7 (a wave reads 4 whole 256 B rows
//    per instruction) and v_perm_b32 packs, per output dim 8c+n, the four tokens' values. The
//    O^T accumulator holds, in lane (g, c), query head c at dims 32g..32g+31.
//  * P is split into hi + lo 16-bit parts (two MFMAs per product) so the P.V contraction keeps
//    ~16 mantissa bits of P; products are exact in fp32 and accumulate in fp32.
//  * Online softmax in the exp2 domain: the only cross-lane step per chunk is the max over the
//    four row groups (two v_permlane*_swap exchanges); running sums stay lane-partial until
//    the end, and the accumulator is rescaled only when some lane's max moved.
#include <math.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "flour_common.h"

namespace flour {

bool simt_supported(int dtype, int head_dim, const void* q, int64_t q_st, int64_t q_sh,
                    const void* k_pool, const void* v_pool);
int launch_attn_simt(int dtype, int out_dtype, void* out, int64_t o_st, int64_t o_sh,
                     const void* q, int64_t q_st, int64_t q_sh, const void* k_pool,
                     const void* v_pool, const int32_t* cu, const int32_t* kv_lens,
                     const int32_t* bt, int max_blocks, int num_seqs, int total_q, int num_heads,
                     int n_rep, int head_dim, int block_size, int64_t num_slots, int max_kv,
                     float scale, hipStream_t stream);
int launch_attn_generic(int dtype, int out_dtype, void* out, int64_t o_st, int64_t o_sh,
                        const void* q, int64_t q_st, int64_t q_sh, const void* k_pool,
                        const void* v_pool, const int32_t* cu, const int32_t* kv_lens,
                        const int32_t* bt, int max_blocks, int num_seqs, int total_q,
                        int num_heads, int n_rep, int head_dim, int block_size, int64_t num_slots,
                        int max_kv, float scale, hipStream_t stream);

static constexpr float LOG2E = 1.4426950408889634f;

static constexpr int DEC_CHUNK = 32;         // tokens per step (two 16-token MFMA tiles)
static constexpr int DEC_SEG = 32;           // chunks per tile-slot refill (64 tiles, one per lane)
static constexpr int DEC_MAX_BATCH = 4096;   // per-sequence chunk prefix sums live in LDS
// Three waves per CU. Each wave keeps one 32-token chunk in flight while it computes the
// previous one (16 KB at head_dim 128), so 768 waves hold ~12 MB of reads, about HBM's
// bandwidth-delay product; more waves only lengthen the queues and open more DRAM rows at once
// on the random 4 KB page runs (measured on the Llama-3-8B / 70B / Qwen2.5-0.5B decode batches:
// 3 per CU stream 0.3-1.5% faster than 4, which stream 3-7% faster than 8; counts that do not
// divide evenly over a CU's 4 SIMDs, 2.5, 3.5 and 5 per CU, are slower than their neighbours).
static constexpr int DEC_WAVES_PER_CU = 3;
// K is read like V, four whole 256 B rows per instruction with the non-temporal hint, and
// turned into the MFMA A-operand layout (row = lane % 16) through a per-wave LDS tile. Reading
// K directly in that layout takes a 64 B quarter of 16 rows per instruction, a pattern that
// streams at most ~6.0 TB/s from HBM against ~6.8 TB/s for whole rows (measured with the same
// 2048-wave, double-buffered access over random 4 KB runs).
// Bytes per K row in LDS (head_dim 128 / 64): conflict-free 16-byte fragment reads of 16 rows.
__host__ __device__ constexpr int dec_kpitch(int d) { return d == 128 ? 272 : 144; }

struct DecodeWs {
    float* ml;  // [2 * num_waves][n_rep][2] (max, sum) in the exp2 domain
    float* o;   // [2 * num_waves][n_rep][D]
    int* pre;   // [batch + 1] chunk prefix sums, written by workgroup 0 for the merge kernel
    // row of q / out that batch entry b reads and writes: rows[b], or b when null (a mixed
    // continuous-batching step runs its one-row sequences, scattered among the packed rows of
    // longer ones, as one decode batch)
    const int32_t* rows;
    // Decode step of a batch with its KV write fused in (the kernel's FUSE instantiation): the
    // new K / V row of entry b and kv head g at k_new / v_new + b * new_st + g * new_sh
    // (elements), written to pool slot new_slots[b] (skipped outside [0, num_slots)) before the
    // attention reads it.
    const void* k_new;
    const void* v_new;
    int64_t new_st, new_sh;
    const int32_t* new_slots;
    int xcd_w;  // wave-range weight w (WaveRanges): even ranges 32 + w, odd 32 - w
};

static int g_wg_override = 0;  // tuning / test hook: number of waves (0 = one resident round)
// Wave-range weight w of WaveRanges (0 .. 16): even-indexed ranges (even XCDs) take w/32 more
// chunks than the mean, odd ones w/32 fewer (a tuning / test switch). Same-box sweep of w = 0 ..
// 4: 2 is best or even on every decode workload (Llama-3-8B batch 5,862 -> 5,989 GB/s, 70B
// batch 6,083 -> 6,231, head_dim-64 batch even).
static int g_xcd_weight = 2;

static int device_cus() {
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

static int decode_workgroups() {
    const int n = g_wg_override > 0 ? g_wg_override : device_cus() * DEC_WAVES_PER_CU;
    return n < 4096 ? n : 4096;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static size_t decode_ws_bytes(int nwg, int n_rep, int head_dim, int batch) {
    const size_t slots = 2 * (size_t)nwg;
    return align256(slots * n_rep * 2 * sizeof(float)) +
           align256(slots * n_rep * (size_t)head_dim * sizeof(float)) +
           align256(((size_t)batch + 1) * sizeof(int));
}

__device__ __forceinline__ int decode_chunks(int ctx, int max_ctx) {
    ctx = min(ctx, max_ctx);
    return ctx > 0 ? (ctx + DEC_CHUNK - 1) / DEC_CHUNK : 0;
}

// Wave ranges over the flattened chunk list. The dispatcher places workgroup i on XCD i % 8,
// and on this path the odd XCDs stream 6-9% slower than their even partners (per-workgroup
// clock stamps: every pair, three machines, both head shapes), so the launch would wait for the
// odd half. Even-indexed ranges therefore hold w/32 more chunks than the mean and odd ones w/32
// fewer: range i is [lo(i), lo(i + 1)) with lo(i) = floor(total (32 i + w (i & 1)) / W),
// W = 32 n + w (n & 1), so lo(0) = 0 and lo(n) = total. The split depends on the shapes alone,
// never on timing, so results stay deterministic. I is uint32_t when total * (W + 32) fits 32
// bits (a 64-bit division is a long instruction sequence), else int64_t.
template <typename I>
struct WaveRanges {
    I total, n, w, W;
    __device__ WaveRanges(int64_t total_, int64_t n_, int w_)
        : total((I)total_), n((I)n_), w((I)w_), W((I)(32 * n_ + w_ * (n_ & 1))) {}
    __device__ I lo(I i) const { return total * (32 * i + w * (i & 1)) / W; }
    // the range holding chunk x (0 <= x < total): the last i < n with lo(i) <= x (the estimate
    // is within a range or two of it, as no range differs from the mean by more than w/32)
    __device__ I owner(I x) const {
        I i = x * W / (32 * total);
        if (i > n - 1) i = n - 1;
        while (i + 1 < n && lo(i + 1) <= x) i++;
        while (i > 0 && lo(i) > x) i--;
        return i;
    }
};

// One wave per workgroup; each wave owns one contiguous range of the chunk list. D is the head
// dim, 128 or 64. A lane's K/V share of a 16-token tile is rows 4lg .. 4lg + 3 at 16-byte
// (D 128: dims 8lc ..) or 8-byte (D 64: dims 4lc ..) width, so a wave reads whole rows.
template <typename T, typename TO, bool BS16, int D, bool FUSE>
__global__ __launch_bounds__(64, 2) void paged_decode_mfma_kernel(
    TO* __restrict__ out, const T* __restrict__ q, const T* __restrict__ k_pool,
    const T* __restrict__ v_pool, const int32_t* __restrict__ block_tables, int max_blocks,
    const int32_t* __restrict__ context_lens, int batch, int num_heads, int kv_heads, int n_rep,
    int block_size, int64_t num_slots, int max_ctx, float scale_log2, DecodeWs ws) {
    static_assert(D == 128 || D == 64, "matrix-core decode: head_dim 128 or 64");
    constexpr int KP = dec_kpitch(D);
    constexpr int NV = D / 16;  // O^T products per chunk (16 output dims each)
    // a lane's load of one row: 8 (D 128) or 4 (D 64) dims
    typedef typename std::conditional<D == 128, u32x4, u32x2>::type Ld;
    extern __shared__ int pre[];  // pre[b] = chunks of sequences 0..b-1; pre[batch] = all
    __shared__ __attribute__((aligned(16))) unsigned char kt[16 * KP];  // one K tile
    const int lane = threadIdx.x, lg = lane >> 4, lc = lane & 15;

    // ---- exclusive prefix sum of per-sequence chunk counts (each lane scans a slice)
    {
        const int per = (batch + 63) / 64;
        int local = 0;
        for (int i = 0; i < per; i++) {
            const int b = lane * per + i;
            if (b < batch) local += decode_chunks(context_lens[b], max_ctx);
        }
        const int incl = wave_incl_sum(local);
        int run = incl - local;
        for (int i = 0; i < per; i++) {
            const int b = lane * per + i;
            if (b < batch) {
                pre[b] = run;
                run += decode_chunks(context_lens[b], max_ctx);
            }
        }
        if (lane == 63) pre[batch] = incl;
        __syncthreads();
        if (blockIdx.x == 0)  // for the merge kernel (ordered by the kernel boundary)
            for (int b = lane; b <= batch; b += 64) ws.pre[b] = pre[b];
    }
    const int64_t total = (int64_t)kv_heads * pre[batch];
    const int64_t nwg = gridDim.x, wgi = blockIdx.x;
    const WaveRanges<int64_t> wr(total, nwg, ws.xcd_w);
    const int64_t lo = wr.lo(wgi), hi = wr.lo(wgi + 1);

    if (lo >= hi) return;

    const uint32_t head_bytes = (uint32_t)(num_slots * D * (int64_t)sizeof(T));
    // K and V: instruction j of a tile reads rows 4lg + j, dims (D / 16) lc .. (4 whole rows)
    const uint32_t v_off = (uint32_t)((4 * lg * D + (D / 16) * lc) * sizeof(T));
    const int64_t max_phys = num_slots / block_size - 1;

    // The wave's range is a stream of segments: up to DEC_SEG consecutive chunks of one
    // (sequence, kv head) pair. Consecutive segments of the same pair form one piece.
    struct Seg {
        int b, g, cb, ce, nch, tok_end;
    };
    auto seg_at = [&](int64_t x) -> Seg {
        int l0 = 0, h0 = batch;  // largest b with kv_heads * pre[b] <= x
        while (h0 - l0 > 1) {
            const int mid = (l0 + h0) >> 1;
            if ((int64_t)kv_heads * pre[mid] <= x)
                l0 = mid;
            else
                h0 = mid;
        }
        Seg sg;
        sg.b = l0;
        sg.nch = pre[l0 + 1] - pre[l0];
        const int64_t rel = x - (int64_t)kv_heads * pre[l0];
        sg.g = (int)(rel / sg.nch);
        sg.cb = (int)(rel - (int64_t)sg.g * sg.nch);
        sg.ce = (int)min(min((int64_t)sg.nch, (int64_t)sg.cb + DEC_SEG), sg.cb + (hi - x));
        sg.tok_end = min(min(context_lens[sg.b], max_ctx), sg.ce * DEC_CHUNK);
        return sg;
    };
    // Pool slot of the first token of each tile of a segment: lane i holds tile i (chunk
    // cb + i/2, half i%2), so the loop fetches it with v_readlane. Tiles past the segment are
    // clamped to its last tile: every address stays valid, their tokens are masked and their V
    // zeroed in compute_chunk.
    // The block id is kept as loaded and clamped only where a tile load reads it (one segment
    // later for the next segment): using it here would make the wave wait for this load, and
    // with it for every chunk load in flight.
    struct Slots {
        int id, off;  // lane i: block id and in-block offset of tile i's first token
    };
    const int max_id = (int)max_phys;
    auto seg_slots = [&](const Seg& sg) -> Slots {
        const int32_t* bt = block_tables + (int64_t)sg.b * max_blocks;
        const int last_tile_tok0 = ((sg.tok_end - 1) >> 4) << 4;
        const int tok0 = min(sg.cb * DEC_CHUNK + lane * 16, last_tile_tok0);
        const int lb = BS16 ? (tok0 >> 4) : tok0 / block_size;
        return Slots{bt[lb], tok0 - lb * block_size};
    };
    // Chunk loads as buffer loads: one resource per pool (the kv head's region), the
    // loop-invariant lane offset (VGPR) and the tile's byte offset (SGPR), so there is no
    // per-lane address arithmetic in the loop; non-temporal (K/V are read exactly once);
    // an out-of-region offset reads zeros instead of faulting.
    auto load_chunk = [&](int g, Slots sl, int tile0, Ld (*kd)[4], Ld (*vd)[4]) {
        const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(k_pool + (int64_t)g * num_slots * D), (short)0, (int)head_bytes, BUF_DWORD3);
        const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(v_pool + (int64_t)g * num_slots * D), (short)0, (int)head_bytes, BUF_DWORD3);
#pragma unroll
        for (int t = 0; t < 2; t++) {
            int id = __builtin_amdgcn_readlane(sl.id, tile0 + t);
            id = id < 0 ? 0 : (id > max_id ? max_id : id);  // a bad block id never leaves the pool
            const uint32_t soff =
                (uint32_t)(id * block_size + __builtin_amdgcn_readlane(sl.off, tile0 + t)) *
                (uint32_t)(D * sizeof(T));
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if constexpr (D == 128)
                    kd[t][j] = __builtin_amdgcn_raw_buffer_load_b128(
                        k_rsrc, v_off + j * D * (uint32_t)sizeof(T), soff, BUF_NT);
                else
                    kd[t][j] = __builtin_amdgcn_raw_buffer_load_b64(
                        k_rsrc, v_off + j * D * (uint32_t)sizeof(T), soff, BUF_NT);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if constexpr (D == 128)
                    vd[t][j] = __builtin_amdgcn_raw_buffer_load_b128(
                        v_rsrc, v_off + j * D * (uint32_t)sizeof(T), soff, BUF_NT);
                else
                    vd[t][j] = __builtin_amdgcn_raw_buffer_load_b64(
                        v_rsrc, v_off + j * D * (uint32_t)sizeof(T), soff, BUF_NT);
            }
        }
    };
    // Q^T as the B operand: lane (lg, lc) holds head lc, dims 32kk + 8lg .. +7.
    u32x4 qb[D / 32];
    auto load_q = [&](int b, int g) {
        const int64_t row = ws.rows ? (int64_t)ws.rows[b] : (int64_t)b;
        const T* qh = q + (row * num_heads + (int64_t)g * n_rep + lc) * D + 8 * lg;
#pragma unroll
        for (int kk = 0; kk < D / 32; kk++)
            qb[kk] = (lc < n_rep) ? *reinterpret_cast<const u32x4*>(qh + 32 * kk) : u32x4{0, 0, 0, 0};
    };

    float m = -INFINITY, lsum = 0.0f;
    f32x4 acc[NV];
#pragma unroll
    for (int nn = 0; nn < NV; nn++) acc[nn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute_chunk = [&](int c, int tok_end, Ld (*ka)[4], Ld (*va)[4]) {
        const int tok0 = c * DEC_CHUNK;
        const bool full = tok0 + DEC_CHUNK <= tok_end;
        if (!full) {  // tokens past the context: zero V so garbage bits cannot leak in
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (tok0 + 16 * t + 4 * lg + j >= tok_end) va[t][j] = Ld{};
        }
        // K rows through LDS into the A-operand layout: lane (lg, lc) needs row lc, dims
        // 32kk + 8lg .. +7. One wave per workgroup and LDS operations of a wave complete in
        // order, so the wave barriers only keep the compiler from moving LDS accesses across.
        // The second tile's writes follow the first tile's reads in that order.
        u32x4 kA[2][D / 32];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int j = 0; j < 4; j++)
                *reinterpret_cast<Ld*>(&kt[(4 * lg + j) * KP + (int)sizeof(Ld) * lc]) = ka[t][j];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int kk = 0; kk < D / 32; kk++)
                kA[t][kk] = *reinterpret_cast<const u32x4*>(&kt[lc * KP + 64 * kk + 16 * lg]);
        }
        __builtin_amdgcn_wave_barrier();
        // S tiles: s[t][r] = score of head lc for token 16t + 4lg + r of the chunk.
        f32x4 s[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            s[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kk = 0; kk < D / 32; kk++) s[t] = mfma16x16x32<T>(kA[t][kk], qb[kk], s[t]);
        }
        float sv[8];
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const bool ok = full || (tok0 + 16 * t + 4 * lg + r < tok_end);
                sv[4 * t + r] = ok ? s[t][r] * scale_log2 : -INFINITY;
                tmax = fmaxf(tmax, sv[4 * t + r]);
            }
        tmax = max_across_rows(tmax);
        const float m_new = fmaxf(m, tmax);
        const float alpha = fast_exp2(m - m_new);
        float p[8];
#pragma unroll
        for (int i = 0; i < 8; i++) p[i] = fast_exp2(sv[i] - m_new);
        lsum = lsum * alpha +
               (((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])));
        if (__builtin_amdgcn_ballot_w64(m_new > m) != 0) {
#pragma unroll
            for (int nn = 0; nn < NV; nn++) acc[nn] *= alpha;
        }
        m = m_new;
        // P^T as the B operand over the 32 tokens: lane (lg, lc) holds head lc at
        // k-slots 8lg + j: j < 4 -> token 4lg + j (tile 0), j >= 4 -> 16 + 4lg + j - 4.
        // Split hi + lo so the product keeps ~16 mantissa bits of P.
        u32x4 PH, PL;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t hi16 = pack2<T>(p[2 * i], p[2 * i + 1]);
            PH[i] = hi16;
            PL[i] = pack2<T>(p[2 * i] - lo_f32<T>(hi16), p[2 * i + 1] - hi_f32<T>(hi16));
        }
        // V^T as the A operand: lane (lg, lc) holds output dim (D / 16) lc + nn at the same
        // k-slots, packed in-lane from its four V rows of each tile.
#pragma unroll
        for (int nn = 0; nn < NV; nn++) {
            const int wd = nn >> 1;
            u32x4 A;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                if (nn & 1) {
                    A[2 * t] = perm_hi16(va[t][0][wd], va[t][1][wd]);
                    A[2 * t + 1] = perm_hi16(va[t][2][wd], va[t][3][wd]);
                } else {
                    A[2 * t] = perm_lo16(va[t][0][wd], va[t][1][wd]);
                    A[2 * t + 1] = perm_lo16(va[t][2][wd], va[t][3][wd]);
                }
            }
            acc[nn] = mfma16x16x32<T>(A, PH, acc[nn]);
            acc[nn] = mfma16x16x32<T>(A, PL, acc[nn]);
        }
    };

    // Piece epilogue from registers: lane (lg, lc) holds head lc, dims (D / 4) lg + NV r + nn
    // (r < 4, nn < NV): D / 4 contiguous dims.
    auto epilogue = [&](int b, int g, bool complete, bool first_piece) {
        lsum = sum_across_rows(lsum);
        // FUSE: lg made opaque here, so the per-lane output addresses are formed at the store
        // instead of being hoisted out of the stream as 64-bit values (which spill in that
        // instantiation, and a spill reload waits for every chunk load in flight)
        int lgo = lg;
        if constexpr (FUSE) asm volatile("" : "+v"(lgo));
        if (lc < n_rep) {
            if (complete) {  // whole pair in this range: final output
                const int64_t row = ws.rows ? (int64_t)ws.rows[b] : (int64_t)b;
                TO* o = out + (row * num_heads + (int64_t)g * n_rep + lc) * D + (D / 4) * lgo;
                const float inv = 1.0f / lsum;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    if constexpr (sizeof(TO) == 4) {
#pragma unroll
                        for (int h4 = 0; h4 < NV; h4 += 4)
                            *reinterpret_cast<f32x4*>(o + NV * r + h4) =
                                f32x4{acc[h4][r] * inv, acc[h4 + 1][r] * inv, acc[h4 + 2][r] * inv,
                                      acc[h4 + 3][r] * inv};
                    } else {
                        uint32_t v[NV / 2];
#pragma unroll
                        for (int i = 0; i < NV / 2; i++)
                            v[i] = pack2<TO>(acc[2 * i][r] * inv, acc[2 * i + 1][r] * inv);
                        if constexpr (NV == 8)
                            *reinterpret_cast<u32x4*>(o + NV * r) = u32x4{v[0], v[1], v[2], v[3]};
                        else
                            *reinterpret_cast<u32x2*>(o + NV * r) = u32x2{v[0], v[1]};
                    }
                }
            } else {  // partial row for the merge kernel
                const int64_t pidx = (2 * wgi + (first_piece ? 0 : 1)) * n_rep + lc;
                float* o = ws.o + pidx * D + (D / 4) * lgo;
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int h4 = 0; h4 < NV; h4 += 4)
                        *reinterpret_cast<f32x4*>(o + NV * r + h4) =
                            f32x4{acc[h4][r], acc[h4 + 1][r], acc[h4 + 2][r], acc[h4 + 3][r]};
                if (lg == 0) {
                    ws.ml[2 * pidx] = m;
                    ws.ml[2 * pidx + 1] = lsum;
                }
            }
        }
        m = -INFINITY;
        lsum = 0.0f;
#pragma unroll
        for (int nn = 0; nn < NV; nn++) acc[nn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };

    // ---- the chunk stream. The next segment's block-table slots are read while the current
    // one streams, and the two register buffers ping-pong across segment and piece boundaries:
    // the next chunk's loads (chosen with uniform selects, never a branch, so the compiler's
    // wait counts stay exact) are in flight while the current chunk is computed and while a
    // finished piece is written out.
    // FUSE: the new K / V row of every pair whose last chunk lies in this wave's range, written
    // to the pool before the range's first chunk load. The lanes that write a row, (lg, lc) with
    // 4 lg <= slot % 16 < 4 lg + 4 (the row's place in its 16-token tile, as the block table
    // places position context_len - 1), are the lanes that load it back in load_chunk, at the
    // same bytes (dims (D / 16) lc ..), so the wave's own program order makes the later load see
    // the row. No other wave reads the slot: the pair's last chunk, the only one holding the
    // new position, is in this range alone, and a batch's new slots are private to their
    // sequences. The first two pairs' rows are requested before the block-table and q loads
    // (their wait then overlaps those loads), stored after them; further pairs (short contexts)
    // two at a time after that.
    struct NewRows {
        int b, g, slot[2], pb[2], pg[2];
        bool pv[2], more;
        int64_t first;
        int nch;
        Ld kr[2], vr[2];
    };
    auto new_rows_load = [&](NewRows& nr) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            nr.pv[i] = nr.more;
            nr.pb[i] = nr.b;
            nr.pg[i] = nr.g;
            if (nr.more) {  // on to the next pair in the flattened order (sequences with chunks)
                nr.first += nr.nch;
                if (++nr.g == kv_heads) {
                    nr.g = 0;
                    do {
                        nr.b++;
                    } while (nr.b < batch && pre[nr.b + 1] == pre[nr.b]);
                }
                if (nr.b < batch) {
                    nr.nch = pre[nr.b + 1] - pre[nr.b];
                    nr.more = nr.first + nr.nch - 1 < hi;
                } else {
                    nr.more = false;
                }
            }
        }
        const T* kn = static_cast<const T*>(ws.k_new);
        const T* vn = static_cast<const T*>(ws.v_new);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            nr.slot[i] = nr.pv[i] ? ws.new_slots[nr.pb[i]] : -1;
            if (nr.pv[i]) {
                const int64_t src = (int64_t)nr.pb[i] * ws.new_st + (int64_t)nr.pg[i] * ws.new_sh +
                                    (D / 16) * lc;
                nr.kr[i] = *reinterpret_cast<const Ld*>(kn + src);
                nr.vr[i] = *reinterpret_cast<const Ld*>(vn + src);
            }
        }
    };
    auto new_rows_store = [&](const NewRows& nr) {
        T* const kpw = const_cast<T*>(k_pool);
        T* const vpw = const_cast<T*>(v_pool);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int sl = nr.slot[i];
            if (nr.pv[i] && sl >= 0 && sl < num_slots && lg == ((sl & 15) >> 2)) {
                const int64_t dst = ((int64_t)nr.pg[i] * num_slots + sl) * D + (D / 16) * lc;
                *reinterpret_cast<Ld*>(kpw + dst) = nr.kr[i];
                *reinterpret_cast<Ld*>(vpw + dst) = nr.vr[i];
            }
        }
    };

    Seg cur = seg_at(lo);
    NewRows nr{};
    if constexpr (FUSE) {
        nr.b = cur.b;
        nr.g = cur.g;
        nr.nch = cur.nch;
        nr.first = lo - cur.cb;  // flattened position of pair (b, g)'s first chunk
        nr.more = nr.first + nr.nch - 1 < hi;
        new_rows_load(nr);
    }
    Slots cur_slots = seg_slots(cur);
    int64_t nx = lo + (cur.ce - cur.cb);
    bool has_nxt = nx < hi;
    Seg nxt = cur;
    Slots nxt_slots = cur_slots;
    if (has_nxt) {
        nxt = seg_at(nx);
        nxt_slots = seg_slots(nxt);
    }
    int pc0 = cur.cb;  // first chunk of the current piece
    bool first_piece = true;
    int c = cur.cb;
    load_q(cur.b, cur.g);

    // One stream step: prefetch the chunk after c into (kn, vn) (PREFETCH is a compile-time
    // constant at each call, so the steady-state loop has no conditional loads), compute c
    // from (kc, vc), then advance the cursor.
    auto step = [&](auto prefetch, Ld (*kc)[4], Ld (*vc)[4], Ld (*kn)[4], Ld (*vn)[4]) {
        const bool seg_end = c + 1 >= cur.ce;
        // At a segment's last chunk the segment after the next one is looked up and its
        // block-table entries are requested before this step's chunk loads, so the rotation at
        // the end of the step waits for that load alone and not for the chunk loads behind it.
        int64_t nn_x = nx;
        bool has_nn = false;
        Seg nn = nxt;
        Slots nn_slots = nxt_slots;
        if (seg_end && has_nxt) {
            nn_x = nx + (nxt.ce - nxt.cb);
            has_nn = nn_x < hi;
            if (has_nn) {
                nn = seg_at(nn_x);
                nn_slots = seg_slots(nn);
            }
        }
        if constexpr (decltype(prefetch)::value) {
            const bool in_cur = c + 1 < cur.ce;
            const int pg = in_cur ? cur.g : nxt.g;
            const Slots pslots = in_cur ? cur_slots : nxt_slots;
            const int ptile = in_cur ? 2 * (c + 1 - cur.cb) : 0;
            load_chunk(pg, pslots, ptile, kn, vn);
        }
        compute_chunk(c, cur.tok_end, kc, vc);
        if (!seg_end) {
            c += 1;
            return;
        }
        // end of a segment
        const bool piece_end = !has_nxt || nxt.b != cur.b || nxt.g != cur.g;
        if (piece_end) epilogue(cur.b, cur.g, pc0 == 0 && cur.ce == cur.nch, first_piece);
        if (!has_nxt) return;
        if (piece_end) {
            pc0 = nxt.cb;
            first_piece = false;
            load_q(nxt.b, nxt.g);
        }
        cur = nxt;
        cur_slots = nxt_slots;
        c = cur.cb;
        nx = nn_x;
        has_nxt = has_nn;
        if (has_nn) {
            nxt = nn;
            nxt_slots = nn_slots;
        }
    };


    if constexpr (FUSE) {
        new_rows_store(nr);
        while (nr.more) {
            new_rows_load(nr);
            new_rows_store(nr);
        }
        asm volatile("" ::: "memory");  // the stores stay before the chunk loads
    }

    using pf_on = std::integral_constant<bool, true>;
    using pf_off = std::integral_constant<bool, false>;
    Ld ka[2][4], va[2][4], kb[2][4], vb[2][4];
    load_chunk(cur.g, cur_slots, 0, ka, va);
    int64_t remaining = hi - lo;  // chunks this wave computes; all but the last prefetch one
    for (; remaining > 2; remaining -= 2) {
        step(pf_on{}, ka, va, kb, vb);
        step(pf_on{}, kb, vb, ka, va);
    }
    if (remaining == 2) {
        step(pf_on{}, ka, va, kb, vb);
        step(pf_off{}, kb, vb, ka, va);
    } else {
        step(pf_off{}, ka, va, kb, vb);
    }
}

// Merge of the pieces of pairs cut by wave ranges, and zero rows for empty contexts: one wave
// per (query head, sequence), lane i owning output dims 2i and 2i + 1, locating its pieces from
// the chunk prefix sums the main kernel left in the workspace. Pieces are taken 64 at a time
// (one per lane): their (max, sum) pairs become weights through wave reductions, then every
// lane accumulates its two dims over the batch with independent loads, reading each piece's
// weight and slot from the lane that holds it; batches combine with the same online rescaling
// as the running update of cpu.rs:96-105. No LDS and no barrier.
template <typename TO, int D>
__global__ __launch_bounds__(64) void paged_decode_merge_kernel(
    TO* __restrict__ out, int batch, int num_heads, int kv_heads, int n_rep, int nwg_i,
    DecodeWs ws) {
    // lane i owns output dims E i .. E i + E - 1
    constexpr int E = D / 64;
    const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    // chunks before sequence b, of sequence b and in all sequences (the main kernel's sums)
    const int before = ws.pre[b], nch = ws.pre[b + 1] - before, all = ws.pre[batch];
    const int64_t orow = ws.rows ? (int64_t)ws.rows[b] : (int64_t)b;
    TO* o = out + (orow * num_heads + h) * D + E * lane;
    if (nch == 0) {
#pragma unroll
        for (int i = 0; i < E; i++) o[i] = from_f32<TO>(0.0f);
        return;
    }
    const int g = h / n_rep, hh = h - g * n_rep;
    const int64_t total = (int64_t)kv_heads * all, nwg = nwg_i;
    const int64_t s = (int64_t)kv_heads * before + (int64_t)g * nch;
    const int64_t e = s + nch;
    // Range owners and bounds, in 32-bit arithmetic whenever chunks x (W + 32) fits (it bounds
    // every numerator of WaveRanges), as it does at any practical size.
    const bool narrow = (uint64_t)total * (uint64_t)(32 * nwg + ws.xcd_w + 32) <= 0xffffffffull;
    const WaveRanges<uint32_t> r32(narrow ? total : 1, nwg, ws.xcd_w);
    const WaveRanges<int64_t> r64(total, nwg, ws.xcd_w);
    auto range_lo = [&](int64_t i) -> int64_t {
        return narrow ? (int64_t)r32.lo((uint32_t)i) : r64.lo(i);
    };
    const int64_t f = narrow ? (int64_t)r32.owner((uint32_t)s) : r64.owner(s);
    const int64_t l = narrow ? (int64_t)r32.owner((uint32_t)(e - 1)) : r64.owner(e - 1);
    const bool f_first = s == range_lo(f);
    if (f == l) return;  // finished inside one wave range
    const int np = (int)(l - f + 1);  // ranges f..l; empty ones wrote nothing

    float M = -INFINITY, L = 0.0f, O[E];
#pragma unroll
    for (int i = 0; i < E; i++) O[i] = 0.0f;
    const int fslot = (int)(f_first ? 2 * f : 2 * f + 1);  // the first piece always exists
    // Wave ranges can be empty only when the smallest share, (32 - w) / 32 of the mean, is below
    // one chunk; otherwise skip the range-bound divisions.
    const bool dense = total * (32 - ws.xcd_w) >= 32 * nwg + 32;
    auto piece_slot = [&](int64_t p) -> int {  // slot of piece p (< np), -1 for an empty range
        const int64_t ij = f + p;
        if (!dense && range_lo(ij) == range_lo(ij + 1)) return -1;
        return (int)((ij == f && !f_first) ? 2 * ij + 1 : 2 * ij);
    };
    typedef typename std::conditional<E == 2, f32x2, float>::type RowV;
    auto row = [&](int slot) -> RowV {  // this lane's E dims of a piece's partial row
        return *reinterpret_cast<const RowV*>(ws.o + ((int64_t)slot * n_rep + hh) * D + E * lane);
    };
    auto add = [&](float wj, RowV v) {
        if constexpr (E == 2) {
            O[0] += wj * v[0];
            O[1] += wj * v[1];
        } else {
            O[0] += wj * v;
        }
    };
    for (int p0 = 0; p0 < np; p0 += 64) {
        // The batch's first 8 pieces' rows are loaded before the (max, sum) reductions, which
        // they do not depend on (a missing piece reads the first piece's row, weight 0).
        RowV v0[8];
        int s0[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            s0[j] = p0 + j < np ? piece_slot(p0 + j) : -1;
            v0[j] = row(s0[j] >= 0 ? s0[j] : fslot);
        }
        const int slot = p0 + lane < np ? piece_slot(p0 + lane) : -1;
        float mx = -INFINITY, lx = 0.0f;
        if (slot >= 0) {
            mx = ws.ml[2 * ((int64_t)slot * n_rep + hh)];
            lx = ws.ml[2 * ((int64_t)slot * n_rep + hh) + 1];
        }
        const float m_new = fmaxf(M, wave_max(mx));
        const float w = (slot >= 0) ? fast_exp2(mx - m_new) : 0.0f;
        const float bl = wave_sum(w * lx);
        const float c_old = (M == -INFINITY) ? 0.0f : fast_exp2(M - m_new);
        L = L * c_old + bl;
#pragma unroll
        for (int i = 0; i < E; i++) O[i] *= c_old;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
            if (s0[j] >= 0) add(wj, v0[j]);
        }
        // The rest in groups of 8 unconditional loads (a missing piece reads the first piece's
        // row) so they are all in flight together; the select drops them, so stale workspace
        // bits (even NaN) never reach the sum.
        const int nb = min(64, np - p0);
        for (int q = 8; q < nb; q += 8) {
            RowV v[8];
            int sl[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                sl[j] = __builtin_amdgcn_readlane(slot, q + j);
                v[j] = row(sl[j] >= 0 ? sl[j] : fslot);
            }
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), q + j));
                if (sl[j] >= 0) add(wj, v[j]);
            }
        }
        M = m_new;
    }
#pragma unroll
    for (int i = 0; i < E; i++) o[i] = from_f32<TO>(O[i] / L);
}

template <typename T, typename TO, int D>
static int launch_decode_mfma_d(void* out, const void* q, const void* k_pool, const void* v_pool,
                                const int32_t* bt, int max_blocks, const int32_t* ctx_lens,
                                int batch, int num_heads, int kv_heads, int n_rep, int block_size,
                                int64_t num_slots, int max_ctx, float scale, int nwg, DecodeWs ws,
                                hipStream_t stream) {
    const size_t lds = (size_t)(batch + 1) * sizeof(int);
    const bool fuse = ws.k_new != nullptr;
    if (fuse && block_size != 16) {  // paged_decode_write_kv takes 16-token pages only
        set_error("paged_decode: the fused KV write needs 16-token pages");
        return FLOUR_ERR_UNSUPPORTED;
    }
    auto kern = block_size == 16 ? (fuse ? paged_decode_mfma_kernel<T, TO, true, D, true>
                                         : paged_decode_mfma_kernel<T, TO, true, D, false>)
                                 : paged_decode_mfma_kernel<T, TO, false, D, false>;
    kern<<<dim3(nwg), dim3(64), lds, stream>>>(
        static_cast<TO*>(out), static_cast<const T*>(q), static_cast<const T*>(k_pool),
        static_cast<const T*>(v_pool), bt, max_blocks, ctx_lens, batch, num_heads, kv_heads, n_rep,
        block_size, num_slots, max_ctx, scale * LOG2E, ws);
    int rc = check_hip(hipGetLastError(), "paged_decode launch");
    if (rc != FLOUR_OK) return rc;
    paged_decode_merge_kernel<TO, D><<<dim3(num_heads, batch), dim3(64), 0, stream>>>(
        static_cast<TO*>(out), batch, num_heads, kv_heads, n_rep, nwg, ws);
    return check_hip(hipGetLastError(), "paged_decode merge launch");
}

template <typename T, typename TO>
static int launch_decode_mfma(int head_dim, void* out, const void* q, const void* k_pool,
                              const void* v_pool, const int32_t* bt, int max_blocks,
                              const int32_t* ctx_lens, int batch, int num_heads, int kv_heads,
                              int n_rep, int block_size, int64_t num_slots, int max_ctx,
                              float scale, int nwg, DecodeWs ws, hipStream_t stream) {
    if (head_dim == 64)
        return launch_decode_mfma_d<T, TO, 64>(out, q, k_pool, v_pool, bt, max_blocks, ctx_lens,
                                               batch, num_heads, kv_heads, n_rep, block_size,
                                               num_slots, max_ctx, scale, nwg, ws, stream);
    return launch_decode_mfma_d<T, TO, 128>(out, q, k_pool, v_pool, bt, max_blocks, ctx_lens,
                                            batch, num_heads, kv_heads, n_rep, block_size,
                                            num_slots, max_ctx, scale, nwg, ws, stream);
}

}  // namespace flour

using namespace flour;

namespace flour {
__global__ void empty_kernel() {}
}  // namespace flour

// One empty one-wave workgroup on `stream`: the floor of a kernel launch on this device, timed
// beside the smallest decode workloads (a measurement helper, not part of the header).
extern "C" int flour_hip_empty_launch(void* stream) {
    flour::empty_kernel<<<dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream)>>>();
    return check_hip(hipGetLastError(), "empty launch");
}

extern "C" int flour_hip_set_decode_xcd_weight(int w) {
    if (w < 0 || w > 16) return FLOUR_ERR_INVALID_ARGUMENT;
    g_xcd_weight = w;
    return FLOUR_OK;
}

extern "C" int flour_hip_set_decode_workgroups(int n) {
    if (n < 0 || n > 4096) return FLOUR_ERR_INVALID_ARGUMENT;
    g_wg_override = n;
    return FLOUR_OK;
}

extern "C" int flour_hip_paged_decode_workspace_size(int batch, int num_heads, int kv_heads,
                                                     int head_dim, int max_context_len,
                                                     size_t* bytes) {
    clear_error();
    if (!bytes || batch < 0 || num_heads <= 0 || kv_heads <= 0 || num_heads % kv_heads != 0 ||
        head_dim <= 0 || max_context_len < 0) {
        set_error("paged_decode_workspace_size: bad arguments");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    *bytes = decode_ws_bytes(decode_workgroups(), num_heads / kv_heads, head_dim, batch);
    return FLOUR_OK;
}

namespace flour {

// Body of flour_hip_paged_decode. `workspace` == nullptr with `ws_from_scratch` set takes the
// split-context workspace from this device's copy of `scratch` (flour_hip_paged_decode_noalloc).
static int paged_decode_impl(void* out, int out_dtype, const void* q, const void* k_pool,
                             const void* v_pool, const int32_t* block_tables,
                             int max_blocks_per_seq, const int32_t* context_lens, int batch,
                             int num_heads, int kv_heads, int head_dim, int block_size,
                             int64_t num_slots, int max_context_len, float scale, int dtype,
                             void* workspace, size_t workspace_bytes, bool ws_from_scratch,
                             const int32_t* rows, const DecodeWs* fused, void* stream);

// ------------------------------------------------------------------ allocation-free variant
// The split-context workspace of flour_hip_paged_decode_noalloc lives in this file-scope device
// array: each device the library runs on holds its own copy, for the life of the process. Host
// code never passes the array's name to a kernel or a copy (on the host it is a stand-in, not a
// device address): it uses the per-device address that hipGetSymbolAddress returns, looked up
// once per device on that device's first call.
static constexpr size_t DEC_SCRATCH_BYTES = (size_t)40 << 20;
static __device__ __align__(256) unsigned char scratch[DEC_SCRATCH_BYTES];
static constexpr int DEC_MAX_DEVICES = 64;
static std::atomic<void*> g_scratch_ptr[DEC_MAX_DEVICES];
static std::mutex g_scratch_mu;

static int scratch_for_current_device(void** ptr) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return check_hip(e, "paged_decode_noalloc: hipGetDevice");
    if (dev < 0 || dev >= DEC_MAX_DEVICES) {
        set_error("paged_decode_noalloc: device %d out of range", dev);
        return FLOUR_ERR_UNSUPPORTED;
    }
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (r != hipSuccess || !p)
                return check_hip(r != hipSuccess ? r : hipErrorInvalidSymbol,
                                 "paged_decode_noalloc: hipGetSymbolAddress(scratch)");
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *ptr = p;
    return FLOUR_OK;
}

}  // namespace flour

extern "C" int flour_hip_paged_decode(void* out, int out_dtype, const void* q,
                                      const void* k_pool, const void* v_pool,
                                      const int32_t* block_tables, int max_blocks_per_seq,
                                      const int32_t* context_lens, int batch, int num_heads,
                                      int kv_heads, int head_dim, int block_size,
                                      int64_t num_slots, int max_context_len, float scale,
                                      int dtype, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    clear_error();
    return flour::paged_decode_impl(out, out_dtype, q, k_pool, v_pool, block_tables,
                                    max_blocks_per_seq, context_lens, batch, num_heads, kv_heads,
                                    head_dim, block_size, num_slots, max_context_len, scale, dtype,
                                    workspace, workspace_bytes, false, nullptr, nullptr, stream);
}

extern "C" size_t flour_hip_paged_decode_noalloc_max_workspace(void) {
    return flour::DEC_SCRATCH_BYTES;
}

extern "C" int flour_hip_paged_decode_noalloc(void* out, int out_dtype, const void* q,
                                              const void* k_pool, const void* v_pool,
                                              const int32_t* block_tables,
                                              int max_blocks_per_seq,
                                              const int32_t* context_lens, int batch,
                                              int num_heads, int kv_heads, int head_dim,
                                              int block_size, int64_t num_slots,
                                              int max_context_len, float scale, int dtype,
                                              void* stream) {
    clear_error();
    return flour::paged_decode_impl(out, out_dtype, q, k_pool, v_pool, block_tables,
                                    max_blocks_per_seq, context_lens, batch, num_heads, kv_heads,
                                    head_dim, block_size, num_slots, max_context_len, scale, dtype,
                                    nullptr, 0, true, nullptr, nullptr, stream);
}

namespace flour {

bool decode_mfma_supported(int dtype, int head_dim, int block_size, int n_rep, int batch,
                           int num_heads, int64_t num_slots, const void* q, const void* k_pool,
                           const void* v_pool) {
    return (dtype == FLOUR_DTYPE_BF16 || dtype == FLOUR_DTYPE_F16) &&
           (head_dim == 128 || head_dim == 64) && block_size % 16 == 0 && n_rep <= 16 &&
           batch <= DEC_MAX_BATCH && num_heads <= 65535 &&
           num_slots * head_dim * 2 <= (int64_t)0x7fffffff && ((uintptr_t)q % 16 == 0) &&
           ((uintptr_t)k_pool % 16 == 0) && ((uintptr_t)v_pool % 16 == 0);
}

static int paged_decode_impl(void* out, int out_dtype, const void* q, const void* k_pool,
                             const void* v_pool, const int32_t* block_tables,
                             int max_blocks_per_seq, const int32_t* context_lens, int batch,
                             int num_heads, int kv_heads, int head_dim, int block_size,
                             int64_t num_slots, int max_context_len, float scale, int dtype,
                             void* workspace, size_t workspace_bytes, bool ws_from_scratch,
                             const int32_t* rows, const DecodeWs* fused, void* stream) {
    if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) {
        set_error("paged_decode: unknown dtype (%d, out %d)", dtype, out_dtype);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (batch < 0 || num_heads <= 0 || kv_heads <= 0 || num_heads % kv_heads != 0 ||
        head_dim <= 0 || block_size <= 0 || num_slots <= 0 || num_slots % block_size != 0 ||
        max_blocks_per_seq <= 0 || max_context_len < 0 ||
        (int64_t)max_context_len > (int64_t)max_blocks_per_seq * block_size) {
        set_error("paged_decode: bad shape (batch=%d heads=%d kv_heads=%d head_dim=%d bs=%d "
                  "num_slots=%lld max_blocks=%d max_ctx=%d)",
                  batch, num_heads, kv_heads, head_dim, block_size, (long long)num_slots,
                  max_blocks_per_seq, max_context_len);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    if (batch == 0) return FLOUR_OK;
    if (!out || !q || !k_pool || !v_pool || !block_tables || !context_lens) {
        set_error("paged_decode: null pointer");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int n_rep = num_heads / kv_heads;
    const bool mfma = decode_mfma_supported(dtype, head_dim, block_size, n_rep, batch, num_heads,
                                            num_slots, q, k_pool, v_pool);
    if (!mfma && (rows || fused)) {
        set_error("paged_decode: row indices and the fused KV write need the matrix-core path");
        return FLOUR_ERR_UNSUPPORTED;
    }
    if (!mfma) {
        // one query row per sequence: cu_seqlens == nullptr
        const int64_t qs = (int64_t)num_heads * head_dim;
        if (simt_supported(dtype, head_dim, q, qs, head_dim, k_pool, v_pool))
            return launch_attn_simt(dtype, out_dtype, out, qs, head_dim, q, qs, head_dim, k_pool,
                                    v_pool, nullptr, context_lens, block_tables,
                                    max_blocks_per_seq, batch, batch, num_heads, n_rep, head_dim,
                                    block_size, num_slots, max_context_len, scale, s);
        return launch_attn_generic(dtype, out_dtype, out, (int64_t)num_heads * head_dim, head_dim,
                                   q, (int64_t)num_heads * head_dim, head_dim, k_pool, v_pool,
                                   nullptr, context_lens, block_tables, max_blocks_per_seq, batch,
                                   batch, num_heads, n_rep, head_dim, block_size, num_slots,
                                   max_context_len, scale, s);
    }
    const int nwg = decode_workgroups();
    const size_t need = decode_ws_bytes(nwg, n_rep, head_dim, batch);
    if (ws_from_scratch) {
        if (need > DEC_SCRATCH_BYTES) {
            set_error("paged_decode_noalloc: this call needs %zu bytes of split-context workspace, "
                      "more than the %zu bytes of the library's scratch; use "
                      "flour_hip_paged_decode with a caller workspace",
                      need, DEC_SCRATCH_BYTES);
            return FLOUR_ERR_WORKSPACE;
        }
        const int rc = scratch_for_current_device(&workspace);
        if (rc != FLOUR_OK) return rc;
        workspace_bytes = DEC_SCRATCH_BYTES;
    }
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace % 256) != 0) {
        set_error("paged_decode: workspace of %zu bytes (256-byte aligned) required, got %zu "
                  "at %p",
                  need, workspace_bytes, workspace);
        return FLOUR_ERR_WORKSPACE;
    }
    DecodeWs ws;
    ws.ml = static_cast<float*>(workspace);
    ws.o = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                    align256((size_t)2 * nwg * n_rep * 2 * sizeof(float)));
    ws.pre = reinterpret_cast<int*>(
        reinterpret_cast<char*>(ws.o) +
        align256((size_t)2 * nwg * n_rep * (size_t)head_dim * sizeof(float)));
    ws.rows = rows;
    ws.xcd_w = g_xcd_weight;
    ws.k_new = fused ? fused->k_new : nullptr;
    ws.v_new = fused ? fused->v_new : nullptr;
    ws.new_st = fused ? fused->new_st : 0;
    ws.new_sh = fused ? fused->new_sh : 0;
    ws.new_slots = fused ? fused->new_slots : nullptr;
#define FLOUR_DEC(T)                                                                            \
    do {                                                                                        \
        if (out_dtype == FLOUR_DTYPE_F32)                                                       \
            return launch_decode_mfma<T, float>(head_dim, out, q, k_pool, v_pool, block_tables,           \
                                                max_blocks_per_seq, context_lens, batch,        \
                                                num_heads, kv_heads, n_rep, block_size,         \
                                                num_slots, max_context_len, scale, nwg, ws, s); \
        if (out_dtype == FLOUR_DTYPE_BF16)                                                      \
            return launch_decode_mfma<T, bf16_t>(head_dim, out, q, k_pool, v_pool, block_tables,          \
                                                 max_blocks_per_seq, context_lens, batch,       \
                                                 num_heads, kv_heads, n_rep, block_size,        \
                                                 num_slots, max_context_len, scale, nwg, ws,    \
                                                 s);                                            \
        return launch_decode_mfma<T, f16_t>(head_dim, out, q, k_pool, v_pool, block_tables,               \
                                            max_blocks_per_seq, context_lens, batch, num_heads, \
                                            kv_heads, n_rep, block_size, num_slots,             \
                                            max_context_len, scale, nwg, ws, s);                \
    } while (0)
    if (dtype == FLOUR_DTYPE_BF16) FLOUR_DEC(bf16_t);
    FLOUR_DEC(f16_t);
#undef FLOUR_DEC
}

}  // namespace flour

namespace flour {

// Paged decode whose batch entry b reads q row rows[b] and writes out row rows[b] of a packed
// (rows, num_heads, head_dim) contiguous layout: the one-row sequences of a mixed
// continuous-batching step. Matrix-core shapes only (FLOUR_ERR_UNSUPPORTED otherwise, before
// any launch).
int paged_decode_rows(void* out, int out_dtype, const void* q, const void* k_pool,
                      const void* v_pool, const int32_t* block_tables, int max_blocks_per_seq,
                      const int32_t* context_lens, const int32_t* rows, int batch, int num_heads,
                      int kv_heads, int head_dim, int block_size, int64_t num_slots,
                      int max_context_len, float scale, int dtype, void* workspace,
                      size_t workspace_bytes, void* stream) {
    if (!rows) {
        set_error("paged_decode_rows: null row indices");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    return paged_decode_impl(out, out_dtype, q, k_pool, v_pool, block_tables, max_blocks_per_seq,
                             context_lens, batch, num_heads, kv_heads, head_dim, block_size,
                             num_slots, max_context_len, scale, dtype, workspace, workspace_bytes,
                             false, rows, nullptr, stream);
}

int paged_decode_write_kv(void* out, int out_dtype, const void* q, void* k_pool, void* v_pool,
                          const int32_t* block_tables, int max_blocks_per_seq,
                          const int32_t* context_lens, int batch, int num_heads, int kv_heads,
                          int head_dim, int block_size, int64_t num_slots, int max_context_len,
                          float scale, int dtype, void* workspace, size_t workspace_bytes,
                          const void* k_new, const void* v_new, int64_t new_stride_tok,
                          int64_t new_stride_head, const int32_t* new_slots, void* stream) {
    const int es = (dtype == FLOUR_DTYPE_F32) ? 4 : 2;
    const uint64_t row_align = head_dim == 128 ? 16 : 8;  // a lane's share of a row
    // 16-token pages only: the fused instantiation for other page sizes spills registers in its
    // piece epilogue (a reload there waits for every chunk load in flight)
    if (!k_new || !v_new || !new_slots || batch < 1 || kv_heads <= 0 || block_size != 16 ||
        num_heads % kv_heads != 0 ||
        !decode_mfma_supported(dtype, head_dim, block_size, num_heads / kv_heads, batch,
                               num_heads, num_slots, q, k_pool, v_pool) ||
        (((uint64_t)(uintptr_t)k_new | (uint64_t)(uintptr_t)v_new |
          (uint64_t)(new_stride_tok * es) | (uint64_t)(new_stride_head * es)) &
         (row_align - 1)) != 0) {
        set_error("paged_decode_write_kv: shape not taken by the fused launch");
        return FLOUR_ERR_UNSUPPORTED;
    }
    DecodeWs fz{};
    fz.k_new = k_new;
    fz.v_new = v_new;
    fz.new_st = new_stride_tok;
    fz.new_sh = new_stride_head;
    fz.new_slots = new_slots;
    return paged_decode_impl(out, out_dtype, q, k_pool, v_pool, block_tables, max_blocks_per_seq,
                             context_lens, batch, num_heads, kv_heads, head_dim, block_size,
                             num_slots, max_context_len, scale, dtype, workspace, workspace_bytes,
                             false, nullptr, &fz, stream);
}

}  // namespace flour
