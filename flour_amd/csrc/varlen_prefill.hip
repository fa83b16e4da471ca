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
//  * One workgroup (8 waves) per (128-row query tile, pair of query heads that share a kv
//    head, sequence); wave w owns 32 query rows of head w / 4, and every K/V tile staged in
//    LDS serves both heads. (Register staging: a sequence's last tile of at most 64 / 32 rows
//    runs as 4 heads x 64 rows / 8 heads x 32 rows per workgroup instead, and with an odd GQA
//    group the last head of two consecutive tiles as 1 head x 256 rows.) By default one
//    persistent workgroup per CU walks its share of the
//    item list (decreasing query-tile index, close to longest-first, dealt as a snake); the
//    next item's Q rows are staged in LDS during the current item and its first K/V tiles
//    loaded by the current item's last steps. Without the persistent schedule, one workgroup
//    per item, issued in the same order over all XCDs.
//  * 64-token K/V tiles are gathered page by page through the block table into LDS with
//    buffer loads (tokens past kv_len read zeros); the loads of tile t+2 are in flight while
//    tile t is computed and tile t+1 is written to the other LDS buffer. K is stored row-major
//    (pitch 272 B, conflict-free 16 B reads); V is stored transposed (V^T, pitch 144 B) with the
//    tokens of each 16-token group permuted (bits 2 and 3 swapped), which is the order in which
//    the score registers feed the P.V product.
//  * S^T = K Q^T on v_mfma_f32_32x32x16 (M = 32 tokens, N = 32 queries, K = 16 dims): lane
//    (h, q) = (lane/32, lane%32) holds query q's scores for tokens 8i + 4h + j. Those registers
//    are, after 16-bit packing, the B operand of O^T = V^T P^T (K = 16 tokens), so P never
//    moves between lanes; V^T rows come straight from LDS as 16 B reads.
//  * Online softmax in the exp2 domain with the scale folded into the exponent's FMA (the
//    MFMA path requires scale > 0), one max exchange between the two lane halves per tile.
//    The reference max may lag the running max by up to 8 (weights up to 2^8), so the output
//    accumulator is rescaled only when some row's max grows past that. Fully masked tiles are
//    skipped per wave; masks are evaluated only on tiles that cross the diagonal.
//  * P.V precision: PV_F16 rounds P once to fp16 and converts bf16 V to fp16 (exact in range);
//    PV_HILO splits P into hi + lo parts of the storage type (two MFMAs per product, ~16
//    significant bits).
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "flour_common.h"

namespace flour {

bool prefill_f32_mfma_supported(int dtype, int head_dim, int num_seqs, int max_seqlen_q,
                                int block_size, int64_t num_slots);
int launch_prefill_f32_mfma(int out_dtype, void* out, int64_t o_st, int64_t o_sh, const void* q,
                            int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool,
                            const int32_t* cu_seqlens_q, const int32_t* q_rows,
                            const int32_t* kv_lens, const int32_t* block_tables, int max_blocks,
                            int num_seqs, int max_seqlen_q, int num_heads, int n_rep,
                            int head_dim, int block_size, int64_t num_slots, float scale,
                            hipStream_t stream);
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

static constexpr int PF_D = 128;   // head dims of the matrix-core path: 128 and PF_D64
static constexpr int PF_D64 = 64;
// a / d for 0 <= a < 2^20 and 0 < d < 2^20: a float estimate (its error is below one) and one
// correction step; a few instructions where an integer division by a runtime value takes ~30.
__device__ __forceinline__ int div_small(int a, int d) {
    const int q = (int)((float)a * __builtin_amdgcn_rcpf((float)d));
    const int r = a - q * d;
    return q + (r >= d ? 1 : 0) - (r < 0 ? 1 : 0);
}

static constexpr int PF_QT = 128;  // query rows per head per workgroup (4 waves x 32)
static constexpr int PF_KT = 64;   // kv tokens per tile
static constexpr int PF_WAVES = 8; // two query heads of one kv head x 4 waves
static constexpr int PF_THREADS = PF_WAVES * 64;
static constexpr float PF_RESCALE_SLACK = 8.0f;  // log2 units the reference max may lag
// K rows in LDS (register staging): head_dim + 8 elements, 272 B at 128 and 144 B at 64
__host__ __device__ constexpr int pf_kpitch(int d) { return d + 8; }
static constexpr int PF_VPITCH = PF_KT + 8;  // elements: 144 B rows
static constexpr int PF_OPITCH = 68;         // elements: 136 B rows of output staging
// Per-wave Q staging block (register staging): 32 rows of up to 128 dims, 8 KB; it also
// stages the output, 32 rows of 64 dims at a time with the PF_OPITCH pitch.
static constexpr int PF_QSTAGE_ELEMS = 32 * PF_D;
static_assert(32 * PF_OPITCH <= PF_QSTAGE_ELEMS, "output staging fits a wave's Q block");
static constexpr float PF_LOG2E = 1.4426950408889634f;
// Persistent schedule limits (the per-workgroup item table lives in LDS); larger batches use
// one workgroup per item.
static constexpr int PF_MAX_SEQS = 2048;
static constexpr int PF_MAX_LEVELS = 512;  // query tiles per sequence (65536 rows)
static constexpr int PF_MAX_WG_ITEMS = 256;  // items per workgroup
// (level, sequence) entries up to which register staging shapes its items per entry
static constexpr int PF_FLEX_ENTRIES = 4096;
// Workgroups up to which register staging deals its last round by load (the load table lives
// in LDS); a larger grid keeps the plain snake.
static constexpr int PF_MAX_GRID = 256;
// Item cost in the load-ranked deal, 5 per kv tile + 7: per-workgroup cycle counts of the
// Llama-3-8B varlen batch fit about 3,950 cycles per kv tile and 5,560 per item.
static constexpr int PF_COST_TILE = 5, PF_COST_ITEM = 7;

__device__ __forceinline__ int swap_bits01(int x) {
    return (x & ~3) | ((x & 1) << 1) | ((x >> 1) & 1);
}

// P.V arithmetic of the MFMA path.
//  PV_F16:   P rounded once to fp16 (11 significant bits; P is in [0, 2^8]) and V converted
//            to fp16 when the pool is bf16 (exact in fp16's range, below); one MFMA per
//            product.
//  PV_HILO:  P split into hi + lo parts of the storage type (~16 significant bits), V in the
//            storage type; two MFMAs per product.
//  exact:    the fallback of PV_F16 for an item whose fp16 P.V cannot be trusted (below):
//            V stays bf16, P is split into bf16 hi + lo parts, and the running max is kept
//            exact (no slack), so every weight is at most 1 and |p v| stays in fp32 range.
//
// bf16 V in PV_F16 mode is converted to fp16 (round to nearest even), which holds every bf16
// value with 2^-17 <= |v| <= 65504 exactly, and 0. Outside that:
//  * |v| >= 65520, inf or NaN become inf or NaN and make the accumulator non-finite;
//  * 0 < |v| < 2^-17 is rounded to the fp16 grid (spacing 2^-24), an error of at most 2^-25 in
//    v, hence at most 2^-25 in any output (the weights sum to 1).
// At the end of each item every wave checks its output block (its valid rows x head_dim): if
// it is not finite, or if its root mean square is below 2^-25 / 5e-4 (where the conversion's
// error could exceed 5e-4 of the block's L2 norm), the workgroup recomputes the item in exact
// mode. Otherwise the block's error from the conversion is at most 5e-4 of its norm and that
// from rounding P to fp16 ~1.5e-4.
static constexpr float PF_MIN_TRUSTED_RMS = 0x1p-25f / 5e-4f;  // ~6e-5
enum { PV_F16 = 0, PV_HILO = 1 };

static constexpr uint32_t PF_OOR = 0x80000000u;  // buffer offset past any pool: loads read 0

// Direct-to-LDS staging (the DMA kernel, head_dim 128): three LDS tile buffers; V comes
// pre-widened from a staging copy of 4 KB pages, each 16 tokens of one kv head as V^T (128 dims
// x 16 fp16, token sigma16(k) at position k), written by prefill_v_stage_kernel before the
// attention launch.
static constexpr int PF_VPAGE_BYTES = 16 * PF_D * 2;

// 64 lanes x 16 bytes from a raw buffer straight into LDS: lane L's bytes come from
// rsrc.base + soff + voff and land at LDS byte lds + 16 L; lanes past the buffer's size write
// zeros. Issued from inline asm so that the compiler's wait-count tracking, which knows nothing
// of these loads, adds no waits for them to the LDS reads; every wait for them is explicit.
// M0 (the LDS destination) is written here. The AMDGPU backend treats M0 as a reserved
// register and ignores it in clobber lists; none of its own code in these kernels reads M0 (the
// generated ISA has no M0 reader other than these loads), so no compiler value can be
// overwritten. The s_nop 0 between the M0 write and the load is the wait state a vector memory
// instruction that reads M0 needs after an SALU write of M0 (the hardware does not interlock
// it, and the compiler's hazard tracking does not look inside inline asm).
__device__ __forceinline__ void dma_b128(uint32_t voff, __amdgpu_buffer_rsrc_t rsrc, uint32_t lds,
                                         uint32_t soff) {
    const uint32_t l = __builtin_amdgcn_readfirstlane(lds);
    const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %3 offen lds"
                 :: "v"(voff), "s"(rsrc), "s"(l), "s"(so) : "memory");
}
// 16-byte global store issued from inline asm: the compiler's wait-count tracking does not see
// it, so pending output stores never turn its waits for tile loads into full drains (loads and
// stores share the counter, and with both pending it would wait for zero). Every wait the
// compiler computes then only over-counts outstanding operations, never under-counts loads.
// Its hazard tracking does not see it either: a vector instruction may not overwrite the data
// registers of a store wider than 8 bytes in the next two cycles, hence the s_nop.
__device__ __forceinline__ void gstore_b128(void* p, u32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off\n\ts_nop 1" :: "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ uint32_t lds_byte_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ int sigma16(int t) {  // swap bits 2 and 3 (token order in V^T rows)
    return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1);
}

template <typename T, typename TO, int PV, bool BS16, bool DMA, int D>
__global__ __launch_bounds__(PF_THREADS, 1) void varlen_prefill_mfma_kernel(
    TO* __restrict__ out, int64_t o_st, int64_t o_sh, const T* __restrict__ q, int64_t q_st,
    int64_t q_sh, const T* __restrict__ k_pool, const T* __restrict__ v_pool,
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ block_tables, int max_blocks, int num_seqs, int num_heads,
    int n_rep, int block_size, int64_t num_slots, int n_qt_max, int persistent,
    float scale_log2, const f16_t* __restrict__ v_stage, uint32_t v_stage_bytes,
    const int32_t* __restrict__ q_rows) {
    // DMA: K and V tiles go straight from memory into LDS (K from the pool, V from the staging
    // copy), three buffers, no staging registers. It needs the persistent schedule and fp16 P.V.
    static_assert(!DMA || PV == PV_F16, "the DMA kernel runs the fp16 P.V path");
    static_assert(!DMA || D == PF_D, "the DMA kernel runs head_dim 128");
    static_assert(D == PF_D || D == PF_D64, "matrix-core prefill: head_dim 128 or 64");
    constexpr int KPITCH = pf_kpitch(D);
    constexpr int CPR = D / 8;         // 16-byte chunks per K / V row
    constexpr int NKQ = D / 16;        // 16-dim k-steps of S^T = K Q^T (Q^T registers)
    constexpr int NMT = D / 32;        // 32-dim blocks of O^T = V^T P^T
    // V^T is staged as fp16 for PV_F16, as the storage type otherwise; K keeps the storage type.
    typedef typename std::conditional<PV == PV_F16, f16_t, T>::type TV;
    // bf16 V is converted to fp16 and each item's output blocks are checked at its
    // end (CHECK_V); a failed check recomputes the item in exact mode.
    constexpr bool CHECK_V = PV == PV_F16 && std::is_same<T, bf16_t>::value;
    // LDS tile buffers, each K then V:
    //  * register staging: K row-major with a 272 B pitch, V^T with a 144 B pitch; two buffers;
    //  * DMA: K row-major without padding, the 16-byte chunk c of row r stored at chunk
    //    c ^ (r % 16) (conflict-free fragment reads); V^T as four 4 KB pages (the staging copy's
    //    layout), or in exact mode the register-staged V^T with a 144 B pitch; three buffers.
    constexpr int NBUF = DMA ? 3 : 2;
    constexpr int K_ELEMS = DMA ? PF_KT * D : PF_KT * KPITCH;
    constexpr int TILE_ELEMS = K_ELEMS + D * PF_VPITCH;
    static_assert(!DMA || 8 * 32 * PF_OPITCH <= TILE_ELEMS, "output staging fits one buffer");
    __shared__ __attribute__((aligned(16))) uint16_t tiles[NBUF * TILE_ELEMS];
    auto kb_ptr = [&](int b) { return &tiles[b * TILE_ELEMS]; };
    auto vb_ptr = [&](int b) { return &tiles[b * TILE_ELEMS + K_ELEMS]; };
    // per wave, item end; two sets by item parity (an item whose first tile is already in LDS
    // starts without a barrier, so its last step may come while the previous item's flags are
    // still being read)
    __shared__ __attribute__((aligned(8))) uint8_t redo_flag[2 * PF_WAVES];

    // ---- work items: (query tile, sequence, pair of query heads), ordered by decreasing
    // query-tile index ("level"): the cost of an item grows with its tile index (its causal kv
    // range is kv_len - q_len + 128 (qt + 1)), so this is close to longest-first order.
    //  * persistent: one workgroup per CU walks the items that exist (sequences too short for
    //    a level are left out); the deal over the workgroups is below;
    //  * otherwise: one workgroup per (level, sequence, pair), items past a sequence's last
    //    tile exit at once, and the dispatcher deals the levels over all XCDs.
    const int pairs_per_kv = (n_rep + 1) >> 1;
    const int kv_heads = num_heads / n_rep;
    const int npairs = kv_heads * pairs_per_kv;
    const int tid = threadIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int h2 = lane >> 5, ql32 = lane & 31;
    const int NQ = n_qt_max;
    const int G = gridDim.x;
    const int wg = blockIdx.x;
    const int kv_cap = max_blocks * block_size;  // kv lengths are clamped to the block table
    // DMA: pages per sequence in the V staging copy (the block table's capacity in whole tiles)
    const int stage_pages = 4 * ((kv_cap + PF_KT - 1) / PF_KT);

    // The schedule tables below are read only while the items are decoded; in the register-
    // staged kernel their LDS is then reused as the Q staging area: one 8 KB block per wave
    // (32 query rows x 256 B, the 16-byte chunk c of row r stored at chunk c ^ (r % 16)),
    // which receives the next item's rows during the current item and stages the output.
    // Register staging shapes items per (level, sequence) entry (FLEX): a sequence's last,
    // partial query tile takes 4 heads x 64 rows or 8 heads x 32 rows per item instead of
    // 2 heads x 128, and the one-head items of two consecutive tiles (odd GQA groups) share
    // one item of 256 rows.
    constexpr bool FLEX = !DMA;
    constexpr int LOAD_INTS = FLEX ? 3 * PF_MAX_GRID + 2 : 0;
    constexpr int SCHED_INTS = 3 * PF_MAX_SEQS + 1 + 3 * (PF_MAX_LEVELS + 1) + 1 + LOAD_INTS;
    constexpr int QSTAGE_BYTES = DMA ? 0 : PF_WAVES * PF_QSTAGE_ELEMS * 2;
    constexpr int SCHED_BYTES = 4 * SCHED_INTS > QSTAGE_BYTES ? 4 * SCHED_INTS : QSTAGE_BYTES;
    __shared__ __attribute__((aligned(16))) uint8_t sched_raw[SCHED_BYTES];
    int* const sched_order = reinterpret_cast<int*>(sched_raw);  // sequences by decreasing tile count
    int* const sched_more = sched_order + PF_MAX_SEQS;  // [v]: sequences with more than v tiles
    int* const sched_fill = sched_more + (PF_MAX_LEVELS + 1);
    int* const sched_cum = sched_fill + (PF_MAX_LEVELS + 1);  // [L]: items before level L
    int* const sched_cu = sched_cum + (PF_MAX_LEVELS + 2);    // cu_seqlens
    int* const sched_kv = sched_cu + (PF_MAX_SEQS + 1);       // clamped kv lengths
    // FLEX: [G + 1] differences of the per-workgroup loads of the deal, then (8-byte aligned)
    // [PF_MAX_GRID] the items of the deal's last round, {seq | level << 11 | part << 20, index}
    int* const sched_load = sched_kv + PF_MAX_SEQS;
    constexpr int LAST_OFF = (4 * (SCHED_INTS - LOAD_INTS + PF_MAX_GRID + 1) + 7) & ~7;  // bytes
    static_assert(!FLEX || LAST_OFF + 8 * PF_MAX_GRID <= 4 * SCHED_INTS, "deal tables fit");
    static_assert(PF_MAX_SEQS <= 2048 && PF_MAX_LEVELS <= 512, "last-round entries pack in 21 bits");
    int2* const sched_last = reinterpret_cast<int2*>(sched_raw + LAST_OFF);
    static_assert(!FLEX || 4 * SCHED_INTS <= QSTAGE_BYTES, "decode tables fit the Q staging");
    // query tiles of a sequence; one with kv_len < q_len still has its tiles, whose items
    // attend nothing and write zero rows (as the generic path and the oracle do)
    auto seq_tiles = [&](int sq) {
        const int l = sched_cu[sq + 1] - sched_cu[sq];
        return l <= 0 ? 0 : min((l + PF_QT - 1) / PF_QT, NQ);
    };
    // exclusive suffix / prefix scans over up to PF_MAX_LEVELS + 1 entries by wave 0
    auto wave_scan = [&](int n, auto&& get, auto&& put, bool suffix) {
        const int per = (n + 63) / 64;
        int local = 0;
        for (int i = 0; i < per; i++) {
            const int x = lane * per + i;
            if (x < n) local += get(suffix ? n - 1 - x : x);
        }
        const int incl = wave_incl_sum(local);
        int run = incl - local;
        for (int i = 0; i < per; i++) {
            const int x = lane * per + i;
            if (x < n) {
                const int v = get(suffix ? n - 1 - x : x);
                put(suffix ? n - 1 - x : x, run);
                run += v;
            }
        }
        return __builtin_amdgcn_readlane(incl, 63);  // total
    };
    // Heads per item of a tile with r rows (FLEX): 8 for at most 32 rows, 4 for at most 64, else
    // 2, but at most the GQA group rounded up to a power of two, and always 2 for groups of 1
    // or 2 heads. Its log2 (1 .. 3) is what the item table keeps.
    auto shape_lg = [&](int r) {
        if (!FLEX || n_rep <= 2 || r > 64) return 1;
        const int cap = n_rep <= 4 ? 2 : 3;
        return min(r <= 32 ? 3 : 2, cap);
    };
    // Entry (sequence sq, tile qt = NQ-1-L): what the schedule needs of it, read from LDS once.
    // Its items: with an odd n_rep the last head of tiles of 2 heads x 128 is a one-head item,
    // tiles 2j and 2j + 1 sharing one of 256 rows that costs about as much as a two-head item of
    // tile 2j + 1. Part 1 (c1): the multi-head items, then at odd qt the shared one-head items;
    // part 2 (c2): one-head items of a single tile (2j without tile 2j + 1).
    struct Entry {
        int seq, qt, L, lg, c0, ql, kvl, c1, c2;
    };
    auto entry_at = [&](int sq, int L) __attribute__((always_inline)) {
        Entry x;
        x.seq = sq;
        x.L = L;
        x.qt = NQ - 1 - L;
        x.c0 = sched_cu[sq];
        x.ql = sched_cu[sq + 1] - x.c0;
        x.kvl = sched_kv[sq];
        const int t = x.ql <= 0 ? 0 : min((x.ql + PF_QT - 1) / PF_QT, NQ);  // as seq_tiles
        // shape of tile qt: its last tile by its rows, the others 2 heads x 128
        auto lg_of = [&](int qt) { return qt < t - 1 ? 1 : shape_lg(x.ql - PF_QT * qt); };
        x.lg = lg_of(x.qt);
        const bool lone = (n_rep & 1) && x.lg == 1;
        x.c1 = kv_heads * (x.lg == 1 ? (n_rep >> 1) : ((n_rep + (1 << x.lg) - 1) >> x.lg)) +
               (lone && (x.qt & 1) ? kv_heads : 0);
        x.c2 = lone && !(x.qt & 1) && !(x.qt + 1 < t && lg_of(x.qt + 1) == 1) ? kv_heads : 0;
        return x;
    };
    int total_items = 0, total_base = 0, total1 = 0;  // items; (level, sequence) pairs; part 1
    bool flex_on = false;
    // ---- this workgroup's items, decoded into LDS. An entry holds {seq, qt, kv head, first
    // head in group | log2(heads per item) << 16, q0, q_len, kv_len, kv tiles}.
    //  * persistent: the item list is longest-first in two parts: the multi-head items of every
    //    level, then (odd n_rep) the one-head items of a single tile, which cost about 0.7 of a
    //    two-head item. Within a part, items go level by level, sequences by decreasing tile
    //    count, then heads; a one-head item of tiles qt - 1 and qt sits in part 1 after tile
    //    qt's multi-head items. The k-th item of workgroup b is number kG + b on even k and
    //    kG + G-1-b on odd k (a snake over the list balances the workgroups without shared
    //    state), except that register staging deals the last round by the workgroups' load;
    //  * otherwise: one workgroup per (level, sequence, pair); items past a sequence's last
    //    tile exit at once.
    __shared__ __attribute__((aligned(16))) int sched_items[PF_MAX_WG_ITEMS][8];
    __shared__ int sched_nitems;
    const int half_rep = n_rep >> 1;
    int wg_items = 0;
    // the snake's share of workgroup wg in a list of n items
    auto items_of_wg = [&](int n) {
        const int rounds = div_small(n, G), rem = n - rounds * G;
        return min(rounds + (((rounds & 1) ? G - 1 - wg : wg) < rem ? 1 : 0), PF_MAX_WG_ITEMS);
    };
    // item k of this workgroup: tile NQ-1-level of sequence seq, heads h0 .. of kv head kvh
    auto put_item = [&](int k, int seq, int level, int kvh, int h0, int lg) __attribute__((always_inline)) {
        // first q / out row of the sequence: q_rows[seq] when given (the sequences of a mixed
        // step, whose rows sit among other sequences' rows), else its cu_seqlens start
        const int c0 = persistent ? sched_cu[seq] : cu_seqlens[seq];
        const int q0 = q_rows ? q_rows[seq] : c0;
        const int ql = (persistent ? sched_cu[seq + 1] : cu_seqlens[seq + 1]) - c0;
        const int kvl = persistent ? sched_kv[seq] : min(kv_lens[seq], kv_cap);
        const int qt = NQ - 1 - level;
        const int row_last = min(qt * PF_QT + (256 >> lg), ql) - 1;  // the item's last row
        const bool ok = qt * PF_QT < ql;  // always true for persistent items
        int* e = sched_items[k];
        e[0] = seq;
        e[1] = qt;
        e[2] = kvh;
        e[3] = h0 | (lg << 16);
        e[4] = q0;
        e[5] = ql;
        e[6] = kvl;
        // causal kv tiles; none when kv_len < q_len (the rows are written as zeros)
        e[7] = (ok && kvl >= ql) ? (kvl - ql + row_last + 1 + PF_KT - 1) / PF_KT : 0;
        return ok;
    };
    // item k of this workgroup from an Entry: the entry's tile, or tile qt - 1 for a one-head item
    // of 256 rows (level L + 1); fields as put_item writes them
    auto put_item_e = [&](int k, const Entry& x, int level, int kvh, int h0, int lg)
                          __attribute__((always_inline)) {
        const int qt = NQ - 1 - level;
        const int row_last = min(qt * PF_QT + (256 >> lg), x.ql) - 1;
        int* e = sched_items[k];
        e[0] = x.seq;
        e[1] = qt;
        e[2] = kvh;
        e[3] = h0 | (lg << 16);
        e[4] = q_rows ? q_rows[x.seq] : x.c0;
        e[5] = x.ql;
        e[6] = x.kvl;
        e[7] = x.kvl >= x.ql ? (x.kvl - x.ql + row_last + 1 + PF_KT - 1) / PF_KT : 0;
    };
    if (persistent) {
        for (int i = tid; i <= num_seqs; i += PF_THREADS) sched_cu[i] = cu_seqlens[i];
        for (int i = tid; i < num_seqs; i += PF_THREADS) sched_kv[i] = min(kv_lens[i], kv_cap);
        if constexpr (FLEX)
            for (int i = tid; i <= G && G <= PF_MAX_GRID; i += PF_THREADS) sched_load[i] = 0;
        __syncthreads();
        if (w == 0 && num_seqs <= 64 && NQ < 64) {
            // One sequence per lane, all in registers: more[v] = sequences with a tile count
            // above v from one ballot per v; a sequence's place in the order (decreasing tile
            // count, then index) is more[its count] plus the lanes of equal count below it;
            // the level offsets are a prefix sum over the lanes.
            const int n = lane < num_seqs ? seq_tiles(lane) : 0;
            const uint64_t below = (1ull << lane) - 1;
            int more_v = 0, more_rev = 0, more_n = 0, eq_rank = 0;
            for (int v = 0; v <= NQ; v++) {
                const int mv = __popcll(__ballot(n > v));
                const uint64_t eq = __ballot(n == v);
                if (lane == v) more_v = mv;
                if (lane == NQ - 1 - v) more_rev = mv;
                if (n == v) {
                    more_n = mv;
                    eq_rank = __popcll(eq & below);
                }
            }
            if (lane <= NQ) sched_more[lane] = more_v;
            if (n > 0) sched_order[more_n + eq_rank] = lane;
            // level L (tile qt = NQ-1-L) holds the sequences with more than qt tiles:
            // sched_cum[L] = sequences on the levels before L
            const int x = lane < NQ ? more_rev : 0;
            const int incl = wave_incl_sum(x);
            if (lane < NQ) sched_cum[lane] = incl - x;
            if (lane == 63) sched_cum[NQ] = incl;
        } else if (w == 0) {
                // Wave 0 alone, without barriers (a wave's LDS operations complete in order):
                // histogram of tile counts, more[v] = sequences with a tile count above v (its
                // suffix sum), a stable counting sort by decreasing tile count, and the level
                // offsets.
                for (int v = lane; v <= NQ; v += 64) sched_fill[v] = 0;
                __builtin_amdgcn_wave_barrier();
                for (int sq = lane; sq < num_seqs; sq += 64) atomicAdd(&sched_fill[seq_tiles(sq)], 1);
                __builtin_amdgcn_wave_barrier();
                wave_scan(NQ + 1, [&](int v) { return sched_fill[v]; },
                          [&](int v, int x) { sched_more[v] = x; }, true);
                __builtin_amdgcn_wave_barrier();
                for (int v = lane; v <= NQ; v += 64) sched_fill[v] = 0;
                __builtin_amdgcn_wave_barrier();
                // stable counting sort (every workgroup must build the same order): 64 sequences
                // at a time, a lane's rank among equal tile counts comes from ballots over the
                // count's bits (counts are at most PF_MAX_LEVELS < 1024)
                for (int base = 0; base < num_seqs; base += 64) {
                    const int sq = base + lane;
                    const int n = sq < num_seqs ? seq_tiles(sq) : 0;
                    uint64_t same = ~0ull;
#pragma unroll
                    for (int b = 0; b < 10; b++) {
                        const uint64_t bal = __ballot((n >> b) & 1);
                        same &= ((n >> b) & 1) ? bal : ~bal;
                    }
                    const int rank = __popcll(same & ((1ull << lane) - 1));
                    const int fill = sched_fill[n];
                    if (n > 0) sched_order[sched_more[n] + fill + rank] = sq;
                    if (rank == 0) sched_fill[n] = fill + __popcll(same);
                    __builtin_amdgcn_wave_barrier();
                }
                // level L (tile qt = NQ-1-L) holds the sequences with more than qt tiles:
                // sched_cum[L] = sequences on the levels before L
                const int t = wave_scan(NQ, [&](int L) { return sched_more[NQ - 1 - L]; },
                                        [&](int L, int x) { sched_cum[L] = x; }, false);
                if (lane == 0) sched_cum[NQ] = t;
        }
        __syncthreads();
        total_base = __builtin_amdgcn_readfirstlane(sched_cum[NQ]);
        total_items = npairs * total_base;
        flex_on = FLEX && total_base <= PF_FLEX_ENTRIES;
        if (flex_on) {
            // Each thread walks a contiguous run of entries (level by level, sequences in
            // tile-count order) twice: once for its item counts, whose exclusive prefix sums
            // over the workgroup give each entry's first item in part 1 and part 2, then to
            // decode the items of its entries that the snake deals to this workgroup.
            const int per = (total_base + PF_THREADS - 1) / PF_THREADS;
            const int e0 = min(tid * per, total_base), e1 = min(e0 + per, total_base);
            int L = 0, hi = NQ - 1;  // level of entry e0: last L with sched_cum[L] <= e0
            while (L < hi) {
                const int mid = (L + hi + 1) >> 1;
                if (sched_cum[mid] <= e0) L = mid; else hi = mid - 1;
            }
            const int L0 = L, i0 = e0 - sched_cum[L];
            int s1 = 0, s2 = 0;
            Entry x0{};  // this thread's first entry, kept for the second walk
            for (int e = e0, i = i0; e < e1; e++) {
                const Entry x = entry_at(sched_order[i], L);
                if (e == e0) x0 = x;
                s1 += x.c1;
                s2 += x.c2;
                if (++i == sched_more[x.qt]) {  // levels are never empty once started
                    L++;
                    i = 0;
                }
            }
            const int x1 = wave_incl_sum(s1), x2 = wave_incl_sum(s2);  // inclusive, in the wave
            if (lane == 63) {  // wave totals (sched_fill is free once the order is built)
                sched_fill[2 * w] = x1;
                sched_fill[2 * w + 1] = x2;
            }
            __syncthreads();
            int b1 = 0, b2 = 0, t1 = 0, t2 = 0;
            for (int v = 0; v < PF_WAVES; v++) {
                const int a1 = sched_fill[2 * v], a2 = sched_fill[2 * v + 1];
                if (v < w) {
                    b1 += a1;
                    b2 += a2;
                }
                t1 += a1;
                t2 += a2;
            }
            total1 = __builtin_amdgcn_readfirstlane(t1);
            total_items = total1 + __builtin_amdgcn_readfirstlane(t2);
            // this run's first item of part 1 and of part 2, as list indices
            const int a1_0 = b1 + x1 - s1, a2_0 = total1 + b2 + x2 - s2;
            // walks this thread's entries: fn(entry, first item of part 1, of part 2)
            auto walk = [&](auto&& fn) {
                int L = L0, a1 = a1_0, a2 = a2_0;
                for (int e = e0, i = i0; e < e1; e++) {
                    const Entry x = e == e0 ? x0 : entry_at(sched_order[i], L);
                    fn(x, a1, a2);
                    a1 += x.c1;
                    a2 += x.c2;
                    if (++i == sched_more[x.qt]) {  // levels are never empty once started
                        L++;
                        i = 0;
                    }
                }
            };
            // item p of part `part` of entry x, into slot k
            auto put_entry_item = [&](int k, int part, int p, const Entry& x) {
                const int L = x.L;
                int level = L, kvh, h0, lg = 1;
                if (part) {
                    kvh = p;
                    h0 = n_rep - 1;
                } else {
                    lg = x.lg;
                    if (lg == 1 && p >= kv_heads * half_rep) {  // 1 head x 256 rows from qt - 1
                        kvh = p - kv_heads * half_rep;
                        h0 = n_rep - 1;
                        lg = 0;
                        level = L + 1;
                    } else if (lg == 1) {
                        kvh = div_small(p, half_rep);
                        h0 = 2 * (p - kvh * half_rep);
                    } else {
                        const int g = (n_rep + (1 << lg) - 1) >> lg;  // items per kv head
                        kvh = div_small(p, g);
                        h0 = (p - kvh * g) << lg;
                    }
                }
                put_item_e(k, x, level, kvh, h0, lg);
            };
            // Rounds 0 .. R-2 follow the snake: item idx of round rd = idx / G goes to workgroup
            // idx % G on even rounds, G-1 - idx % G on odd ones. From three rounds on, the last
            // round is dealt by load instead: with every workgroup's cost over the earlier rounds
            // (5 per kv tile + 7 per item), its items in list order go to the workgroups by
            // increasing cost (ties by index), so the longest of them land where the snake left
            // the least work (with two rounds the snake already pairs long with short). Every
            // workgroup computes the same costs and so the same ranks.
            const int rounds = (total_items + G - 1) / G;
            const bool ranked = rounds >= 3 && rounds <= PF_MAX_WG_ITEMS && G <= PF_MAX_GRID;
            const int cut = ranked ? (rounds - 1) * G : total_items;
            wg_items = ranked ? rounds - 1 : items_of_wg(total_items);
            walk([&](const Entry& x, int a1, int a2) {
#pragma unroll
                for (int part = 0; part < 2; part++) {
                    const int a = part ? a2 : a1, c = part ? x.c2 : x.c1;
                    for (int rd = div_small(a, G); rd * G < a + c && rd < wg_items; rd++) {
                        const int idx = rd * G + ((rd & 1) ? G - 1 - wg : wg);
                        if (idx >= a && idx < a + c) put_entry_item(rd, part, idx - a, x);
                    }
                }
                if (!ranked) return;
                // the entry's items of the last round, for the workgroup that ranks there
#pragma unroll
                for (int part = 0; part < 2; part++) {
                    const int a = part ? a2 : a1, end = a + (part ? x.c2 : x.c1);
                    for (int idx = max(a, cut); idx < end; idx++)
                        sched_last[idx - cut] = int2{x.seq | (x.L << 11) | (part << 20), idx - a};
                }
                // the entry's items before the cut add their cost to the workgroups the snake
                // gives them: per round one contiguous range of workgroups, as differences. All
                // items of an entry share its kv tile count (a one-head item of tiles qt - 1 and
                // qt ends on tile qt's last row).
                const int row_end = min((x.qt + 1) * PF_QT, x.ql);
                const int n_kt = x.kvl >= x.ql ? (x.kvl - x.ql + row_end + PF_KT - 1) / PF_KT : 0;
                const int cost = PF_COST_TILE * n_kt + PF_COST_ITEM;
#pragma unroll
                for (int part = 0; part < 2; part++) {
                    const int a = part ? a2 : a1, end = min(a + (part ? x.c2 : x.c1), cut);
                    for (int rd = div_small(a, G); rd * G < end; rd++) {
                        const int p0 = max(a, rd * G) - rd * G, p1 = min(end, rd * G + G) - rd * G;
                        atomicAdd(&sched_load[(rd & 1) ? G - p1 : p0], cost);
                        atomicAdd(&sched_load[(rd & 1) ? G - p0 : p1], -cost);
                    }
                }
            });
            if (ranked) {
                __syncthreads();
                // Every wave ranks this workgroup by itself (no further barrier): lane l holds
                // the loads of workgroups 4l .. 4l+3, inclusive prefix sums of the differences.
                static_assert(PF_MAX_GRID <= 256, "four workgroups per lane");
                int x[4], local = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    x[j] = 4 * lane + j < G ? sched_load[4 * lane + j] : 0;
                    local += x[j];
                }
                int run = wave_incl_sum(local) - local;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    run += x[j];
                    x[j] = run;
                }
                const int jm = wg & 3;
                const int mine = __builtin_amdgcn_readlane(
                    jm == 0 ? x[0] : jm == 1 ? x[1] : jm == 2 ? x[2] : x[3], wg >> 2);
                int rank = 0;  // workgroups with less load, or as much and a lower index
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int b = 4 * lane + j;
                    rank += __popcll(__ballot(b < G && (x[j] < mine || (x[j] == mine && b < wg))));
                }
                if (__builtin_amdgcn_readfirstlane(rank) < total_items - cut) {
                    wg_items = rounds;
                    if (tid == 0) {
                        const int2 d = sched_last[rank];
                        put_entry_item(rounds - 1, d.x >> 20, d.y,
                                       entry_at(d.x & 2047, (d.x >> 11) & 511));
                    }
                }
            }
        } else {
            wg_items = items_of_wg(total_items);
        }
    } else {
        wg_items = 1;
    }
    if (!flex_on) {
        const int np_full = kv_heads * half_rep, np_lone = kv_heads * (n_rep & 1);
        for (int k = tid; k < wg_items; k += PF_THREADS) {
            int seq, level, kvh, h0;  // h0: the item's first head in its GQA group
            if (persistent) {
                const int idx = k * G + ((k & 1) ? G - 1 - wg : wg);
                const int n_full = np_full * total_base;
                const bool lone = idx >= n_full;
                const int ii = lone ? idx - n_full : idx;
                const int np = lone ? np_lone : np_full;
                const int key = ii / np;  // (level, sequence) pairs before this item in its part
                int lo = 0, hi = NQ - 1;  // last level L with sched_cum[L] <= key
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (sched_cum[mid] <= key) lo = mid; else hi = mid - 1;
                }
                level = lo;
                seq = sched_order[key - sched_cum[lo]];
                const int p = ii - np * key;
                kvh = lone ? p : p / half_rep;
                h0 = 2 * (lone ? half_rep : p - kvh * half_rep);
            } else {
                const int per_rank = num_seqs * npairs;
                level = wg / per_rank;
                const int r = wg - level * per_rank;
                seq = r / npairs;
                const int hp = r - seq * npairs;
                kvh = hp / pairs_per_kv;
                h0 = 2 * (hp - kvh * pairs_per_kv);
            }
            const bool ok = put_item(k, seq, level, kvh, h0, 1);
            if (!persistent) sched_nitems = ok ? 1 : 0;
        }
    }
    if (persistent && tid == 0) sched_nitems = wg_items;
    __syncthreads();
    const int n_items = __builtin_amdgcn_readfirstlane(sched_nitems);

    // A work item (all fields workgroup-uniform); valid == 0 past the end of the list.
    struct Item {
        int valid, seq, qt, kvh, h0, lg, q0, ql, kv_len, n_kt, last_page, vpage;
    };
    auto uni = [](int x) { return __builtin_amdgcn_readfirstlane(x); };
    auto fetch = [&](int k) __attribute__((always_inline)) {
        Item it{};
        if (k < n_items) {
            const int4 a = *reinterpret_cast<const int4*>(&sched_items[k][0]);
            const int4 b = *reinterpret_cast<const int4*>(&sched_items[k][4]);
            it.valid = 1;
            it.seq = uni(a.x);
            it.qt = uni(a.y);
            it.kvh = uni(a.z);
            it.h0 = uni(a.w & 0xffff);
            it.lg = uni(a.w >> 16);
            it.q0 = uni(b.x);
            it.ql = uni(b.y);
            it.kv_len = uni(b.z);
            it.n_kt = uni(b.w);
            // (page 0 for an empty sequence: its loads are all masked, its table row exists)
            it.last_page = it.kv_len > 0 ? (BS16 ? (it.kv_len - 1) >> 4 : (it.kv_len - 1) / block_size) : 0;
            if constexpr (DMA) it.vpage = it.seq * stage_pages;
        }
        return it;
    };

    // a wave's head in the item's group and its 32-row block: heads of 8 / hpi waves each
    // (hpi = 1 << lg heads per item). Waves w and w + 4 share a SIMD; the second four take their
    // row blocks in mirrored order, so that each SIMD holds one early and one late block: on an
    // item's last kv tiles, which only its later rows see, every SIMD then keeps one wave busy
    // instead of half the SIMDs two.
    auto wave_hl = [&](const Item& it) { return it.h0 + ((w << it.lg) >> 3); };
    auto wave_rb = [&](const Item& it) {
        const int nb = 8 >> it.lg;  // row blocks per head
        return w < 4 ? (w & (nb - 1)) : (nb - 1) - ((w - 4) & (nb - 1));
    };
    const int max_phys = (int)(num_slots / block_size - 1);
    const uint32_t head_bytes = (uint32_t)(num_slots * D * (int64_t)sizeof(T));

    // ---- staging assignment (a 64-token tile is four 16-token groups, each inside one page)
    // K: KPASS 16 B chunks per thread: token (tid / CPR) + RPP i of the tile, dims
    //    (tid % CPR) * 8 (head_dim 128: two chunks, rows tid / 16 and + 32; head_dim 64: one,
    //    row tid / 8); the group of each chunk, k_grp + (RPP / 16) i, is the same for the whole
    //    wave.
    // V: token pair tp = tid % 32 (tokens 2tp, 2tp+1), dims 8dg..8dg+7 with dg = tid / 32 (at
    //    head_dim 64 only waves 0-3, dg < 8, stage V); stored transposed, token t at column
    //    sigma16(t). Its group tp / 8 varies per lane.
    constexpr int RPP = PF_THREADS / CPR;  // K rows per staging pass
    constexpr int KPASS = PF_KT / RPP;
    const int k_row = tid / CPR, k_col = (tid % CPR) * 8;
    const int v_tp = tid & 31, v_dg = tid >> 5;
    const bool v_on = D == PF_D || v_dg < CPR;  // wave-uniform
    const int k_grp = (64 / CPR) * w / 16;
    constexpr uint32_t ROW_BYTES = D * sizeof(T);
    const uint32_t k_lane = (uint32_t)((k_row & 15) * D + k_col) * (uint32_t)sizeof(T);
    const uint32_t v_lane = (uint32_t)((2 * v_tp & 15) * D + 8 * v_dg) * (uint32_t)sizeof(T);
    const bool v_g1 = (v_tp >> 3) & 1, v_g2 = (v_tp >> 4) & 1;
    // DMA: wave w fills K rows 8w .. 8w+7 of the tile (all in group w / 2) with two 1 KB loads;
    // lane (r4, c) = (lane / 16, lane % 16) of load i reads row 8w + 4i + r4 (row r of the
    // group), 16-byte chunk c ^ r, which lands at chunk c of that row. For V, wave w copies half
    // w % 2 of page w / 2 of the tile (two 1 KB loads).
    uint32_t kdma_lane[2] = {0u, 0u};
    if constexpr (DMA) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int r = 8 * (w & 1) + 4 * i + (lane >> 4);
            kdma_lane[i] = (uint32_t)(r * (int)ROW_BYTES + ((lane & 15) ^ r) * 16);
        }
    }
    const __amdgpu_buffer_rsrc_t vst_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)v_stage, (short)0, (int)v_stage_bytes, BUF_DWORD3);

    // ---- load context: the item whose K / V tiles are being fetched
    __amdgpu_buffer_rsrc_t k_rsrc, v_rsrc;
    const int32_t* bt = block_tables;
    int kv_len = 0, last_page = 0, n_kt = 0, ld_vpage = 0, ld_kvh = 0;
    auto set_load = [&](const Item& it) {
        k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(k_pool + (int64_t)it.kvh * num_slots * D), (short)0, (int)head_bytes, BUF_DWORD3);
        v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(v_pool + (int64_t)it.kvh * num_slots * D), (short)0, (int)head_bytes, BUF_DWORD3);
        bt = block_tables + (int64_t)it.seq * max_blocks;
        kv_len = it.kv_len;
        last_page = it.last_page;
        n_kt = it.n_kt;
        ld_vpage = it.vpage;
        ld_kvh = it.kvh;
    };
    // Block ids reach the tile loads through a window of the block table held in VGPRs (lane
    // i: entry wbase + i in win_cur, wbase + 64 + i in win_next), refilled 64 entries ahead
    // with vector loads. Scalar loads would share the LDS wait counter, so every LDS wait of a
    // tile would also wait for them.
    uint32_t win_cur = 0, win_next = 0;
    uint32_t win_ld = 0;  // entries wbase + 128 + i once ld_ok: becomes win_next at the crossing
    int wbase = 0;
    bool ld_ok = false;
    auto load_window = [&](const int32_t* row, int base, int n_entries) __attribute__((always_inline)) {
        const int e = min(base + lane, n_entries - 1);  // entries past the last page are unused
        return (uint32_t)row[e];
    };
    // Byte offset (in the kv head's pool) of the first token of each group of tile kt
    // (workgroup-uniform). A bad block id is clamped into the pool; groups past kv_len reuse
    // the last page (their loads are masked off). Tiles are visited in non-decreasing order.
    auto page_bases = [&](int kt, int* pb) __attribute__((always_inline)) {
        const int lb0 = min(BS16 ? (kt * PF_KT) >> 4 : kt * PF_KT / block_size, last_page);
        // lb0 grows by at most PF_KT / block_size <= 4 pages a call (block_size is a multiple of
        // 16), so a call crosses at most one window, and the call before a crossing already
        // had lb0 + 4 - wbase >= 64 and issued the refill into win_ld. The crossing then only
        // moves values loaded at least one tile load earlier: a register move of a value that
        // is still the newest load in flight would wait for every tile load behind it.
        if (lb0 - wbase >= 64) {
            asm volatile("" ::: "memory");
            win_cur = win_next;
            win_next = win_ld;
            wbase += 64;
            ld_ok = false;
        }
        if (!ld_ok && lb0 + 4 - wbase >= 64) {
            win_ld = load_window(bt, wbase + 128, last_page + 1);
            ld_ok = true;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tok0 = kt * PF_KT + 16 * i;
            const int lb = min(BS16 ? (tok0 >> 4) : tok0 / block_size, last_page);
            // < 64 for 16-token pages (a tile's 4 ids are aligned); negative only for the
            // masked tiles before the first of an item with no kv tiles
            const int idx = max(lb - wbase, 0);
            int id;
            if (BS16 || idx < 64) {
                id = __builtin_amdgcn_readlane((int)win_cur, min(idx, 63));
            } else {
                asm volatile("" ::: "memory");
                id = __builtin_amdgcn_readlane((int)win_next, idx - 64);
            }
            const int phys = min(max(id, 0), max_phys);
            pb[i] = (int)((uint32_t)(phys * block_size + (tok0 - lb * block_size)) * ROW_BYTES);
        }
    };
    // Branch-free tile loads into (kd, vd): tokens past kv_len (or a tile past the last) get an
    // out-of-range offset and read zeros.
    auto gload_v = [&](int kt, const int* pb, bool valid, u32x4* vd) {
        // tile tokens t < lim_rel exist (none for the waves without V staging)
        const int lim_rel = (valid && v_on ? kv_len : 0) - kt * PF_KT;
        const int b01 = v_g1 ? pb[1] : pb[0], b23 = v_g1 ? pb[3] : pb[2];
        const uint32_t vb = (uint32_t)(v_g2 ? b23 : b01) + v_lane;
#pragma unroll
        for (int j = 0; j < 2; j++)
            vd[j] = __builtin_amdgcn_raw_buffer_load_b128(
                v_rsrc, 2 * v_tp + j < lim_rel ? vb + j * ROW_BYTES : PF_OOR, 0, BUF_NT);
    };
    // (kd, vd) from the kv head with pools krs / vrs; tile tokens t < lim_rel exist
    auto gload_to = [&](__amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs, int lim_rel,
                        const int* pb, u32x4* kd, u32x4* vd) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < KPASS; i++) {
            int kpb;
            if constexpr (D == PF_D) {
                kpb = k_grp ? pb[2 * i + 1] : pb[2 * i];
            } else {
                kpb = k_grp == 0 ? pb[0] : k_grp == 1 ? pb[1] : k_grp == 2 ? pb[2] : pb[3];
            }
            const uint32_t o = (uint32_t)kpb + k_lane;
            kd[i] = __builtin_amdgcn_raw_buffer_load_b128(
                krs, k_row + RPP * i < lim_rel ? o : PF_OOR, 0, 0);
        }
        const int b01 = v_g1 ? pb[1] : pb[0], b23 = v_g1 ? pb[3] : pb[2];
        const uint32_t vb = (uint32_t)(v_g2 ? b23 : b01) + v_lane;
        const int vlim = v_on ? lim_rel : 0;
#pragma unroll
        for (int j = 0; j < 2; j++)
            vd[j] = __builtin_amdgcn_raw_buffer_load_b128(
                vrs, 2 * v_tp + j < vlim ? vb + j * ROW_BYTES : PF_OOR, 0, BUF_NT);
    };
    auto gload = [&](int kt, const int* pb, bool valid, u32x4* kd, u32x4* vd) {
        gload_to(k_rsrc, v_rsrc, (valid ? kv_len : 0) - kt * PF_KT, pb, kd, vd);
    };
    // Register staging across items: an item of at least 3 tiles that has a successor loads
    // that item's tile j as its own tile pf_base + j (pf_base: its tile count rounded up to
    // even, so that tile 0 arrives in register set A and LDS buffer 0 like a first tile). The
    // successor's kv head, kv length and last page; pf_base is 2^30 without one.
    int pf_base = 1 << 30, nx_kvh = 0, nx_kv_len = 0, nx_last_page = 0;
    const int64_t head_elems = num_slots * D;
    // page byte offsets of the successor's tile j (j <= 2: inside its first window `win`)
    auto page_nx = [&](int j, int* pb, uint32_t win) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tok0 = j * PF_KT + 16 * i;
            const int lb = min(BS16 ? tok0 >> 4 : tok0 / block_size, nx_last_page);
            const int id = __builtin_amdgcn_readlane((int)win, lb);
            const int phys = min(max(id, 0), max_phys);
            pb[i] = (int)((uint32_t)(phys * block_size + (tok0 - lb * block_size)) * ROW_BYTES);
        }
    };
    // DMA: tile kt's K into buffer b (rows past kv_len read zeros) and, outside exact mode, its
    // V pages from the staging copy.
    auto dma_tile = [&](auto ex, int kt, const int* pb, int b) __attribute__((always_inline)) {
        const int lim_rel = kv_len - kt * PF_KT;
        const int g = w >> 1;  // this wave's 16-token group
        const int pgb = g == 0 ? pb[0] : g == 1 ? pb[1] : g == 2 ? pb[2] : pb[3];
        const uint32_t kdst = lds_byte_addr(kb_ptr(b)) + (uint32_t)w * 2048u;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int row = 8 * w + 4 * i + (lane >> 4);
            dma_b128(row < lim_rel ? kdma_lane[i] : PF_OOR, k_rsrc, kdst + 1024u * i, (uint32_t)pgb);
        }
        if constexpr (!decltype(ex)::value) {
            const uint32_t vdst = lds_byte_addr(vb_ptr(b)) + (uint32_t)w * 2048u;
            const uint32_t vso =
                (uint32_t)((ld_vpage + 4 * kt + g) * kv_heads + ld_kvh) * (uint32_t)PF_VPAGE_BYTES +
                (uint32_t)(w & 1) * 2048u;
#pragma unroll
            for (int i = 0; i < 2; i++)
                dma_b128((uint32_t)lane * 16u + 1024u * i, vst_rsrc, vdst + 1024u * i, vso);
        }
    };
    // `ex` true: exact mode, V is stored as bf16 without widening
    auto lds_store_v = [&](auto ex, int buf, u32x4* vd) {
        if (!v_on) return;  // head_dim 64: waves 4-7 stage no V
        const int col = sigma16(2 * v_tp);  // the pair stays adjacent under sigma16
        // V^T row 8 v_dg + e holds dim 8 v_dg + e of the thread's two tokens as one dword
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int wd = e >> 1;
            uint32_t pr;
            if constexpr (CHECK_V && !decltype(ex)::value) {
                // bf16 V to fp16 (exact for 2^-17 <= |v| <= 65504 and 0), packed straight into
                // the token pair of one dim: no permute after the conversion
                pr = (e & 1) ? pack2<f16_t>(hi_f32<bf16_t>(vd[0][wd]), hi_f32<bf16_t>(vd[1][wd]))
                             : pack2<f16_t>(lo_f32<bf16_t>(vd[0][wd]), lo_f32<bf16_t>(vd[1][wd]));
            } else {
                pr = (e & 1) ? perm_hi16(vd[0][wd], vd[1][wd]) : perm_lo16(vd[0][wd], vd[1][wd]);
            }
            *reinterpret_cast<uint32_t*>(&vb_ptr(buf)[(8 * v_dg + e) * PF_VPITCH + col]) = pr;
        }
    };
    auto lds_store = [&](auto ex, int buf, u32x4* kd, u32x4* vd) {
#pragma unroll
        for (int i = 0; i < KPASS; i++)
            *reinterpret_cast<u32x4*>(&kb_ptr(buf)[(k_row + RPP * i) * KPITCH + k_col]) = kd[i];
        lds_store_v(ex, buf, vd);
    };

    // ---- per-item compute state (the item whose tile the workgroup is computing)
    int head = 0, q0 = 0, ql = 0, wr0 = 0, lim = 0, wave_lim = 0, wave_min_lim = 0;
    bool wave_active = false;
    auto set_compute = [&](const Item& it) {
        const int hl = wave_hl(it);
        head = it.kvh * n_rep + hl;
        q0 = it.q0;
        ql = it.ql;
        const int off = it.kv_len - it.ql;
        wr0 = it.qt * PF_QT + 32 * wave_rb(it);
        wave_active = hl < n_rep && wr0 < it.ql;
        lim = off + min(wr0 + ql32, it.ql - 1);        // this lane's row sees kv j <= lim
        wave_lim = off + min(wr0 + 31, it.ql - 1);     // largest limit in the wave
        wave_min_lim = off + wr0;                      // smallest limit in the wave
    };
    // Q^T as the B operand: lane (h2, q) holds row q, dims 16kk + 8h2 .. +7 (idle waves and
    // padded rows read a valid row)
    u32x4 qb[NKQ];
    auto load_q = [&](const Item& it) __attribute__((always_inline)) {
        const int hq = it.kvh * n_rep + min(wave_hl(it), n_rep - 1);
        const int row = min(it.qt * PF_QT + 32 * wave_rb(it) + ql32, it.ql - 1);
        const T* qp = q + (int64_t)(it.q0 + row) * q_st + (int64_t)hq * q_sh + 8 * h2;
#pragma unroll
        for (int kk = 0; kk < NKQ; kk++) qb[kk] = *reinterpret_cast<const u32x4*>(qp + 16 * kk);
    };
    // Register staging: an item's Q rows reach this wave's staging block straight from memory
    // (D / 16 loads of 1 KB issued an item ahead, no registers held), then qb comes from LDS.
    // Lane (r, c) = (lane / CPR, lane % CPR) of load i reads chunk c ^ (row % CPR) of row
    // (64 / CPR) i + r, clamped to the sequence's last row like load_q.
    uint16_t* const qstage = reinterpret_cast<uint16_t*>(sched_raw) + w * PF_QSTAGE_ELEMS;
    auto dma_q = [&](const Item& it) __attribute__((always_inline)) {
        const int hq = it.kvh * n_rep + min(wave_hl(it), n_rep - 1);
        const int row0 = it.qt * PF_QT + 32 * wave_rb(it);
        const int rb = min(row0, it.ql - 1);
        const T* qp = q + (int64_t)(it.q0 + rb) * q_st + (int64_t)hq * q_sh;
        const __amdgpu_buffer_rsrc_t q_rsrc =
            __builtin_amdgcn_make_buffer_rsrc((void*)qp, (short)0, (int)0x7fffffff, BUF_DWORD3);
        const uint32_t qs = lds_byte_addr(qstage);
#pragma unroll
        for (int i = 0; i < NKQ; i++) {
            const int r = (64 / CPR) * i + lane / CPR;
            const int row = min(row0 + r, it.ql - 1) - rb;
            const uint32_t off = (uint32_t)row * (uint32_t)(q_st * (int64_t)sizeof(T)) +
                                 (uint32_t)(((lane % CPR) ^ (r % CPR)) * 16);
            dma_b128(off, q_rsrc, qs + 1024u * i, 0u);
        }
    };
    // qb from the staging block (the loads that filled it must be complete)
    auto read_q = [&]() __attribute__((always_inline)) {
        const uint16_t* qr = qstage + ql32 * D;
#pragma unroll
        for (int kk = 0; kk < NKQ; kk++)
            qb[kk] = *reinterpret_cast<const u32x4*>(qr + 8 * ((2 * kk + h2) ^ (ql32 % CPR)));
    };

    // Running state: the reference max m may lag the true running max by up to
    // PF_RESCALE_SLACK (weights then reach 2^8), which skips most accumulator rescales.
    float m = -INFINITY, lsum = 0.0f;
    f32x16 o[NMT];
    auto reset_state = [&]() {
        m = -INFINITY;
        lsum = 0.0f;
#pragma unroll
        for (int x = 0; x < NMT; x++)
#pragma unroll
            for (int y = 0; y < 16; y++) o[x][y] = 0.0f;
    };
    // ---- epilogue: lane (h2, q) holds dims 32 mt2 + 8 i + 4 h2 + j of query row wr0 + q
    auto store_output = [&](int sbuf) __attribute__((always_inline)) {
        const float l = sum_across_halves(lsum);
        if (wave_active) {
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;  // 0: an item that attends nothing
            if constexpr (sizeof(TO) == 4) {
                const int orow = wr0 + ql32;
                if (orow < ql) {
                    TO* op = out + (int64_t)(q0 + orow) * o_st + (int64_t)head * o_sh + 4 * h2;
#pragma unroll
                    for (int mt2 = 0; mt2 < NMT; mt2++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const f32x4 v = f32x4{o[mt2][4 * i] * inv, o[mt2][4 * i + 1] * inv,
                                                  o[mt2][4 * i + 2] * inv, o[mt2][4 * i + 3] * inv};
                            if constexpr (DMA)
                                *reinterpret_cast<f32x4*>(op + 32 * mt2 + 8 * i) = v;
                            else
                                gstore_b128(op + 32 * mt2 + 8 * i, __builtin_bit_cast(u32x4, v));
                        }
                }
            } else {
                // 16-bit output goes through LDS (DMA: tile buffer sbuf, idle until a barrier
                // that comes before its next fill; register staging: this wave's Q staging
                // block, whose rows are in qb by now) in 64-dim halves, so that each store
                // writes whole 128 B row segments: lane (r, c) = (lane / 8, lane % 8) stores
                // dims 8c .. 8c + 7 of rows r, r + 8, r + 16, r + 24.
                uint16_t* stg = DMA ? kb_ptr(sbuf) + w * (32 * PF_OPITCH) : qstage;
                const int rr = lane >> 3, cc = lane & 7;
                TO* ob = out + (int64_t)(q0 + wr0) * o_st + (int64_t)head * o_sh + 8 * cc;
#pragma unroll
                for (int half = 0; half < D / 64; half++) {
#pragma unroll
                    for (int mt = 0; mt < 2; mt++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const f32x16& x = o[2 * half + mt];
                            *reinterpret_cast<u32x2*>(&stg[ql32 * PF_OPITCH + 32 * mt + 8 * i + 4 * h2]) =
                                u32x2{pack2<TO>(x[4 * i] * inv, x[4 * i + 1] * inv),
                                      pack2<TO>(x[4 * i + 2] * inv, x[4 * i + 3] * inv)};
                        }
                    // the four row reads go out together (one LDS wait), then the stores
                    u32x4 rowv[4];
#pragma unroll
                    for (int s4 = 0; s4 < 4; s4++) {
                        const uint16_t* src = &stg[(rr + 8 * s4) * PF_OPITCH + 8 * cc];
                        const u32x2 lo = *reinterpret_cast<const u32x2*>(src);
                        const u32x2 hi = *reinterpret_cast<const u32x2*>(src + 4);
                        rowv[s4] = u32x4{lo[0], lo[1], hi[0], hi[1]};
                    }
#pragma unroll
                    for (int s4 = 0; s4 < 4; s4++) asm volatile("" ::"v"(rowv[s4]));
#pragma unroll
                    for (int s4 = 0; s4 < 4; s4++) {
                        const int r = rr + 8 * s4;
                        if (wr0 + r < ql) {
                            TO* dst = ob + (int64_t)r * o_st + 64 * half;
                            if constexpr (DMA)
                                *reinterpret_cast<u32x4*>(dst) = rowv[s4];
                            else
                                gstore_b128(dst, rowv[s4]);
                        }
                    }
                }
            }
        }
    };

    // S^T of the tile in flight (64 tokens x 32 queries, two 32-token halves, raw q.k).
    f32x16 st[2];
    auto visible = [&](int kt) { return wave_active && kt * PF_KT <= wave_lim; };  // per wave
    // ---- S^T tile (64 tokens x 32 queries) in two 32-token halves, raw q.k: 16 products in
    // kk-major order alternating the halves (two independent accumulation chains), K fragments
    // read four products ahead. `fill` is work independent of the scores (the staging of the
    // next tile) that the products are interleaved with.
    auto qk = [&](int kbuf, auto&& fill) __attribute__((always_inline)) {
        const uint16_t* kr = DMA ? kb_ptr(kbuf) + ql32 * D : kb_ptr(kbuf) + ql32 * KPITCH + 8 * h2;
        auto frag = [&](int i) {  // product i: half i & 1, dims 16 (i >> 1) .. of the K rows
            if constexpr (DMA) {
                // 16-byte chunk 2 (i >> 1) + h2 of row ql32 + 32 (i & 1), stored at chunk
                // (2 (i >> 1) + h2) ^ (ql32 % 16)
                return *reinterpret_cast<const u32x4*>(
                    kr + (i & 1) * 32 * D + 8 * ((2 * (i >> 1) + h2) ^ (ql32 & 15)));
            } else {
                return *reinterpret_cast<const u32x4*>(kr + (i & 1) * 32 * KPITCH + 16 * (i >> 1));
            }
        };
        constexpr int NP = 2 * NKQ;  // products: two 32-token halves x the k-steps
        u32x4 fr[NP];
#pragma unroll
        for (int i = 0; i < 4; i++) fr[i] = frag(i);
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int y = 0; y < 16; y++) st[mt][y] = 0.0f;
        __builtin_amdgcn_sched_barrier(0);
        // The matrix sections run at raised wave priority: when both waves of a SIMD are ready,
        // the one feeding MFMAs issues first and the other's VALU work fills behind it
        // (measured +2% on the Llama-3-8B batch, +3.5% on the prefix batch).
        __builtin_amdgcn_s_setprio(1);
        fill();
#pragma unroll
        for (int i = 0; i < NP; i++) {
            if (i + 4 < NP) fr[i + 4] = frag(i + 4);
            st[i & 1] = mfma32x32x16<T>(fr[i], qb[i >> 1], st[i & 1]);
        }
#pragma unroll
        for (int i = 0; i < NP; i++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // a K fragment read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one product
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // up to three VALU
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // up to one LDS write
        }
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
    };
    // ---- mask, tile max and lazy rescale of tile kt's scores; `slack` is how far (in log2
    // units) the reference max may lag the running max.
    auto softmax_max = [&](int kt, float slack) __attribute__((always_inline)) {
        const int kv0 = kt * PF_KT;
        // mask, on tiles that cross the diagonal of some row of this wave only. The empty asm
        // statements keep the compiler from if-converting these uniform branches into
        // per-element selects on every tile.
        if (kv0 + PF_KT - 1 > wave_min_lim) {
            asm volatile("" ::: "memory");
            const int tl = lim - kv0 - 4 * h2;  // token offset 32mt + 8i + j visible iff <= tl
            // bit p of vis[mt]: offset 32 mt + p visible. Each score then takes a sign-extended
            // bit extract and a bit-field select (two VALU, no scalar masks: 32 compares into
            // scalar masks used to spill scalar registers here).
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                const int width = min(max(tl + 1 - 32 * mt, 0), 32);
                const uint32_t vis = width >= 32 ? 0xffffffffu : (1u << width) - 1u;
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t keep = (uint32_t)__builtin_amdgcn_sbfe((int)vis, 8 * i + j, 1);
                        const uint32_t b = __float_as_uint(st[mt][4 * i + j]);
                        st[mt][4 * i + j] = __uint_as_float((b & keep) | (0xff800000u & ~keep));
                    }
            }
        }
        // tile max of the raw scores (scale > 0, so the max commutes with the scaling)
        float tm[2] = {-INFINITY, -INFINITY};
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int y = 0; y < 16; y += 2) tm[mt] = vmax(vmax(tm[mt], st[mt][y]), st[mt][y + 1]);
        const float tmax = max_across_halves(vmax(tm[0], tm[1])) * scale_log2;
        if (__builtin_amdgcn_ballot_w64(tmax > m + slack) != 0) {
            asm volatile("" ::: "memory");
            const float m_new = fmaxf(m, tmax);
            const float alpha = fast_exp2(m - m_new);
            lsum *= alpha;
#pragma unroll
            for (int x = 0; x < NMT; x++) o[x] *= alpha;
            m = m_new;
        }
    };
    auto sm_pv = [&](int kt, int vbuf) __attribute__((always_inline)) {
        softmax_max(kt, PF_RESCALE_SLACK);
        // ---- p = 2^(s * scale_log2 - m), one FMA + exp per score, packed as the P^T B operand
        // of step kk2 (tokens of half kk2/2, rows i = 2(kk2&1), +1); then O^T += V^T P^T in
        // kk2-major order, so that the exps of step kk2+1 and the V reads of step kk2+1 can run
        // under the matrix products of step kk2. The row sum is taken over the rounded weights
        // that enter the product (v_dot2 over fp16 pairs) in PV_F16 mode.
        const float nm = -m;
        u32x4 pb_hi[4], pb_lo[4];
        float psum = 0.0f;
        // weights of step kk2, rows 2x and 2x+1 of the P^T B operand
        auto weight = [&](int kk2, int x) __attribute__((always_inline)) {
            const int mt = kk2 >> 1, y0 = 8 * (kk2 & 1);
            const float a0 = fast_exp2(fmaf(st[mt][y0 + 2 * x], scale_log2, nm));
            const float a1 = fast_exp2(fmaf(st[mt][y0 + 2 * x + 1], scale_log2, nm));
            const uint32_t hi = pack2<TV>(a0, a1);
            pb_hi[kk2][x] = hi;
            if constexpr (PV == PV_HILO) {
                pb_lo[kk2][x] = pack2<TV>(a0 - lo_f32<TV>(hi), a1 - hi_f32<TV>(hi));
                psum += a0 + a1;
            } else {
                psum = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, hi), f16x2{1, 1}, psum,
                                              false);
            }
        };
        // Issue order, pinned with scheduling fences: the V reads and weights of step 0, then
        // each product of step kk2 followed by one V read and its share of the weights of
        // step kk2 + 1 (a quarter at head_dim 128, a half at 64).
        // V^T fragment (dims 32 mt2 + ql32, tokens 8 h2 .. of group kk2): register staging keeps
        // V^T rows with a 144 B pitch; the DMA path has four 4 KB pages (128 dims x 16 tokens)
        const uint16_t* vr = DMA ? vb_ptr(vbuf) + ql32 * 16 + 8 * h2 : vb_ptr(vbuf) + ql32 * PF_VPITCH + 8 * h2;
        auto vfrag = [&](int mt2, int kk2) {
            return *reinterpret_cast<const u32x4*>(
                DMA ? vr + kk2 * (16 * D) + mt2 * 512 : vr + 32 * mt2 * PF_VPITCH + 16 * kk2);
        };
        u32x4 vf[2][NMT];
#pragma unroll
        for (int mt2 = 0; mt2 < NMT; mt2++) vf[0][mt2] = vfrag(mt2, 0);
#pragma unroll
        for (int x = 0; x < 4; x++) weight(0, x);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kk2 = 0; kk2 < 4; kk2++) {
#pragma unroll
            for (int mt2 = 0; mt2 < NMT; mt2++) {
                o[mt2] = mfma32x32x16<TV>(vf[kk2 & 1][mt2], pb_hi[kk2], o[mt2]);
                if constexpr (PV == PV_HILO)
                    o[mt2] = mfma32x32x16<TV>(vf[kk2 & 1][mt2], pb_lo[kk2], o[mt2]);
                if (kk2 < 3) {
                    vf[(kk2 + 1) & 1][mt2] = vfrag(mt2, kk2 + 1);
#pragma unroll
                    for (int x = mt2 * (4 / NMT); x < (mt2 + 1) * (4 / NMT); x++) weight(kk2 + 1, x);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        lsum += psum;
    };
    // Exact-mode softmax and P.V of tile kt over a bf16 V^T tile: exact running max, P split
    // into bf16 hi + lo, one k-step at a time (the rare path; few live registers).
    auto sm_pv_exact = [&](int kt, int vbuf) __attribute__((always_inline)) {
        softmax_max(kt, 0.0f);
        const float nm = -m;
        float psum = 0.0f;
        const uint16_t* vr = vb_ptr(vbuf) + ql32 * PF_VPITCH + 8 * h2;
#pragma unroll
        for (int kk2 = 0; kk2 < 4; kk2++) {
            const int mt = kk2 >> 1, y0 = 8 * (kk2 & 1);
            u32x4 ph, pl;
#pragma unroll
            for (int x = 0; x < 4; x++) {
                const float a0 = fast_exp2(fmaf(st[mt][y0 + 2 * x], scale_log2, nm));
                const float a1 = fast_exp2(fmaf(st[mt][y0 + 2 * x + 1], scale_log2, nm));
                const uint32_t hi = pack2<T>(a0, a1);
                ph[x] = hi;
                pl[x] = pack2<T>(a0 - lo_f32<T>(hi), a1 - hi_f32<T>(hi));
                psum += a0 + a1;
            }
#pragma unroll
            for (int mt2 = 0; mt2 < NMT; mt2++) {
                const u32x4 vv = *reinterpret_cast<const u32x4*>(vr + 32 * mt2 * PF_VPITCH + 16 * kk2);
                o[mt2] = mfma32x32x16<T>(vv, ph, o[mt2]);
                o[mt2] = mfma32x32x16<T>(vv, pl, o[mt2]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        lsum += psum;
    };

    // ---- items. Within an item, one barrier per tile: global loads run two tiles ahead of the
    // compute (register sets A / B alternate), LDS double-buffered, page ids three tiles ahead.
    // Across items (register staging): the next item's Q rows go to the staging block at the
    // start of the current one, and an item of 3 or more tiles loads the next item's tiles 0
    // and 1 in its last steps, so an item boundary costs its output store and no memory round
    // trip (measured ~5,900 cycles instead of ~11,600 per item on the Llama-3-8B batch). The DMA
    // kernel fetches the next item's Q and first tiles while the epilogue stores the output.
    if (n_items == 0) return;
    u32x4 ka[2], va[2], kb[2], vb[2];
    int pb0[4], pb1[4], pb2[4];
    // DMA: the buffers rotate over the tiles of consecutive items; buf0 is the buffer of the
    // first tile of the item in the load context
    int buf0 = 0;
    auto next_buf = [](int b) { return b == NBUF - 1 ? 0 : b + 1; };
    auto prev_buf = [](int b) { return b == 0 ? NBUF - 1 : b - 1; };
    // the first tiles of the item in the load context: tiles 0 and 1 in flight, page ids of
    // tile 2 ready, the block-table window at the start (win_cur must hold entries 0..63; the
    // caller loads win_next, entries 64..127)
    auto start_window = [&](uint32_t win) __attribute__((always_inline)) {
        wbase = 0;
        ld_ok = false;
        win_cur = win;
    };
    auto start_tiles = [&](auto ex) __attribute__((always_inline)) {
        page_bases(0, pb0);
        if constexpr (DMA) {
            if (0 < n_kt) dma_tile(ex, 0, pb0, buf0);
            if constexpr (decltype(ex)::value) gload_v(0, pb0, true, va);
        } else {
            gload(0, pb0, true, ka, va);
        }
        page_bases(min(1, n_kt - 1), pb1);
        if constexpr (DMA) {
            if (1 < n_kt) dma_tile(ex, 1, pb1, next_buf(buf0));
            if constexpr (decltype(ex)::value) gload_v(1, pb1, 1 < n_kt, vb);
        } else {
            gload(1, pb1, 1 < n_kt, kb, vb);
        }
        page_bases(min(2, n_kt - 1), pb2);
    };
    // `win`: the item's first block-table window, loaded well before (a register move of a
    // load still in flight would wait for it)
    // `staged`: register staging after the first item (Q is in the staging block already)
    auto prologue = [&](const Item& it, uint32_t win, bool staged) __attribute__((always_inline)) {
        const int n_kt_done = n_kt;  // tiles of the item whose loads are in flight
        set_load(it);
        if constexpr (DMA) {
            load_q(it);
        } else {
            if (staged) {
                // the staging loads were issued before the last step's tile loads, which leave
                // at most four younger loads in flight; an item without steps issued none
                // after them
                if (n_kt_done > 0)
                    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
                else
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            } else {  // the first item: through the staging block as well (one wait)
                dma_q(it);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            read_q();
        }
        start_window(win);
        start_tiles(std::false_type{});
    };
    // first window of item k, or of the last sequence's row if there is none (a valid address)
    auto window_of = [&](const Item& it) __attribute__((always_inline)) {
        return load_window(block_tables + (int64_t)(it.valid ? it.seq : 0) * max_blocks, 0,
                           it.last_page + 1);
    };
    auto item_window = [&](int k) __attribute__((always_inline)) { return window_of(fetch(k)); };
    // Item-end check of the fp16 path (CHECK_V): true if this wave's output block (its valid
    // rows) is not finite or its root mean square is below PF_MIN_TRUSTED_RMS. Lane (h2, q)
    // holds 16 NMT outputs of row q, all scaled by the row's 1 / l.
    auto block_untrusted = [&]() __attribute__((always_inline)) {
        float ss = 0.0f;
#pragma unroll
        for (int x = 0; x < NMT; x++)
#pragma unroll
            for (int y = 0; y < 16; y++) ss = fmaf(o[x][y], o[x][y], ss);
        const float l = sum_across_halves(lsum);
        const bool row_ok = wr0 + ql32 < ql;
        const bool nonfinite = !(ss < INFINITY);  // NaN compares false
        // sum over the valid rows of the block of (outputs)^2
        float blk = row_ok && l > 0.0f ? ss / (l * l) : 0.0f;
        blk = wave_sum(blk);
        const float n = (float)(__popcll(__builtin_amdgcn_ballot_w64(row_ok)) * 16 * NMT);
        const bool small = !(blk >= n * PF_MIN_TRUSTED_RMS * PF_MIN_TRUSTED_RMS);
        return wave_active && (__builtin_amdgcn_ballot_w64(nonfinite) != 0 || small);
    };
    Item ci = fetch(0);
    prologue(ci, item_window(0), false);
    win_next = load_window(bt, 64, last_page + 1);
    set_compute(ci);
    // register staging: how the current item's first tiles arrived. 0: tiles 0 and 1 in flight
    // (start_tiles); 1: tile 0 in set A from the previous item, tile 1 not loaded, page ids of
    // tile 1 in pb2; 2: tile 0 in LDS buffer 0 (published), tile 1 in flight in set B, page
    // ids of tile 2 in pb2
    int state = 0;
    for (int k = 0;;) {
        uint32_t win_nx = 0;  // first window of item k + 1, loaded during item k's first tile
        // compute tile kt from LDS buffer bc; `ex`: exact mode. On the fp16 path the last step
        // records this wave's item-end check before its barrier, which publishes it.
        auto compute = [&](auto ex, int kt, int bc) __attribute__((always_inline)) {
            constexpr bool EX = decltype(ex)::value;
            if (visible(kt)) {
                qk(bc, [] {});
                if constexpr (EX)
                    sm_pv_exact(kt, bc);
                else
                    sm_pv(kt, bc);
            }
            if constexpr (CHECK_V && !EX) {
                if (kt == n_kt - 1) redo_flag[PF_WAVES * (k & 1) + w] = block_untrusted() ? 1 : 0;
            }
        };
        auto rotate_pages = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < 4; i++) {  // pb2 <- tile kt + 3
                const int x = pb2[i];
                pb2[i] = pb0[i];
                pb0[i] = x;
            }
        };
        // register staging, step kt: refill `nx` with tile kt + 2, compute tile kt, store tile
        // kt + 1 (in `st1`).
        auto step = [&](auto ex, int kt, u32x4* knx, u32x4* vnx, u32x4* kst1,
                        u32x4* vst1) __attribute__((always_inline)) {
            gload(kt + 2, pb2, kt + 2 < n_kt, knx, vnx);
            page_bases(min(kt + 3, n_kt - 1), pb0);
            compute(ex, kt, kt & 1);
            lds_store(ex, (kt + 1) & 1, kst1, vst1);
            rotate_pages();
            __syncthreads();
        };
        // register staging, cross-item step kt (tile kt in LDS buffer bc): as `step`, but the
        // loads are the successor's tile j (whose page ids are in pb2) and the page ids
        // computed are its tile j + 1's
        auto step_x = [&](int kt, int bc, int j, u32x4* knx, u32x4* vnx, u32x4* kst1,
                          u32x4* vst1) __attribute__((always_inline)) {
            gload(j, pb2, true, knx, vnx);
            page_nx(j + 1, pb0, win_nx);
            compute(std::false_type{}, kt, bc);
            lds_store(std::false_type{}, 1 - bc, kst1, vst1);
            rotate_pages();
            __syncthreads();
        };
        // DMA, step kt with tile kt in buffer bc: tile kt + 2 goes to the buffer of tile kt - 1
        // (free since the last barrier), then tile kt is computed and the wait for tile kt + 1
        // (the oldest loads in flight) precedes the barrier. The page ids of tile kt + 3 come
        // first: a block-table window move waits for every load in flight, and at that point
        // the newest are tile kt + 1's, due before the barrier anyway. In exact mode V goes
        // through registers (tile kt + 2 loaded, tile kt + 1 written to LDS).
        auto step_dma = [&](auto ex, int kt, int bc, u32x4* vnx, u32x4* vst1) __attribute__((always_inline)) {
            constexpr bool EX = decltype(ex)::value;
            page_bases(min(kt + 3, n_kt - 1), pb0);
            const bool more = kt + 2 < n_kt;
            if (more) dma_tile(ex, kt + 2, pb2, prev_buf(bc));
            if constexpr (EX) gload_v(kt + 2, pb2, more, vnx);
            compute(ex, kt, bc);
            if constexpr (EX) lds_store_v(ex, next_buf(bc), vst1);
            rotate_pages();
            if constexpr (EX) {
                asm volatile("s_waitcnt vmcnt(2)" ::: "memory");  // all but tile kt + 2's V
            } else if (more) {
                asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // all but tile kt + 2's
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            __syncthreads();
        };
        // all tiles of the current item, from tiles 0 and 1 in flight (start_tiles). Outside
        // exact mode the next item's first window is loaded along the way: on the DMA path
        // before the first wait (every explicit count leaves only younger loads outstanding),
        // on the register path after the first barrier (the compiler waits for all loads
        // there).
        auto run_tiles = [&](auto ex, int st0) __attribute__((always_inline)) {
            constexpr bool EX = decltype(ex)::value;
            reset_state();
            if constexpr (DMA && !EX) win_nx = item_window(k + 1);
            // Q must have landed before the loop (its loads precede the tile loads, so this
            // waits for them alone); otherwise the compiler sinks the Q loads past the first
            // barrier and keeps a conservative wait for them inside the loop
#pragma unroll
            for (int kk = 0; kk < 8; kk++) asm volatile("" ::"v"(qb[kk]));
            if constexpr (DMA) {
                if constexpr (EX) {
                    lds_store_v(ex, buf0, va);
                    asm volatile("s_waitcnt vmcnt(2)" ::: "memory");  // all but tile 1's V
                } else if (1 < n_kt) {
                    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // all but tile 1's
                } else {
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                }
                __syncthreads();
                int bc = buf0;
                for (int kt = 0; kt < n_kt; kt += 2) {
                    step_dma(ex, kt, bc, va, vb);
                    bc = next_buf(bc);
                    if (kt + 1 < n_kt) {
                        step_dma(ex, kt + 1, bc, vb, va);
                        bc = next_buf(bc);
                    }
                }
                buf0 = bc;
            } else {
                if (!EX && st0 == 1) {  // tile 0 came with the previous item; tile 1 now
                    gload(1, pb2, 1 < n_kt, kb, vb);
                    page_bases(min(2, n_kt - 1), pb2);
                }
                if (EX || st0 != 2) {
                    lds_store(ex, 0, ka, va);
                    __syncthreads();
                }
                if constexpr (!EX) {
                    // the next item's Q rows into the staging block, once this wave's reads
                    // of it (Q, output staging) are complete; its first window and, for an
                    // item of 3 tiles or more, the cross-item loads
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    const Item nq = fetch(k + 1);
                    if (nq.valid) dma_q(nq);
                    win_nx = window_of(nq);
                    pf_base = (nq.valid && n_kt >= 3) ? n_kt + (n_kt & 1) : (1 << 30);
                    nx_kvh = nq.kvh;
                    nx_kv_len = nq.kv_len;
                    nx_last_page = nq.last_page;
                }
                // with a successor to load, the loop stops two tiles short of pf_base (an even
                // count) and the remaining one or two steps load its tiles 0 and 1: tile
                // pf_base - 2 + i runs from set A / buffer 0 for even i
                const int n_main = (!EX && pf_base < (1 << 30)) ? pf_base - 2 : n_kt;
                for (int kt = 0; kt < n_main; kt += 2) {
                    step(ex, kt, ka, va, kb, vb);
                    if (kt + 1 < n_main) step(ex, kt + 1, kb, vb, ka, va);
                }
                if constexpr (!EX) {
                    if (n_main < n_kt) {
                        // the successor's pool resources and kv length from here on (a redo
                        // restores this item's)
                        k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
                            (void*)(k_pool + nx_kvh * head_elems), (short)0, (int)head_bytes, BUF_DWORD3);
                        v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
                            (void*)(v_pool + nx_kvh * head_elems), (short)0, (int)head_bytes, BUF_DWORD3);
                        kv_len = nx_kv_len;
                        page_nx(0, pb2, win_nx);
                        // even n_kt: tiles 0 and 1 (sets A, B); odd: tile 0 (set A) only
                        step_x(n_main, 0, 0, ka, va, kb, vb);
                        if (n_main + 1 < n_kt) step_x(n_main + 1, 1, 1, kb, vb, ka, va);
                    }
                }
            }
        };
        run_tiles(std::false_type{}, state);
        bool redo = false;
        if constexpr (CHECK_V) {
            if (n_kt > 0) {  // flags written before the last step's barrier
                const u32x2 f = *reinterpret_cast<const u32x2*>(&redo_flag[PF_WAVES * (k & 1)]);
                redo = uni((int)(f[0] | f[1])) != 0;
            }
            if (redo) {  // the whole item again in exact mode (every wave, uniform branch)
                set_load(fetch(k));  // the cross-item loads may have switched the resources
                start_window(load_window(bt, 0, last_page + 1));
                win_next = load_window(bt, 64, last_page + 1);
                start_tiles(std::true_type{});
                run_tiles(std::true_type{}, 0);
            }
        }
        // output staging (DMA): the buffer of the item's last tile (the next item's first tiles
        // go to the two after it); register staging stages through the wave's Q block
        const int sbuf = DMA ? prev_buf(buf0) : 0;
        // register staging: the next item's first tiles are in flight if this one loaded them
        // (a redo reloaded the buffers and registers)
        const int nstate = (!DMA && !redo && pf_base < (1 << 30)) ? ((n_kt & 1) ? 1 : 2) : 0;
        const Item nx = fetch(++k);
        if (nx.valid) {
            if (nstate != 0) {
                set_load(nx);
                // the staging loads precede the last step's four tile loads
                asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
                read_q();
                start_window(win_nx);
            } else {
                prologue(nx, win_nx, true);
            }
            win_next = load_window(bt, 64, last_page + 1);
        }
        store_output(sbuf);
        if (!nx.valid) break;
        set_compute(nx);
        state = nstate;
    }
}

// Staging copy of V for the DMA kernel: every 16-token page of each sequence's kv range,
// rounded up to whole 64-token tiles, as V^T in fp16 (128 dims x 16 tokens, token sigma16(k) at
// position k; bf16 values converted as on the register-staged path), tokens
// past kv_len zero. Page p of sequence s and kv head h is at ((s * P + p) * kv_heads + h) * 4 KB,
// P = 4 * ceil(max_blocks * block_size / 64) pages per sequence (the block table's capacity in
// whole tiles). One four-wave workgroup per 64-token tile, one wave per page; tiles past a
// sequence's kv range exit at once. The kv length and the page's block id are loaded
// independently, so a page costs two dependent memory round trips (ids, then rows) before its
// store, and every load and store instruction moves whole 256 B rows or 1 KB runs.
template <typename T>
__global__ __launch_bounds__(256) void prefill_v_stage_kernel(
    f16_t* __restrict__ ws, const T* __restrict__ v_pool, const int32_t* __restrict__ kv_lens,
    const int32_t* __restrict__ block_tables, int max_blocks, int kv_heads, int block_size,
    int64_t num_slots, int pages_per_seq) {
    __shared__ __attribute__((aligned(16))) uint16_t tp[4][PF_D * 16];
    const int tiles_per_seq = pages_per_seq >> 2;
    const int seq = blockIdx.x / tiles_per_seq;
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int p = 4 * (blockIdx.x - seq * tiles_per_seq) + wv;
    const int kvh = blockIdx.y;
    const int kv_cap = max_blocks * block_size;
    const int lb = min((16 * p) / block_size, max_blocks - 1);  // the page lies in one block
    const int kvl_raw = kv_lens[seq];
    const int bid = block_tables[(int64_t)seq * max_blocks + lb];
    const int kvl = max(min(kvl_raw, kv_cap), 0);
    if (p >= 4 * ((kvl + PF_KT - 1) / PF_KT)) return;  // the whole workgroup (same tile)
    // lane (m, c) = (lane / 16, lane % 16): tokens 4m .. 4m + 3, dims 8c .. 8c + 7. Tokens
    // 4m + j sit at positions sigma16(4m) + j, so each dim's four values are one 8-byte LDS store.
    const int m = lane >> 4, c = lane & 15;
    const int tok0 = 16 * p + 4 * m;
    const int max_phys = (int)(num_slots / block_size - 1);
    const int phys = min(max(bid, 0), max_phys);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(v_pool + (int64_t)kvh * num_slots * PF_D), (short)0,
        (int)(num_slots * PF_D * (int64_t)sizeof(T)), BUF_DWORD3);
    const uint32_t row0 = (uint32_t)(phys * block_size + (tok0 - lb * block_size));
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; j++)  // tokens past kv_len read zeros (out-of-range offset)
        v[j] = __builtin_amdgcn_raw_buffer_load_b128(
            rsrc, tok0 + j < kvl ? ((row0 + j) * PF_D + 8 * c) * (uint32_t)sizeof(T) : PF_OOR, 0,
            BUF_NT);
    if constexpr (std::is_same<T, bf16_t>::value) {
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int x = 0; x < 4; x++)
                v[j][x] = pack2<f16_t>(lo_f32<bf16_t>(v[j][x]), hi_f32<bf16_t>(v[j][x]));
    }
    uint16_t* t = tp[wv];
    const int pos = sigma16(4 * m);
#pragma unroll
    for (int x = 0; x < 4; x++) {
        // dims 8c + 2x (low halves) and 8c + 2x + 1 (high halves) of tokens 4m .. 4m + 3
        *reinterpret_cast<u32x2*>(&t[(8 * c + 2 * x) * 16 + pos]) =
            u32x2{perm_lo16(v[0][x], v[1][x]), perm_lo16(v[2][x], v[3][x])};
        *reinterpret_cast<u32x2*>(&t[(8 * c + 2 * x + 1) * 16 + pos]) =
            u32x2{perm_hi16(v[0][x], v[1][x]), perm_hi16(v[2][x], v[3][x])};
    }
    __syncthreads();
    // the page in four 1 KB runs
    u32x4* dst = reinterpret_cast<u32x4*>(
        ws + ((int64_t)(seq * pages_per_seq + p) * kv_heads + kvh) * (PF_D * 16));
    const u32x4* src = reinterpret_cast<const u32x4*>(t);
#pragma unroll
    for (int x = 0; x < 4; x++) dst[lane + 64 * x] = src[lane + 64 * x];
}

static int g_prefill_persistent = 1;  // a tuning / test switch
// Direct-to-LDS staging: 0 never, 1 for long prompts (PF_DMA_MIN_MEAN_Q), 2 whenever the
// persistent fp16 P.V path runs; a tuning / test switch.
static int g_prefill_dma = 1;
// The V staging copy is paid once per kv tile; the saving comes with every query tile that reads
// it. Measured on Llama-3-8B heads (32 q / 8 kv, causal, no prefix), DMA over register staging:
// +2% at 16 x 1,024 rows, +6% at 8 x 2,048, +7% at 4 x 4,096 and 1 x 16,384; a ragged batch
// of 8 x 256-2,048 rows (mean ~1,150) breaks even.
static constexpr int PF_DMA_MIN_MEAN_Q = 1536;
// Largest staging copy the DMA path takes; beyond it the launch uses register staging.
static constexpr int64_t PF_STAGE_MAX_BYTES = int64_t(1) << 30;

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

// Bytes of the V staging copy the direct-to-LDS path reads for a call with num_seqs sequences
// and block-table rows of max_blocks pages of block_size tokens (kv_heads heads, head_dim 128):
// every 16-token page of the block table's capacity in whole 64-token tiles, per sequence and
// kv head. 0 when it exceeds PF_STAGE_MAX_BYTES (the staging copy's buffer resource holds a
// 32-bit size).
static int64_t prefill_stage_bytes(int64_t num_seqs, int64_t max_blocks, int64_t block_size,
                                   int64_t kv_heads) {
    const int64_t pages_per_seq = 4 * ((max_blocks * block_size + PF_KT - 1) / PF_KT);
    const int64_t bytes = num_seqs * pages_per_seq * kv_heads * PF_VPAGE_BYTES;
    return bytes <= PF_STAGE_MAX_BYTES ? bytes : 0;
}

template <typename T, typename TO, int PV, int D>
static int launch_prefill_mfma(void* out, int64_t o_st, int64_t o_sh, const void* q,
                               int64_t q_st, int64_t q_sh, const void* k_pool, const void* v_pool,
                               const int32_t* cu, const int32_t* kv_lens, const int32_t* bt,
                               int max_blocks, int num_seqs, int max_seqlen_q, int total_q,
                               int num_heads, int n_rep, int block_size, int64_t num_slots,
                               float scale, void* ws, size_t ws_size, const int32_t* q_rows,
                               hipStream_t stream) {
    const int64_t n_qt = (max_seqlen_q + PF_QT - 1) / PF_QT;
    const int64_t items = n_qt * num_seqs * (num_heads / n_rep) * ((n_rep + 1) / 2);
    const int64_t cus = device_cus();
    const bool persistent = g_prefill_persistent && num_seqs <= PF_MAX_SEQS &&
                            n_qt <= PF_MAX_LEVELS && (items + cus - 1) / cus <= PF_MAX_WG_ITEMS;
    const int64_t grid = persistent ? std::min<int64_t>(items, cus) : items;
    if (grid > 0x7fffffff) {
        set_error("varlen_prefill: grid too large");
        return FLOUR_ERR_UNSUPPORTED;
    }
    if (grid == 0) return FLOUR_OK;
    if constexpr (PV == PV_F16 && D == PF_D) {
        // DMA path: the V staging copy lives in the caller's workspace; two launches, the
        // staging pre-pass then the attention kernel.
        const int kv_heads = num_heads / n_rep;
        const int64_t pages_per_seq = 4 * (((int64_t)max_blocks * block_size + PF_KT - 1) / PF_KT);
        const int64_t need = prefill_stage_bytes(num_seqs, max_blocks, block_size, kv_heads);
        const bool want = g_prefill_dma == 2 ||
                          (g_prefill_dma == 1 && total_q >= (int64_t)PF_DMA_MIN_MEAN_Q * num_seqs);
        if (want && persistent && ws != nullptr && need > 0 && (int64_t)ws_size >= need) {
            prefill_v_stage_kernel<T><<<dim3((unsigned)(num_seqs * pages_per_seq / 4),
                                             (unsigned)kv_heads),
                                        dim3(256), 0, stream>>>(
                static_cast<f16_t*>(ws), static_cast<const T*>(v_pool), kv_lens, bt, max_blocks,
                kv_heads, block_size, num_slots, (int)pages_per_seq);
            const int rc = check_hip(hipGetLastError(), "varlen_prefill V staging launch");
            if (rc != FLOUR_OK) return rc;
            auto kern = block_size == 16 ? varlen_prefill_mfma_kernel<T, TO, PV, true, true, D>
                                         : varlen_prefill_mfma_kernel<T, TO, PV, false, true, D>;
            kern<<<dim3((unsigned)grid), dim3(PF_THREADS), 0, stream>>>(
                static_cast<TO*>(out), o_st, o_sh, static_cast<const T*>(q), q_st, q_sh,
                static_cast<const T*>(k_pool), static_cast<const T*>(v_pool), cu, kv_lens, bt,
                max_blocks, num_seqs, num_heads, n_rep, block_size, num_slots, (int)n_qt,
                (int)persistent, scale * PF_LOG2E, static_cast<const f16_t*>(ws),
                (uint32_t)need, q_rows);
            return check_hip(hipGetLastError(), "varlen_prefill launch");
        }
    }
    auto kern = block_size == 16 ? varlen_prefill_mfma_kernel<T, TO, PV, true, false, D>
                                 : varlen_prefill_mfma_kernel<T, TO, PV, false, false, D>;
    kern<<<dim3((unsigned)grid), dim3(PF_THREADS), 0, stream>>>(
        static_cast<TO*>(out), o_st, o_sh, static_cast<const T*>(q), q_st, q_sh,
        static_cast<const T*>(k_pool), static_cast<const T*>(v_pool), cu, kv_lens, bt, max_blocks,
        num_seqs, num_heads, n_rep, block_size, num_slots, (int)n_qt, (int)persistent,
        scale * PF_LOG2E, nullptr, 0u, q_rows);
    return check_hip(hipGetLastError(), "varlen_prefill launch");
}

// P.V mode of the MFMA path (PV_F16 or PV_HILO); a test / tuning switch.
static int g_prefill_pv_mode = PV_F16;

}  // namespace flour

using namespace flour;

extern "C" int flour_hip_set_prefill_persistent(int on) {
    g_prefill_persistent = on ? 1 : 0;
    return FLOUR_OK;
}

// 0: register staging only; 1: direct-to-LDS staging for long prompts (the default);
// 2: direct-to-LDS staging whenever the persistent fp16 P.V path runs.
extern "C" int flour_hip_set_prefill_dma(int mode) {
    if (mode < 0 || mode > 2) {
        set_error("set_prefill_dma: mode %d is not 0, 1 or 2", mode);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    g_prefill_dma = mode;
    return FLOUR_OK;
}

extern "C" int flour_hip_set_prefill_precise_p(int on) {
    g_prefill_pv_mode = on ? PV_HILO : PV_F16;
    return FLOUR_OK;
}

namespace flour {

bool prefill_mfma_supported(int dtype, int head_dim, int block_size, int64_t num_slots,
                            float scale, int64_t q_stride_tok) {
    // (the Q rows of a wave are loaded with 32-bit offsets from its first row: 31 row strides)
    return (dtype == FLOUR_DTYPE_BF16 || dtype == FLOUR_DTYPE_F16) &&
           (head_dim == PF_D || head_dim == PF_D64) && block_size % 16 == 0 && num_slots % block_size == 0 && scale > 0.0f &&
           num_slots * head_dim * 2 <= (int64_t)0x7fffffff && q_stride_tok >= 0 &&
           q_stride_tok * 2 * 32 <= (int64_t)0x7fffffff;
}

}  // namespace flour

static int varlen_prefill_impl(void* out, int out_dtype, int64_t o_stride_tok,
                               int64_t o_stride_head, const void* q, int64_t q_stride_tok,
                               int64_t q_stride_head, const void* k_pool, const void* v_pool,
                               const int32_t* cu_seqlens_q, const int32_t* kv_lens,
                               const int32_t* block_tables, int max_blocks_per_seq, int num_seqs,
                               int max_seqlen_q, int total_q, int num_heads, int kv_heads,
                               int head_dim, int block_size, int64_t num_slots, float scale,
                               int dtype, void* workspace, size_t workspace_bytes,
                               const int32_t* q_rows, void* stream) {
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
    // (the Q rows of a wave are loaded with 32-bit offsets from its first row: 31 row strides)
    const bool mfma = aligned && prefill_mfma_supported(dtype, head_dim, block_size, num_slots,
                                                        scale, q_stride_tok);
    // fp32 pools at head_dim 64 / 128: the fp32 matrix cores
    if (!mfma && !q_rows && aligned &&
        prefill_f32_mfma_supported(dtype, head_dim, num_seqs, max_seqlen_q, block_size, num_slots))
        return launch_prefill_f32_mfma(out_dtype, out, o_stride_tok, o_stride_head, q, q_stride_tok,
                                       q_stride_head, k_pool, v_pool, cu_seqlens_q, nullptr,
                                       kv_lens, block_tables, max_blocks_per_seq, num_seqs,
                                       max_seqlen_q, num_heads, n_rep, head_dim, block_size,
                                       num_slots, scale, s);
    if (!mfma && q_rows) {
        set_error("varlen_prefill: row indices need the matrix-core path");
        return FLOUR_ERR_UNSUPPORTED;
    }
    if (!mfma) {
        if (simt_supported(dtype, head_dim, q, q_stride_tok, q_stride_head, k_pool, v_pool))
            return launch_attn_simt(dtype, out_dtype, out, o_stride_tok, o_stride_head, q,
                                    q_stride_tok, q_stride_head, k_pool, v_pool, cu_seqlens_q,
                                    kv_lens, block_tables, max_blocks_per_seq, num_seqs, total_q,
                                    num_heads, n_rep, head_dim, block_size, num_slots, INT_MAX,
                                    scale, s);
        return launch_attn_generic(dtype, out_dtype, out, o_stride_tok, o_stride_head, q,
                                   q_stride_tok, q_stride_head, k_pool, v_pool, cu_seqlens_q,
                                   kv_lens, block_tables, max_blocks_per_seq, num_seqs, total_q,
                                   num_heads, n_rep, head_dim, block_size, num_slots, INT_MAX,
                                   scale, s);
    }
#define FLOUR_PF_D(T, TO, D)                                                                     \
    return g_prefill_pv_mode == PV_HILO                                                          \
               ? launch_prefill_mfma<T, TO, PV_HILO, D>(                                         \
                     out, o_stride_tok, o_stride_head, q, q_stride_tok, q_stride_head, k_pool,   \
                     v_pool, cu_seqlens_q, kv_lens, block_tables, max_blocks_per_seq, num_seqs,  \
                     max_seqlen_q, total_q, num_heads, n_rep, block_size, num_slots, scale,      \
                     workspace, workspace_bytes, q_rows, s)                                      \
               : launch_prefill_mfma<T, TO, PV_F16, D>(                                          \
                     out, o_stride_tok, o_stride_head, q, q_stride_tok, q_stride_head, k_pool,   \
                     v_pool, cu_seqlens_q, kv_lens, block_tables, max_blocks_per_seq, num_seqs,  \
                     max_seqlen_q, total_q, num_heads, n_rep, block_size, num_slots, scale,      \
                     workspace, workspace_bytes, q_rows, s)
#define FLOUR_PF(T, TO)                                                                          \
    do {                                                                                         \
        if (head_dim == PF_D64) FLOUR_PF_D(T, TO, PF_D64);                                       \
        FLOUR_PF_D(T, TO, PF_D);                                                                 \
    } while (0)
    if (dtype == FLOUR_DTYPE_BF16) {
        if (out_dtype == FLOUR_DTYPE_F32) FLOUR_PF(bf16_t, float);
        if (out_dtype == FLOUR_DTYPE_BF16) FLOUR_PF(bf16_t, bf16_t);
        FLOUR_PF(bf16_t, f16_t);
    }
    if (out_dtype == FLOUR_DTYPE_F32) FLOUR_PF(f16_t, float);
    if (out_dtype == FLOUR_DTYPE_BF16) FLOUR_PF(f16_t, bf16_t);
    FLOUR_PF(f16_t, f16_t);
#undef FLOUR_PF
#undef FLOUR_PF_D
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
    return varlen_prefill_impl(out, out_dtype, o_stride_tok, o_stride_head, q, q_stride_tok,
                               q_stride_head, k_pool, v_pool, cu_seqlens_q, kv_lens, block_tables,
                               max_blocks_per_seq, num_seqs, max_seqlen_q, total_q, num_heads,
                               kv_heads, head_dim, block_size, num_slots, scale, dtype, nullptr, 0,
                               nullptr, stream);
}

extern "C" int flour_hip_varlen_prefill_workspace_size(int num_seqs, int max_blocks_per_seq,
                                                       int block_size, int kv_heads, int head_dim,
                                                       int dtype, size_t* bytes) {
    clear_error();
    if (!bytes) {
        set_error("varlen_prefill_workspace_size: null output");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    *bytes = 0;
    if (num_seqs < 0 || max_blocks_per_seq <= 0 || block_size <= 0 || kv_heads <= 0 ||
        head_dim <= 0 || !valid_dtype(dtype)) {
        set_error("varlen_prefill_workspace_size: bad shape (seqs=%d max_blocks=%d bs=%d "
                  "kv_heads=%d head_dim=%d dtype=%d)",
                  num_seqs, max_blocks_per_seq, block_size, kv_heads, head_dim, dtype);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    // only 16-bit pools at head_dim 128 with 16-token-aligned pages take the staged path
    if ((dtype == FLOUR_DTYPE_BF16 || dtype == FLOUR_DTYPE_F16) && head_dim == PF_D &&
        block_size % 16 == 0)
        *bytes = (size_t)prefill_stage_bytes(num_seqs, max_blocks_per_seq, block_size, kv_heads);
    return FLOUR_OK;
}

extern "C" int flour_hip_varlen_prefill_ws(void* out, int out_dtype, int64_t o_stride_tok,
                                           int64_t o_stride_head, const void* q,
                                           int64_t q_stride_tok, int64_t q_stride_head,
                                           const void* k_pool, const void* v_pool,
                                           const int32_t* cu_seqlens_q, const int32_t* kv_lens,
                                           const int32_t* block_tables, int max_blocks_per_seq,
                                           int num_seqs, int max_seqlen_q, int total_q,
                                           int num_heads, int kv_heads, int head_dim,
                                           int block_size, int64_t num_slots, float scale,
                                           int dtype, void* workspace, size_t workspace_bytes,
                                           void* stream) {
    if (workspace != nullptr && (uintptr_t)workspace % 256 != 0) {
        clear_error();
        set_error("varlen_prefill_ws: workspace must be 256-byte aligned");
        return FLOUR_ERR_WORKSPACE;
    }
    return varlen_prefill_impl(out, out_dtype, o_stride_tok, o_stride_head, q, q_stride_tok,
                               q_stride_head, k_pool, v_pool, cu_seqlens_q, kv_lens, block_tables,
                               max_blocks_per_seq, num_seqs, max_seqlen_q, total_q, num_heads,
                               kv_heads, head_dim, block_size, num_slots, scale, dtype, workspace,
                               workspace_bytes, nullptr, stream);
}

namespace flour {

// Varlen prefill whose sequence s takes its q / out rows from row q_rows[s] on (its row count
// still cu_seqlens_q[s + 1] - cu_seqlens_q[s]): the multi-row sequences of a mixed
// continuous-batching step, whose packed rows sit among one-row sequences' rows. Matrix-core
// shapes only (FLOUR_ERR_UNSUPPORTED otherwise, before any launch).
int varlen_prefill_rows(void* out, int out_dtype, int64_t o_stride_tok, int64_t o_stride_head,
                        const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                        const void* k_pool, const void* v_pool, const int32_t* cu_seqlens_q,
                        const int32_t* q_rows, const int32_t* kv_lens,
                        const int32_t* block_tables, int max_blocks_per_seq, int num_seqs,
                        int max_seqlen_q, int total_q, int num_heads, int kv_heads, int head_dim,
                        int block_size, int64_t num_slots, float scale, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream) {
    if (!q_rows) {
        set_error("varlen_prefill_rows: null row indices");
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    return varlen_prefill_impl(out, out_dtype, o_stride_tok, o_stride_head, q, q_stride_tok,
                               q_stride_head, k_pool, v_pool, cu_seqlens_q, kv_lens, block_tables,
                               max_blocks_per_seq, num_seqs, max_seqlen_q, total_q, num_heads,
                               kv_heads, head_dim, block_size, num_slots, scale, dtype, workspace,
                               workspace_bytes, q_rows, stream);
}

}  // namespace flour
