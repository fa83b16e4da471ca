/*
 * flour_oracle.c — CPU restatement of flour's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP kernels are compared
 * against and the CPU baseline that bench.py times beside them. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; nothing in the product
 * path (flour_amd/, libflour_hip.so) links or calls it.
 *
 * Reference files (lltsdyp/flour, Rust/candle 0.9.2; not buildable here — no cargo, candle
 * not vendored) restated below, each function citing the lines it follows:
 *   src/models/common/paged.rs:114-121   BlockTable::slot / slots
 *   src/models/common/paged.rs:186-204   PagedKvPool::write (both its documented scatter
 *                                        semantics and its literal run loop, :196 quirk)
 *   src/models/common/paged.rs:266-279   PagedKvPool::block_view (block walk of the pool)
 *   src/models/common/cache.rs:83-96     KvCache::gather_blocks (logical block list)
 *   src/backend/cpu.rs:57-112            paged_attention (online softmax over blocks)
 *   src/backend/cpu.rs:24-42, :148-165   causal_attention / dense_reference (fp64 here)
 *   src/models/common/attention.rs:96-104  rope(q), rope(k) (candle_nn::rotary_emb::rope with
 *                                        the cache.rs:377-393 tables), then write_kv
 *
 * Arithmetic: fp32 as in the reference's accumulation (cpu.rs:71-73, :84-85, :104); bf16/f16
 * inputs are widened exactly to fp32 (the "fp32 CPU reference"), the dense check runs in
 * fp64. Parity pins: see tests/test_oracle.py (reference KATs, closed forms, fp64 brute force,
 * torch SDPA, permutation/block-size invariance, and planted-mistake checks via
 * oracle_set_mutation()).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* dtype codes, same values as enum flour_dtype in include/flour_hip.h */
#define DT_F32 0
#define DT_BF16 1
#define DT_F16 2

/* ---------------------------------------------------------------- element conversions */

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) /* NaN: keep quiet NaN */
        return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

static inline float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while (!(man & 0x400u));
            man &= 0x3ffu;
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t f32_to_f16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0));
    if (a >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) { /* result is subnormal or zero in f16 */
        if (a < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to 0 */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e; /* 14..24 */
        uint32_t res = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (res & 1u))) res++;
        return (uint16_t)(sign | res);
    }
    uint32_t res = ((a >> 13) - ((127 - 15) << 10));
    uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (res & 1u))) res++;
    return (uint16_t)(sign | res);
}

static inline float load_elem(const void* p, int64_t i, int dt) {
    if (dt == DT_F32) return ((const float*)p)[i];
    if (dt == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
    return f16_to_f32(((const uint16_t*)p)[i]);
}

static inline void store_elem(void* p, int64_t i, int dt, float x) {
    if (dt == DT_F32)
        ((float*)p)[i] = x;
    else if (dt == DT_BF16)
        ((uint16_t*)p)[i] = f32_to_bf16_rne(x);
    else
        ((uint16_t*)p)[i] = f32_to_f16_rne(x);
}

static inline int elem_size(int dt) { return dt == DT_F32 ? 4 : 2; }

/* Exported conversions so tests can pin them against numpy/torch. */
void oracle_f32_to_bf16(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = f32_to_bf16_rne(x[i]);
}
void oracle_bf16_to_f32(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = bf16_to_f32(x[i]);
}
void oracle_f32_to_f16(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = f32_to_f16_rne(x[i]);
}
void oracle_f16_to_f32(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = f16_to_f32(x[i]);
}

/* ---------------------------------------------------------------- planted mistakes
 * Test-only switch: a nonzero code makes the attention restatement commit one plausible
 * mistake, so tests can show that the pinning checks catch it. 0 = faithful. */
enum {
    MUT_NONE = 0,
    MUT_MASK_OFF_BY_ONE = 1,  /* mask j >= offset+i instead of j > offset+i       */
    MUT_NO_CORRECTION = 2,    /* forget to rescale acc/sum by exp(m_old - m_new)  */
    MUT_WRONG_KV_HEAD = 3,    /* GQA map h % kv_heads instead of h / n_rep         */
    MUT_NO_SCALE = 4,         /* drop the softmax scale                           */
    MUT_OFFSET_ZERO = 5,      /* causal offset 0 instead of kv_len - q_len        */
    MUT_SLOT_SWAP = 6,        /* slot = pos%bs * nblk + blk (transposed index)    */
    MUT_ROPE_INTERLEAVED = 7, /* rotate pairs (2i, 2i+1) instead of (i, i + d/2)  */
    MUT_ROPE_SIGN = 8,        /* rotate by -angle (sin sign flipped)              */
};
static int g_mutation = MUT_NONE;
void oracle_set_mutation(int code) { g_mutation = code; }
int oracle_get_mutation(void) { return g_mutation; }

/* ---------------------------------------------------------------- paged.rs:114-121 */

/* BlockTable::slot: blocks[pos / block_size] * block_size + pos % block_size. */
int64_t oracle_slot(const int32_t* blocks, int block_size, int64_t pos) {
    int64_t lb = pos / block_size, off = pos % block_size;
    if (g_mutation == MUT_SLOT_SWAP) return off * block_size + blocks[lb];
    return (int64_t)blocks[lb] * block_size + off;
}

/* BlockTable::slots(start, end) as u32. */
void oracle_slots(const int32_t* blocks, int block_size, int64_t start, int64_t end,
                  uint32_t* out) {
    for (int64_t p = start; p < end; p++) out[p - start] = (uint32_t)oracle_slot(blocks, block_size, p);
}

/* ---------------------------------------------------------------- paged.rs:186-204 */

/* Documented semantics of PagedKvPool::write (paged.rs:186-187, test :287-306): a pure
 * scatter pool[h, slots[t], :] = k[t, h, :]. Element (t,h,d) of k/v is at
 * t*stride_tok + h*stride_head + d. Negative slots are skipped (padding), slots beyond
 * num_slots are skipped and counted. Returns the number of skipped out-of-range rows. */
int64_t oracle_kv_write_scatter(const void* k, const void* v, int64_t stride_tok,
                                int64_t stride_head, void* k_pool, void* v_pool,
                                const int32_t* slots, int num_tokens, int kv_heads,
                                int head_dim, int64_t num_slots, int dtype) {
    int es = elem_size(dtype);
    int64_t bad = 0;
    for (int t = 0; t < num_tokens; t++) {
        int64_t s = slots[t];
        if (s < 0) continue;
        if (s >= num_slots) {
            bad++;
            continue;
        }
        for (int h = 0; h < kv_heads; h++) {
            int64_t src = (int64_t)t * stride_tok + (int64_t)h * stride_head;
            int64_t dst = ((int64_t)h * num_slots + s) * head_dim;
            memcpy((char*)k_pool + dst * es, (const char*)k + src * es, (size_t)head_dim * es);
            memcpy((char*)v_pool + dst * es, (const char*)v + src * es, (size_t)head_dim * es);
        }
    }
    return bad;
}

/* ---------------------------------------------------------------- attention.rs:96-104 */

/* Round to the element type and back (fp32: unchanged). */
static inline float round_dt(float x, int dt) {
    if (dt == DT_F32) return x;
    if (dt == DT_BF16) return bf16_to_f32(f32_to_bf16_rne(x));
    return f16_to_f32(f32_to_f16_rne(x));
}

/* One row of candle_nn::rotary_emb::rope (candle-nn 0.9.2; not vendored here), the
 * non-interleaved ("rotate half") form that attention.rs:98-99 calls: for i < d/2 with
 * c = cos[p][i], s = sin[p][i],
 *   dst[i]       = x[i] * c - x[i + d/2] * s
 *   dst[i + d/2] = x[i] * s + x[i + d/2] * c
 * evaluated in the element type: half::bf16 / half::f16 operations compute in f32 and round the
 * result to the type (nearest even), f32 rounds each operation (no fused multiply-add: this
 * function is compiled without contraction). The reference's own tests hold no RoPE vectors;
 * the closed forms in tests/test_oracle.py pin the rotation (identity at position 0, exact
 * quarter turns, fp64 rotation within the per-step roundings), not the last bit of the
 * rounding sequence. src may equal dst. */
__attribute__((optimize("fp-contract=off"))) static void rope_row(
    void* dst, int64_t dst_off, const void* src, int64_t src_off, const void* cos_t,
    const void* sin_t, int64_t tab_off, int d, int dt) {
    const int half = d / 2;
    for (int i = 0; i < half; i++) {
        int i1 = i, i2 = i + half;
        if (g_mutation == MUT_ROPE_INTERLEAVED) {
            i1 = 2 * i;
            i2 = 2 * i + 1;
        }
        const float x1 = load_elem(src, src_off + i1, dt), x2 = load_elem(src, src_off + i2, dt);
        const float c = load_elem(cos_t, tab_off + i, dt);
        float sn = load_elem(sin_t, tab_off + i, dt);
        if (g_mutation == MUT_ROPE_SIGN) sn = -sn;
        const float a = round_dt(x1 * c, dt), b = round_dt(x2 * sn, dt);
        const float e = round_dt(x1 * sn, dt), f = round_dt(x2 * c, dt);
        store_elem(dst, dst_off + i1, dt, round_dt(a - b, dt));
        store_elem(dst, dst_off + i2, dt, round_dt(e + f, dt));
    }
}

/* RoPE on the new q / k rows, then Cache::write_kv's scatter (paged.rs:186-187): the order of
 * attention.rs:96-104 for token t at table row positions[t]. q / q_out share strides (in place
 * allowed); k / v share kv strides; tables are (max_pos, d/2). A token whose slot is outside
 * [0, num_slots) writes no K/V; one whose position is outside [0, max_pos) writes nothing.
 * Returns the number of tokens skipped for their position. */
int64_t oracle_rope_kv_write(void* q_out, const void* q, int64_t q_stride_tok,
                             int64_t q_stride_head, int num_heads, const void* k, const void* v,
                             int64_t kv_stride_tok, int64_t kv_stride_head, void* k_pool,
                             void* v_pool, const int32_t* slots, const int32_t* positions,
                             const void* cos_t, const void* sin_t, int max_pos, int num_tokens,
                             int kv_heads, int head_dim, int64_t num_slots, int dtype) {
    const int es = elem_size(dtype);
    int64_t skipped = 0;
    for (int t = 0; t < num_tokens; t++) {
        const int p = positions[t];
        if (p < 0 || p >= max_pos) {
            skipped++;
            continue;
        }
        const int64_t tab = (int64_t)p * (head_dim / 2);
        for (int h = 0; h < num_heads; h++) {
            const int64_t off = (int64_t)t * q_stride_tok + (int64_t)h * q_stride_head;
            rope_row(q_out, off, q, off, cos_t, sin_t, tab, head_dim, dtype);
        }
        const int64_t sl = slots[t];
        if (sl < 0 || sl >= num_slots) continue;
        for (int h = 0; h < kv_heads; h++) {
            const int64_t src = (int64_t)t * kv_stride_tok + (int64_t)h * kv_stride_head;
            const int64_t dst = ((int64_t)h * num_slots + sl) * head_dim;
            rope_row(k_pool, dst, k, src, cos_t, sin_t, tab, head_dim, dtype);
            memcpy((char*)v_pool + dst * es, (const char*)v + src * es, (size_t)head_dim * es);
        }
    }
    return skipped;
}

/* Literal restatement of the run loop at paged.rs:192-202, including the run condition at
 * :196 `i + n < slots.len() && i + n == start_slot + n`, which holds exactly when
 * i == start_slot: a run that starts at a token index equal to its slot then extends to the
 * end of the batch and is written contiguously from start_slot. k/v are in the reference
 * layout (kv_heads, seq, head_dim) (the squeezed (1, kv_heads, seq, head_dim), :188-189).
 * Returns 0, or -1 where candle's slice_set would reject a run that ends past num_slots
 * (nothing of that run is written, as candle checks before copying). */
int oracle_kv_write_reference_loop(const void* k, const void* v, void* k_pool, void* v_pool,
                                   const uint32_t* slots, int seq, int kv_heads, int head_dim,
                                   int64_t num_slots, int dtype) {
    int es = elem_size(dtype);
    int i = 0;
    while (i < seq) {
        int n = 1;
        int64_t start_slot = slots[i];
        while (i + n < seq && (int64_t)(i + n) == start_slot + n) n++;
        if (start_slot + n > num_slots) return -1;
        for (int h = 0; h < kv_heads; h++) {
            for (int r = 0; r < n; r++) {
                int64_t src = ((int64_t)h * seq + (i + r)) * head_dim;
                int64_t dst = ((int64_t)h * num_slots + start_slot + r) * head_dim;
                memcpy((char*)k_pool + dst * es, (const char*)k + src * es, (size_t)head_dim * es);
                memcpy((char*)v_pool + dst * es, (const char*)v + src * es, (size_t)head_dim * es);
            }
        }
        i += n;
    }
    return 0;
}

/* Whether a slot mapping hits the :196 quirk: some run start i has slots[i] == i and at
 * least one token follows it. Returns the first such i, or -1. */
int oracle_kv_write_quirk_index(const uint32_t* slots, int seq) {
    int i = 0;
    while (i < seq) {
        int n = 1;
        int64_t start_slot = slots[i];
        while (i + n < seq && (int64_t)(i + n) == start_slot + n) n++;
        if (n > 1) return i;
        i += n;
    }
    return -1;
}

/* ---------------------------------------------------------------- cpu.rs:57-112 */

/* One (sequence, query head, query row) of paged_attention, following cpu.rs:57-112:
 * stream the logical blocks (cache.rs:83-96: block b covers kv positions
 * [b*bs, min((b+1)*bs, kv_len)) and lives at pool slots block_table[b]*bs + ...), with
 * scores = q.k * scale in fp32 (:84-85), the mask kv_start+j > offset+i -> -inf (:88-95),
 * block max / new max / correction / probs (:96-100), running sum and acc (:102-104), and
 * out = acc / sum (:111). */
static void paged_row(float* out_row /* [D] */, const float* qrow /* [D] */,
                      const void* k_pool, const void* v_pool, int kv_dtype, int64_t num_slots,
                      int kvh, const int32_t* btab, int block_size, int kv_len, int q_len,
                      int i, int D, float scale, float* scores /* [block_size] */,
                      float* acc /* [D] */, float* pv /* [D] */) {
    int64_t offset = (g_mutation == MUT_OFFSET_ZERO) ? 0 : (int64_t)kv_len - q_len;
    float run_max = -INFINITY, run_sum = 0.0f;
    for (int d = 0; d < D; d++) acc[d] = 0.0f;
    float sc = (g_mutation == MUT_NO_SCALE) ? 1.0f : scale;
    int nblocks = (kv_len + block_size - 1) / block_size;
    for (int b = 0; b < nblocks; b++) {
        int64_t kv_start = (int64_t)b * block_size;
        int block_n = kv_len - (int)kv_start < block_size ? kv_len - (int)kv_start : block_size;
        int64_t slot0 = (int64_t)btab[b] * block_size;
        const int64_t base = ((int64_t)kvh * num_slots + slot0) * D;
        float bmax = -INFINITY;
        for (int j = 0; j < block_n; j++) {
            float dot = 0.0f;
            int64_t kb = base + (int64_t)j * D;
            if (kv_dtype == DT_F32) {
                const float* kr = (const float*)k_pool + kb;
#pragma omp simd reduction(+ : dot)
                for (int d = 0; d < D; d++) dot += qrow[d] * kr[d];
            } else if (kv_dtype == DT_BF16) {
                const uint16_t* kr = (const uint16_t*)k_pool + kb;
#pragma omp simd reduction(+ : dot)
                for (int d = 0; d < D; d++) dot += qrow[d] * bf16_to_f32(kr[d]);
            } else {
                const uint16_t* kr = (const uint16_t*)k_pool + kb;
                for (int d = 0; d < D; d++) dot += qrow[d] * f16_to_f32(kr[d]);
            }
            float s = dot * sc;
            int masked = (g_mutation == MUT_MASK_OFF_BY_ONE) ? (kv_start + j >= offset + i)
                                                             : (kv_start + j > offset + i);
            if (masked) s = -INFINITY;
            scores[j] = s;
            if (s > bmax) bmax = s;
        }
        float new_max = run_max > bmax ? run_max : bmax;
        float corr;
        if (g_mutation == MUT_NO_CORRECTION)
            corr = 1.0f;
        else
            corr = (new_max == -INFINITY) ? 1.0f : expf(run_max - new_max);
        float psum = 0.0f;
        for (int j = 0; j < block_n; j++) {
            float p = (scores[j] == -INFINITY) ? 0.0f : expf(scores[j] - new_max);
            scores[j] = p;
            psum += p;
        }
        run_sum = run_sum * corr + psum;
        /* probs @ v (cpu.rs:103-104): pv[d] = sum_j p_j v[j][d], j ascending for every d. */
        for (int d = 0; d < D; d++) pv[d] = 0.0f;
        for (int j = 0; j < block_n; j++) {
            float p = scores[j];
            int64_t vb = base + (int64_t)j * D;
            if (kv_dtype == DT_F32) {
                const float* vr = (const float*)v_pool + vb;
                for (int d = 0; d < D; d++) pv[d] += p * vr[d];
            } else if (kv_dtype == DT_BF16) {
                const uint16_t* vr = (const uint16_t*)v_pool + vb;
                for (int d = 0; d < D; d++) pv[d] += p * bf16_to_f32(vr[d]);
            } else {
                for (int d = 0; d < D; d++) pv[d] += p * load_elem(v_pool, vb + d, kv_dtype);
            }
        }
        for (int d = 0; d < D; d++) acc[d] = acc[d] * corr + pv[d];
        run_max = new_max;
    }
    for (int d = 0; d < D; d++) out_row[d] = (run_sum > 0.0f) ? acc[d] / run_sum : 0.0f;
}

/* Batched paged_attention: sequence s owns query rows cu_seqlens_q[s]..cu_seqlens_q[s+1]-1,
 * attends kv_lens[s] positions through block_tables[s*max_blocks ..]. q / out element
 * (row, head, d) at row*stride_tok + head*stride_head + d. Query head h reads kv head
 * h / n_rep (repeat_kv, cpu.rs:5-13). Parallel over (sequence, kv head, row chunk) with
 * OpenMP on num_threads threads (<= 0: all). Returns 0, or -1 on a bad argument. */
int oracle_paged_attention(void* out, int out_dtype, int64_t o_stride_tok, int64_t o_stride_head,
                           const void* q, int q_dtype, int64_t q_stride_tok,
                           int64_t q_stride_head, const void* k_pool, const void* v_pool,
                           int kv_dtype, int64_t num_slots, const int32_t* block_tables,
                           int max_blocks, const int32_t* cu_seqlens_q, const int32_t* kv_lens,
                           int num_seqs, int num_heads, int kv_heads, int head_dim,
                           int block_size, float scale, int num_threads) {
    if (num_heads <= 0 || kv_heads <= 0 || num_heads % kv_heads != 0 || head_dim <= 0 ||
        block_size <= 0)
        return -1;
    const int n_rep = num_heads / kv_heads;
    const int ROWS = 16; /* rows per task */
    /* task list: (seq, kv head, row chunk) */
    int64_t ntasks = 0;
    for (int s = 0; s < num_seqs; s++) {
        int ql = cu_seqlens_q[s + 1] - cu_seqlens_q[s];
        if (ql < 0 || kv_lens[s] < 0) return -1;
        if ((kv_lens[s] + block_size - 1) / block_size > max_blocks) return -1;
        ntasks += (int64_t)kv_heads * ((ql + ROWS - 1) / ROWS);
    }
    int64_t* task_seq = (int64_t*)malloc(sizeof(int64_t) * (ntasks > 0 ? ntasks : 1));
    int64_t t = 0;
    for (int s = 0; s < num_seqs; s++) {
        int ql = cu_seqlens_q[s + 1] - cu_seqlens_q[s];
        int nc = (ql + ROWS - 1) / ROWS;
        for (int g = 0; g < kv_heads; g++)
            for (int c = 0; c < nc; c++) task_seq[t++] = ((int64_t)s << 32) | ((int64_t)g << 16) | c;
    }
#ifdef _OPENMP
    int nt = num_threads > 0 ? num_threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float* qrow = (float*)malloc(sizeof(float) * head_dim);
        float* orow = (float*)malloc(sizeof(float) * head_dim);
        float* acc = (float*)malloc(sizeof(float) * head_dim);
        float* scores = (float*)malloc(sizeof(float) * block_size);
        float* pv = (float*)malloc(sizeof(float) * head_dim);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t ti = 0; ti < ntasks; ti++) {
            int s = (int)(task_seq[ti] >> 32);
            int g = (int)((task_seq[ti] >> 16) & 0xffff);
            int c = (int)(task_seq[ti] & 0xffff);
            int q0 = cu_seqlens_q[s], ql = cu_seqlens_q[s + 1] - q0;
            int kv_len = kv_lens[s];
            const int32_t* btab = block_tables + (int64_t)s * max_blocks;
            int r_end = (c + 1) * ROWS < ql ? (c + 1) * ROWS : ql;
            for (int r = 0; r < n_rep; r++) {
                int h = g * n_rep + r;
                int kvh = (g_mutation == MUT_WRONG_KV_HEAD) ? h % kv_heads : h / n_rep;
                for (int i = c * ROWS; i < r_end; i++) {
                    int64_t row = q0 + i;
                    for (int d = 0; d < head_dim; d++)
                        qrow[d] = load_elem(q, row * q_stride_tok + h * q_stride_head + d, q_dtype);
                    if (kv_len < ql) { /* reference precondition kv_len >= seq_q (cpu.rs:68) */
                        for (int d = 0; d < head_dim; d++) orow[d] = 0.0f;
                    } else {
                        paged_row(orow, qrow, k_pool, v_pool, kv_dtype, num_slots, kvh, btab,
                                  block_size, kv_len, ql, i, head_dim, scale, scores, acc, pv);
                    }
                    for (int d = 0; d < head_dim; d++)
                        store_elem(out, row * o_stride_tok + h * o_stride_head + d, out_dtype, orow[d]);
                }
            }
        }
        free(qrow);
        free(orow);
        free(acc);
        free(scores);
        free(pv);
    }
    free(task_seq);
    return 0;
}

/* ---------------------------------------------------------------- cpu.rs:24-42 in fp64 */

/* Dense causal SDPA brute force in double over the same paged inputs: for each row, the full
 * score vector over kv positions 0..kv_len-1 (mask j > kv_len - q_len + i, as cpu.rs:148-165
 * builds it), softmax in double, out = sum p_j v_j. out is float64, packed
 * (total_q, num_heads, head_dim). Single-threaded; meant for small shapes. */
int oracle_dense_attention_f64(double* out, const void* q, int q_dtype, int64_t q_stride_tok,
                               int64_t q_stride_head, const void* k_pool, const void* v_pool,
                               int kv_dtype, int64_t num_slots, const int32_t* block_tables,
                               int max_blocks, const int32_t* cu_seqlens_q,
                               const int32_t* kv_lens, int num_seqs, int num_heads,
                               int kv_heads, int head_dim, int block_size, double scale) {
    if (num_heads <= 0 || kv_heads <= 0 || num_heads % kv_heads != 0) return -1;
    int n_rep = num_heads / kv_heads;
    for (int s = 0; s < num_seqs; s++) {
        int q0 = cu_seqlens_q[s], ql = cu_seqlens_q[s + 1] - q0, kv_len = kv_lens[s];
        const int32_t* btab = block_tables + (int64_t)s * max_blocks;
        double* p = (double*)malloc(sizeof(double) * (kv_len > 0 ? kv_len : 1));
        for (int h = 0; h < num_heads; h++) {
            int kvh = h / n_rep;
            for (int i = 0; i < ql; i++) {
                int64_t row = q0 + i;
                double* o = out + (row * num_heads + h) * head_dim;
                for (int d = 0; d < head_dim; d++) o[d] = 0.0;
                int64_t lim = (int64_t)kv_len - ql + i; /* visible j <= lim */
                if (kv_len < ql || lim < 0) continue;
                double mx = -INFINITY;
                for (int64_t j = 0; j <= lim; j++) {
                    int64_t slot = (int64_t)btab[j / block_size] * block_size + j % block_size;
                    int64_t kb = ((int64_t)kvh * num_slots + slot) * head_dim;
                    double dot = 0.0;
                    for (int d = 0; d < head_dim; d++)
                        dot += (double)load_elem(q, row * q_stride_tok + h * q_stride_head + d, q_dtype) *
                               (double)load_elem(k_pool, kb + d, kv_dtype);
                    p[j] = dot * scale;
                    if (p[j] > mx) mx = p[j];
                }
                double sum = 0.0;
                for (int64_t j = 0; j <= lim; j++) {
                    p[j] = exp(p[j] - mx);
                    sum += p[j];
                }
                for (int64_t j = 0; j <= lim; j++) {
                    int64_t slot = (int64_t)btab[j / block_size] * block_size + j % block_size;
                    int64_t vb = ((int64_t)kvh * num_slots + slot) * head_dim;
                    double w = p[j] / sum;
                    for (int d = 0; d < head_dim; d++) o[d] += w * (double)load_elem(v_pool, vb + d, kv_dtype);
                }
            }
        }
        free(p);
    }
    return 0;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
