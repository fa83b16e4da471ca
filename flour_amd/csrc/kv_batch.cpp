// kv_batch.cpp — many sequences over one device pool (continuous batching), behind the
// flour_kv_batch_* functions of include/flour_cache.h.
//
// The reference engine serves one sequence at a time: Engine holds one Mutex<Cache>
// (src/engine.rs:88) and its generation loop (engine.rs:219-263) runs CausalLM::forward for that
// sequence alone. Here one pool, its BlockAllocator and its prefix registry are shared by up to
// max_seqs sequences, each with its own BlockTable and the per-sequence operations of KvCache
// (src/models/common/cache.rs:13-165, :429-505: allocate_kv, reset_sequence, match_prefix,
// register_prefix). Because the registry is shared, one sequence reuses the full prefix blocks
// another registered (the shared cached prefix of the prefix-cached prefill workload).
//
// A forward step is planned once, not per layer: plan() takes the step's sequences and the
// number of new rows each brings, and uploads their block tables, kv lengths, cu_seqlens and the
// slot mapping of the new rows through pinned staging. Every layer then calls write_kv (the KV
// write kernel over the packed new rows) and attention on those device arrays, as
// attention.rs:104-109 does for one sequence: paged decode when every sequence brings one row,
// varlen prefill when none does, and for a mixed step (sequences decoding while others bring a
// prompt) one decode launch over the one-row sequences plus one prefill launch over the rest,
// each reading and writing its rows of the packed layout through row indices.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <memory>
#include <vector>

#include "flour_cache.h"
#include "flour_common.h"
#include "flour_hip.h"
#include "kv_host.h"

namespace flour {
namespace host {

// 1: a mixed step's one-row sequences run on the decode kernel (default); 0: every row of a
// mixed step on the prefill kernel. A tuning / test switch.
static int g_batch_split = 1;
// Decode steps through flour_kv_batch_write_kv_attention take the fused launch (1) or the KV
// write and the attention as two launches (0); a tuning / test switch.
static int g_batch_fuse = 1;

struct KvBatchImpl {
    int num_layers, max_seqs, max_seq_len, max_tokens, num_heads, kv_heads, head_dim,
        block_size, dtype;
    int num_blocks, max_blocks;  // pool blocks; table row length (blocks of one sequence)
    int64_t num_slots;
    BlockAllocator allocator;
    PrefixRegistry registry;
    std::vector<BlockTable> tables;
    std::vector<uint8_t> live;

    bool device = false;
    std::vector<void*> k_pools, v_pools;
    // plan arrays: [max_seqs x max_blocks] block tables | [max_seqs] kv lengths |
    // [max_seqs + 1] cu_seqlens | [max_tokens] slot mapping of the new rows |
    // [max_tokens] positions of the new rows in their sequences (RoPE table rows)
    int32_t* d_plan = nullptr;
    int32_t* h_plan = nullptr;
    hipEvent_t plan_done = nullptr;
    bool plan_pending = false;
    void* d_ws = nullptr;  // decode split-context partials
    size_t ws_bytes = 0;
    void* d_pf_ws = nullptr;  // prefill V staging copy (long prompts)
    size_t pf_ws_bytes = 0;

    bool planned = false, plan_decode = false;
    int plan_n = 0, plan_total = 0, plan_max_q = 0, plan_max_ctx = 0;
    // mixed step: n_dec one-row sequences (longest context dec_max_ctx) and the longer ones
    // (pf_max_q rows at most, pf_total in all)
    bool plan_mixed = false;
    int plan_n_dec = 0, plan_dec_max_ctx = 0, plan_pf_max_q = 0, plan_pf_total = 0;
    // decode step whose new positions all sit in blocks held by their sequence alone (reference
    // count 1), so no other sequence of the step reads them: the fused KV write may run
    bool plan_private = false;

    KvBatchImpl(int L, int nblk, int nseq, int max_len, int max_tok, int H, int G, int D, int bs,
                int dt)
        : num_layers(L),
          max_seqs(nseq),
          max_seq_len(max_len),
          max_tokens(max_tok),
          num_heads(H),
          kv_heads(G),
          head_dim(D),
          block_size(bs),
          dtype(dt),
          num_blocks(nblk),
          max_blocks((int)(((int64_t)max_len + bs - 1) / bs)),
          num_slots((int64_t)nblk * bs),
          allocator(nblk),
          tables(nseq, BlockTable(bs)),
          live(nseq, 0) {}

    // A mixed step (one-row and longer sequences together) also uploads its tables and lengths
    // again, one-row sequences first, with each entry's first packed row and the cu_seqlens of
    // the longer sequences alone: [max_seqs x max_blocks] | [max_seqs] | [max_seqs] |
    // [max_seqs + 1].
    int64_t plan_ints() const {
        return (int64_t)max_seqs * max_blocks + max_seqs + max_seqs + 1 + 2 * (int64_t)max_tokens +
               (int64_t)max_seqs * max_blocks + 3 * (int64_t)max_seqs + 1;
    }
    int32_t* d_tables() const { return d_plan; }
    int32_t* d_lens() const { return d_plan + (int64_t)max_seqs * max_blocks; }
    int32_t* d_cu() const { return d_lens() + max_seqs; }
    int32_t* d_slots() const { return d_cu() + max_seqs + 1; }
    int32_t* d_pos() const { return d_slots() + max_tokens; }
    int32_t* d_mtab() const { return d_plan + off_mtab(); }
    int32_t* d_mlens() const { return d_plan + off_mlens(); }
    int32_t* d_mrows() const { return d_plan + off_mrows(); }
    int32_t* d_mcu() const { return d_plan + off_mcu(); }
    int64_t off_lens() const { return (int64_t)max_seqs * max_blocks; }
    int64_t off_cu() const { return off_lens() + max_seqs; }
    int64_t off_slots() const { return off_cu() + max_seqs + 1; }
    int64_t off_pos() const { return off_slots() + max_tokens; }
    int64_t off_mtab() const { return off_pos() + max_tokens; }
    int64_t off_mlens() const { return off_mtab() + (int64_t)max_seqs * max_blocks; }
    int64_t off_mrows() const { return off_mlens() + max_seqs; }
    int64_t off_mcu() const { return off_mrows() + max_seqs; }

    ~KvBatchImpl() {
        if (plan_done) {
            if (plan_pending) (void)hipEventSynchronize(plan_done);
            (void)hipEventDestroy(plan_done);
        }
        for (void* p : k_pools)
            if (p) (void)hipFree(p);
        for (void* p : v_pools)
            if (p) (void)hipFree(p);
        if (d_plan) (void)hipFree(d_plan);
        if (h_plan) (void)hipHostFree(h_plan);
        if (d_ws) (void)hipFree(d_ws);
        if (d_pf_ws) (void)hipFree(d_pf_ws);
    }

    int alloc_device() {
        const size_t pool_bytes = (size_t)kv_heads * num_slots * head_dim * elem_bytes(dtype);
        k_pools.assign(num_layers, nullptr);
        v_pools.assign(num_layers, nullptr);
        for (int l = 0; l < num_layers; l++) {
            if (check_hip(hipMalloc(&k_pools[l], pool_bytes), "kv_batch: pool allocation") ||
                check_hip(hipMalloc(&v_pools[l], pool_bytes), "kv_batch: pool allocation") ||
                check_hip(hipMemset(k_pools[l], 0, pool_bytes), "kv_batch: pool zero fill") ||
                check_hip(hipMemset(v_pools[l], 0, pool_bytes), "kv_batch: pool zero fill"))
                return FLOUR_ERR_HIP;
        }
        const size_t plan_bytes = (size_t)plan_ints() * sizeof(int32_t);
        if (check_hip(hipMalloc(&d_plan, plan_bytes), "kv_batch: plan allocation") ||
            check_hip(hipHostMalloc(&h_plan, plan_bytes, hipHostMallocDefault),
                      "kv_batch: pinned staging") ||
            check_hip(hipEventCreateWithFlags(&plan_done, hipEventDisableTiming),
                      "kv_batch: event"))
            return FLOUR_ERR_HIP;
        if (flour_hip_paged_decode_workspace_size(max_seqs, num_heads, kv_heads, head_dim,
                                                  max_seq_len, &ws_bytes) != FLOUR_OK)
            return FLOUR_ERR_INVALID_ARGUMENT;
        if (ws_bytes && check_hip(hipMalloc(&d_ws, ws_bytes), "kv_batch: decode workspace"))
            return FLOUR_ERR_HIP;
        // The prefill staging copy serves steps whose rows average at least 1,536 per sequence
        // (the only ones that take it), so at most max_tokens / 1,536 sequences.
        const int pf_seqs = std::max(1, std::min(max_seqs, max_tokens / 1536));
        if (flour_hip_varlen_prefill_workspace_size(pf_seqs, max_blocks, block_size, kv_heads,
                                                    head_dim, dtype, &pf_ws_bytes) != FLOUR_OK)
            return FLOUR_ERR_INVALID_ARGUMENT;
        if (pf_ws_bytes &&
            check_hip(hipMalloc(&d_pf_ws, pf_ws_bytes), "kv_batch: prefill workspace"))
            return FLOUR_ERR_HIP;
        device = true;
        return FLOUR_OK;
    }

    int need_live(int id) const {
        if (id < 0 || id >= max_seqs || !live[id]) {
            set_error("kv_batch: no live sequence %d", id);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        return FLOUR_OK;
    }

    // ---- sequences
    int add_sequence(int* id) {
        for (int i = 0; i < max_seqs; i++) {
            if (!live[i]) {
                live[i] = 1;
                tables[i].clear();
                *id = i;
                return FLOUR_OK;
            }
        }
        set_error("kv_batch: all %d sequence slots are in use", max_seqs);
        return FLOUR_ERR_CAPACITY;
    }
    void release(int id) {
        for (int b : tables[id].blocks()) allocator.decref(b);
        tables[id].clear();
        planned = false;
    }
    int remove_sequence(int id) {
        if (int rc = need_live(id)) return rc;
        release(id);
        live[id] = 0;
        return FLOUR_OK;
    }
    int reset_sequence(int id) {
        if (int rc = need_live(id)) return rc;
        release(id);
        return FLOUR_OK;
    }
    // Cache::allocate_kv (cache.rs:429-447) for one sequence
    int allocate_kv(int id, int n) {
        if (int rc = need_live(id)) return rc;
        BlockTable& t = tables[id];
        if (n < 0) {
            set_error("kv_batch: negative seq_len %d", n);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        const int64_t end = (int64_t)t.len() + n;
        if (end > max_seq_len) {
            set_error("paged kv cache overflow: %lld tokens exceeds max_seq_len %d",
                      (long long)end, max_seq_len);
            return FLOUR_ERR_CAPACITY;
        }
        t.reserve_blocks((end + block_size - 1) / block_size);
        while (t.capacity() < end) {
            const int b = allocator.allocate();
            if (b < 0) {
                set_error("out of kv blocks");
                return FLOUR_ERR_OUT_OF_BLOCKS;
            }
            t.push_block(b);
        }
        t.advance(n);
        planned = false;
        return FLOUR_OK;
    }
    // KvCache::match_prefix (cache.rs:112-143) into an empty sequence
    int match_prefix(int id, const uint32_t* tok, int n) {
        if (int rc = need_live(id)) return rc;
        BlockTable& t = tables[id];
        if (t.len() != 0 || !t.blocks().empty()) {
            set_error("kv_batch: match_prefix needs an empty sequence (reset it first)");
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        const int bs = block_size, full = n / bs;
        const int reusable = (n % bs == 0) ? (full > 0 ? full - 1 : 0) : full;
        uint64_t parent = PREFIX_SEED;
        int matched = 0;
        t.reserve_blocks(reusable);
        for (int b = 0; b < reusable; b++) {
            const uint32_t* chunk = tok + (int64_t)b * bs;
            const uint64_t h = block_hash(parent, chunk, bs);
            const int blk = registry.get(h, chunk, bs);
            if (blk < 0) break;
            t.push_block(blk);
            allocator.incref(blk);
            matched += bs;
            parent = h;
        }
        t.advance(matched);
        planned = false;
        return matched;
    }
    // KvCache::register_prefix (cache.rs:145-159)
    int register_prefix(int id, const uint32_t* tok, int n) {
        if (int rc = need_live(id)) return rc;
        const BlockTable& t = tables[id];
        const int bs = block_size, full = n / bs;
        if (full > (int)t.blocks().size()) {
            set_error("kv_batch: register_prefix over %d full blocks, the sequence holds %d", full,
                      (int)t.blocks().size());
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        uint64_t parent = PREFIX_SEED;
        for (int b = 0; b < full; b++) {
            const uint32_t* chunk = tok + (int64_t)b * bs;
            const uint64_t h = block_hash(parent, chunk, bs);
            if (!registry.contains(h)) {
                const int blk = t.block_at(b);
                registry.insert(h, chunk, bs, blk);
                allocator.incref(blk);
            }
            parent = h;
        }
        return FLOUR_OK;
    }
    void clear_prefix_cache() {
        for (int b : registry.drain_block_ids()) allocator.decref(b);
    }

    // ---- the step plan
    int plan(const int* ids, const int* q, int n, hipStream_t s) {
        planned = false;
        if (n < 1 || n > max_seqs || !ids || !q) {
            set_error("kv_batch: plan over %d sequences (1 .. %d)", n, max_seqs);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        std::vector<uint8_t> seen(max_seqs, 0);
        int64_t total = 0;
        int max_q = 0, max_ctx = 0;
        bool decode = true;
        for (int i = 0; i < n; i++) {
            if (int rc = need_live(ids[i])) return rc;
            if (seen[ids[i]]++) {
                set_error("kv_batch: sequence %d listed twice in one step", ids[i]);
                return FLOUR_ERR_INVALID_ARGUMENT;
            }
            const int len = tables[ids[i]].len();
            if (q[i] < 1 || q[i] > len) {
                set_error("kv_batch: sequence %d brings %d new rows over %d live positions",
                          ids[i], q[i], len);
                return FLOUR_ERR_INVALID_ARGUMENT;
            }
            total += q[i];
            max_q = std::max(max_q, q[i]);
            max_ctx = std::max(max_ctx, len);
            decode = decode && q[i] == 1;
        }
        if (total > max_tokens) {
            set_error("kv_batch: %lld new rows exceed max_batch_tokens %d", (long long)total,
                      max_tokens);
            return FLOUR_ERR_CAPACITY;
        }
        if (!device) {
            set_error("kv_batch: no device pool");
            return FLOUR_ERR_UNSUPPORTED;
        }
        if (plan_pending) {  // the previous upload must have read the staging buffer
            plan_pending = false;
            if (check_hip(hipEventSynchronize(plan_done), "kv_batch: staging wait"))
                return FLOUR_ERR_HIP;
        }
        int32_t* tab = h_plan;
        int32_t* lens = h_plan + off_lens();
        int32_t* cu = h_plan + off_cu();
        int32_t* slots = h_plan + off_slots();
        int32_t* pos = h_plan + off_pos();
        cu[0] = 0;
        for (int i = 0; i < n; i++) {
            const BlockTable& t = tables[ids[i]];
            const auto& b = t.blocks();
            int32_t* row = tab + (int64_t)i * max_blocks;
            for (int j = 0; j < (int)b.size(); j++) row[j] = b[j];
            for (int j = (int)b.size(); j < max_blocks; j++) row[j] = 0;
            lens[i] = t.len();
            cu[i + 1] = cu[i] + q[i];
            for (int p = t.len() - q[i], k = cu[i]; p < t.len(); p++, k++) {
                slots[k] = (int32_t)t.slot(p);
                pos[k] = p;
            }
        }
        // mixed step: the one-row sequences first (a decode batch), then the others (a prefill
        // batch), each entry with its first packed row
        int n_dec = 0, dec_max_ctx = 0, pf_max_q = 0;
        for (int i = 0; i < n; i++) n_dec += q[i] == 1;
        const bool mixed = n_dec > 0 && n_dec < n;
        if (mixed) {
            int32_t* mtab = h_plan + off_mtab();
            int32_t* mlens = h_plan + off_mlens();
            int32_t* mrows = h_plan + off_mrows();
            int32_t* mcu = h_plan + off_mcu();
            int jd = 0, jp = n_dec;
            mcu[0] = 0;
            for (int i = 0; i < n; i++) {
                const int j = q[i] == 1 ? jd++ : jp++;
                memcpy(mtab + (int64_t)j * max_blocks, tab + (int64_t)i * max_blocks,
                       sizeof(int32_t) * (size_t)max_blocks);
                mlens[j] = lens[i];
                mrows[j] = cu[i];
                if (q[i] == 1) {
                    dec_max_ctx = std::max(dec_max_ctx, lens[i]);
                } else {
                    mcu[j - n_dec + 1] = mcu[j - n_dec] + q[i];
                    pf_max_q = std::max(pf_max_q, q[i]);
                }
            }
        }
        const struct {
            int64_t off, n;
        } parts[9] = {{0, (int64_t)n * max_blocks}, {off_lens(), n}, {off_cu(), n + 1},
                      {off_slots(), total}, {off_pos(), total},
                      {off_mtab(), mixed ? (int64_t)n * max_blocks : 0},
                      {off_mlens(), mixed ? n : 0}, {off_mrows(), mixed ? n : 0},
                      {off_mcu(), mixed ? n - n_dec + 1 : 0}};
        for (const auto& pr : parts)
            if (pr.n > 0)
            if (check_hip(hipMemcpyAsync(d_plan + pr.off, h_plan + pr.off, pr.n * sizeof(int32_t),
                                         hipMemcpyHostToDevice, s),
                          "kv_batch: plan upload"))
                return FLOUR_ERR_HIP;
        if (check_hip(hipEventRecord(plan_done, s), "kv_batch: event record")) return FLOUR_ERR_HIP;
        plan_pending = true;
        planned = true;
        plan_decode = decode;
        plan_n = n;
        plan_total = (int)total;
        plan_max_q = max_q;
        plan_max_ctx = max_ctx;
        plan_mixed = mixed;
        plan_n_dec = n_dec;
        plan_dec_max_ctx = dec_max_ctx;
        plan_pf_max_q = pf_max_q;
        plan_pf_total = (int)(total - n_dec);
        plan_private = decode;
        for (int i = 0; i < n && plan_private; i++) {
            const BlockTable& t = tables[ids[i]];
            plan_private = allocator.ref_count(t.blocks()[(t.len() - 1) / block_size]) == 1;
        }
        return FLOUR_OK;
    }
    // allocate_kv(ids[i], q[i]) for every sequence of the step, then plan(): all checks
    // (sequences, max_seq_len, max_batch_tokens, free blocks, the device pool) come first, so a
    // refused step changes no sequence.
    int step(const int* ids, const int* q, int n, hipStream_t s) {
        planned = false;
        if (n < 1 || n > max_seqs || !ids || !q) {
            set_error("kv_batch: step over %d sequences (1 .. %d)", n, max_seqs);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        std::vector<uint8_t> seen(max_seqs, 0);
        int64_t total = 0, need = 0;
        for (int i = 0; i < n; i++) {
            if (int rc = need_live(ids[i])) return rc;
            if (seen[ids[i]]++) {
                set_error("kv_batch: sequence %d listed twice in one step", ids[i]);
                return FLOUR_ERR_INVALID_ARGUMENT;
            }
            if (q[i] < 1) {
                set_error("kv_batch: sequence %d brings %d new rows", ids[i], q[i]);
                return FLOUR_ERR_INVALID_ARGUMENT;
            }
            const BlockTable& t = tables[ids[i]];
            const int64_t end = (int64_t)t.len() + q[i];
            if (end > max_seq_len) {
                set_error("paged kv cache overflow: %lld tokens exceeds max_seq_len %d",
                          (long long)end, max_seq_len);
                return FLOUR_ERR_CAPACITY;
            }
            need += std::max<int64_t>(0, (end + block_size - 1) / block_size -
                                             (int64_t)t.blocks().size());
            total += q[i];
        }
        if (total > max_tokens) {
            set_error("kv_batch: %lld new rows exceed max_batch_tokens %d", (long long)total,
                      max_tokens);
            return FLOUR_ERR_CAPACITY;
        }
        if (need > allocator.num_free()) {
            set_error("out of kv blocks");
            return FLOUR_ERR_OUT_OF_BLOCKS;
        }
        if (!device) {
            set_error("kv_batch: no device pool");
            return FLOUR_ERR_UNSUPPORTED;
        }
        // table room first (the only step that can fail now), so no sequence changes unless all do
        for (int i = 0; i < n; i++) {
            BlockTable& t = tables[ids[i]];
            t.reserve_blocks((t.len() + (int64_t)q[i] + block_size - 1) / block_size);
        }
        for (int i = 0; i < n; i++)
            if (int rc = allocate_kv(ids[i], q[i])) return rc;  // cannot fail after the checks
        return plan(ids, q, n, s);
    }
    int need_plan(int layer) const {
        if (!planned) {
            set_error("kv_batch: no current plan (plan() after the last change to a sequence)");
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (layer < 0 || layer >= num_layers) {
            set_error("kv_batch: layer %d of %d", layer, num_layers);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        return FLOUR_OK;
    }
};

}  // namespace host
}  // namespace flour

using namespace flour;
using namespace flour::host;

struct flour_kv_batch {
    KvBatchImpl b;
};

#define BATCH_NEED(cond, ...)                  \
    do {                                       \
        if (!(cond)) {                         \
            set_error(__VA_ARGS__);            \
            return FLOUR_ERR_INVALID_ARGUMENT; \
        }                                      \
    } while (0)

extern "C" int flour_kv_batch_create(int num_layers, int num_blocks, int max_seqs,
                                     int max_seq_len, int max_batch_tokens, int num_heads,
                                     int kv_heads, int head_dim, int block_size, int dtype,
                                     int device_pool, flour_kv_batch** out) {
    clear_error();
    BATCH_NEED(out, "kv_batch: null output");
    *out = nullptr;
    BATCH_NEED(num_layers > 0 && num_blocks > 0 && max_seqs > 0 && max_seq_len > 0 &&
                   max_batch_tokens > 0 && num_heads > 0 && kv_heads > 0 &&
                   num_heads % kv_heads == 0 && head_dim > 0 && block_size > 0 &&
                   valid_dtype(dtype),
               "kv_batch: bad shape (layers=%d blocks=%d seqs=%d max_seq_len=%d tokens=%d "
               "heads=%d kv_heads=%d head_dim=%d block_size=%d dtype=%d)",
               num_layers, num_blocks, max_seqs, max_seq_len, max_batch_tokens, num_heads,
               kv_heads, head_dim, block_size, dtype);
    BATCH_NEED((int64_t)num_blocks * block_size < (1ll << 31),
               "kv_batch: %lld slots exceed int32 slot ids", (long long)num_blocks * block_size);
    return abi_guard("kv_batch", [&]() -> int {
        std::unique_ptr<flour_kv_batch> x(new flour_kv_batch{
            KvBatchImpl(num_layers, num_blocks, max_seqs, max_seq_len, max_batch_tokens, num_heads,
                        kv_heads, head_dim, block_size, dtype)});
        if (device_pool) {
            const int rc = x->b.alloc_device();
            if (rc != FLOUR_OK) return rc;
        }
        *out = x.release();
        return FLOUR_OK;
    });
}
extern "C" void flour_kv_batch_destroy(flour_kv_batch* b) { delete b; }

extern "C" int flour_kv_batch_add_sequence(flour_kv_batch* b, int* seq_id) {
    clear_error();
    BATCH_NEED(b && seq_id, "kv_batch: bad arguments");
    return b->b.add_sequence(seq_id);
}
extern "C" int flour_kv_batch_remove_sequence(flour_kv_batch* b, int seq_id) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    return b->b.remove_sequence(seq_id);
}
extern "C" int flour_kv_batch_reset_sequence(flour_kv_batch* b, int seq_id) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    return b->b.reset_sequence(seq_id);
}
extern "C" int flour_kv_batch_allocate_kv(flour_kv_batch* b, int seq_id, int seq_len) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    return abi_guard("kv_batch", [&] { return b->b.allocate_kv(seq_id, seq_len); });
}
extern "C" int flour_kv_batch_len(const flour_kv_batch* b, int seq_id) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    if (int rc = b->b.need_live(seq_id)) return rc;
    return b->b.tables[seq_id].len();
}
extern "C" int flour_kv_batch_free_blocks(const flour_kv_batch* b) {
    return b ? b->b.allocator.num_free() : FLOUR_ERR_INVALID_ARGUMENT;
}
extern "C" int flour_kv_batch_ref_count(const flour_kv_batch* b, int block_id) {
    clear_error();
    BATCH_NEED(b && block_id >= 0 && block_id < b->b.num_blocks, "kv_batch: bad block %d",
               block_id);
    return b->b.allocator.ref_count(block_id);
}
extern "C" int flour_kv_batch_blocks(const flour_kv_batch* b, int seq_id, int32_t* out, int cap,
                                     int* n) {
    clear_error();
    BATCH_NEED(b && n && (out || cap == 0), "kv_batch: bad arguments");
    if (int rc = b->b.need_live(seq_id)) return rc;
    const auto& v = b->b.tables[seq_id].blocks();
    *n = (int)v.size();
    for (int i = 0; i < (int)v.size() && i < cap; i++) out[i] = v[i];
    return FLOUR_OK;
}
extern "C" int flour_kv_batch_match_prefix(flour_kv_batch* b, int seq_id, const uint32_t* tokens,
                                           int n) {
    clear_error();
    BATCH_NEED(b && (tokens || n == 0) && n >= 0, "kv_batch: bad arguments");
    return abi_guard("kv_batch", [&] { return b->b.match_prefix(seq_id, tokens, n); });
}
extern "C" int flour_kv_batch_register_prefix(flour_kv_batch* b, int seq_id,
                                              const uint32_t* tokens, int n) {
    clear_error();
    BATCH_NEED(b && (tokens || n == 0) && n >= 0, "kv_batch: bad arguments");
    return abi_guard("kv_batch", [&] { return b->b.register_prefix(seq_id, tokens, n); });
}
extern "C" int flour_kv_batch_clear_prefix_cache(flour_kv_batch* b) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    return abi_guard("kv_batch", [&]() -> int {
        b->b.clear_prefix_cache();
        return FLOUR_OK;
    });
}
extern "C" int flour_kv_batch_plan(flour_kv_batch* b, const int* seq_ids, const int* seq_q,
                                   int n_seqs, void* stream) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    return abi_guard("kv_batch", [&] {
        return b->b.plan(seq_ids, seq_q, n_seqs, static_cast<hipStream_t>(stream));
    });
}
extern "C" int flour_kv_batch_step(flour_kv_batch* b, const int* seq_ids, const int* seq_q,
                                   int n_seqs, void* stream) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    return abi_guard("kv_batch", [&] {
        return b->b.step(seq_ids, seq_q, n_seqs, static_cast<hipStream_t>(stream));
    });
}
extern "C" int flour_kv_batch_write_kv(flour_kv_batch* b, int layer, const void* k, const void* v,
                                       int64_t stride_tok, int64_t stride_head, void* stream) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    KvBatchImpl& x = b->b;
    if (int rc = x.need_plan(layer)) return rc;
    return flour_hip_kv_write(k, v, stride_tok, stride_head, x.k_pools[layer], x.v_pools[layer],
                              x.d_slots(), x.plan_total, x.kv_heads, x.head_dim, x.num_slots,
                              x.dtype, stream);
}
extern "C" int flour_kv_batch_rope_write_kv(flour_kv_batch* b, int layer, void* q_out,
                                            const void* q, int64_t q_stride_tok,
                                            int64_t q_stride_head, int num_heads, const void* k,
                                            const void* v, int64_t kv_stride_tok,
                                            int64_t kv_stride_head, const void* cos_table,
                                            const void* sin_table, int max_pos, void* stream) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    KvBatchImpl& x = b->b;
    if (int rc = x.need_plan(layer)) return rc;
    BATCH_NEED(num_heads > 0 && num_heads <= x.num_heads && num_heads % x.kv_heads == 0,
               "kv_batch: %d query heads (built for up to %d, %d kv heads)", num_heads,
               x.num_heads, x.kv_heads);
    BATCH_NEED(max_pos >= x.max_seq_len, "kv_batch: RoPE tables of %d rows do not cover max_seq_len %d",
               max_pos, x.max_seq_len);
    return flour_hip_rope_kv_write(q_out, q, q_stride_tok, q_stride_head, num_heads, k, v,
                                   kv_stride_tok, kv_stride_head, x.k_pools[layer],
                                   x.v_pools[layer], x.d_slots(), x.d_pos(), cos_table, sin_table,
                                   max_pos, x.plan_total, x.kv_heads, x.head_dim, x.num_slots,
                                   x.dtype, stream);
}
extern "C" int flour_kv_batch_attention(flour_kv_batch* b, int layer, const void* q,
                                        int num_heads, int64_t q_stride_tok, int64_t q_stride_head,
                                        void* out, int out_dtype, int64_t o_stride_tok,
                                        int64_t o_stride_head, float scale, void* stream) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    KvBatchImpl& x = b->b;
    if (int rc = x.need_plan(layer)) return rc;
    BATCH_NEED(num_heads > 0 && num_heads <= x.num_heads && num_heads % x.kv_heads == 0,
               "kv_batch: %d query heads (built for up to %d, %d kv heads)", num_heads,
               x.num_heads, x.kv_heads);
    if (x.plan_decode) {
        BATCH_NEED(q_stride_head == x.head_dim && q_stride_tok == (int64_t)num_heads * x.head_dim &&
                       o_stride_head == x.head_dim &&
                       o_stride_tok == (int64_t)num_heads * x.head_dim,
                   "kv_batch: decode needs q and out as (sequences, num_heads, head_dim) "
                   "contiguous");
        return flour_hip_paged_decode(out, out_dtype, q, x.k_pools[layer], x.v_pools[layer],
                                      x.d_tables(), x.max_blocks, x.d_lens(), x.plan_n,
                                      num_heads, x.kv_heads, x.head_dim, x.block_size,
                                      x.num_slots, x.plan_max_ctx, scale, x.dtype, x.d_ws,
                                      x.ws_bytes, stream);
    }
    // A mixed step runs its one-row sequences on the decode kernel and the rest on the prefill
    // kernel (both over the packed rows, through row indices), when both take the shape.
    const bool packed = q_stride_head == x.head_dim &&
                        q_stride_tok == (int64_t)num_heads * x.head_dim &&
                        o_stride_head == x.head_dim &&
                        o_stride_tok == (int64_t)num_heads * x.head_dim;
    const int n_pf = x.plan_n - x.plan_n_dec;
    if (x.plan_mixed && g_batch_split && packed &&
        decode_mfma_supported(x.dtype, x.head_dim, x.block_size, num_heads / x.kv_heads,
                              x.plan_n_dec, num_heads, x.num_slots, q, x.k_pools[layer],
                              x.v_pools[layer])) {
        int rc = varlen_prefill_rows(
            out, out_dtype, o_stride_tok, o_stride_head, q, q_stride_tok, q_stride_head,
            x.k_pools[layer], x.v_pools[layer], x.d_mcu(), x.d_mrows() + x.plan_n_dec,
            x.d_mlens() + x.plan_n_dec, x.d_mtab() + (int64_t)x.plan_n_dec * x.max_blocks,
            x.max_blocks, n_pf, x.plan_pf_max_q, x.plan_pf_total, num_heads, x.kv_heads,
            x.head_dim, x.block_size, x.num_slots, scale, x.dtype, x.d_pf_ws, x.pf_ws_bytes,
            stream);
        if (rc == FLOUR_OK)
            return paged_decode_rows(out, out_dtype, q, x.k_pools[layer], x.v_pools[layer],
                                     x.d_mtab(), x.max_blocks, x.d_mlens(), x.d_mrows(),
                                     x.plan_n_dec, num_heads, x.kv_heads, x.head_dim,
                                     x.block_size, x.num_slots, x.plan_dec_max_ctx, scale,
                                     x.dtype, x.d_ws, x.ws_bytes, stream);
        if (rc != FLOUR_ERR_UNSUPPORTED) return rc;
        clear_error();  // nothing launched: every row through the prefill kernel
    }
    return flour_hip_varlen_prefill_ws(out, out_dtype, o_stride_tok, o_stride_head, q,
                                       q_stride_tok, q_stride_head, x.k_pools[layer],
                                       x.v_pools[layer], x.d_cu(), x.d_lens(), x.d_tables(),
                                       x.max_blocks, x.plan_n, x.plan_max_q, x.plan_total,
                                       num_heads, x.kv_heads, x.head_dim, x.block_size,
                                       x.num_slots, scale, x.dtype, x.d_pf_ws, x.pf_ws_bytes,
                                       stream);
}
extern "C" int flour_kv_batch_write_kv_attention(flour_kv_batch* b, int layer, const void* k,
                                                 const void* v, int64_t kv_stride_tok,
                                                 int64_t kv_stride_head, const void* q,
                                                 int num_heads, int64_t q_stride_tok,
                                                 int64_t q_stride_head, void* out, int out_dtype,
                                                 int64_t o_stride_tok, int64_t o_stride_head,
                                                 float scale, void* stream) {
    clear_error();
    BATCH_NEED(b, "kv_batch: null");
    KvBatchImpl& x = b->b;
    if (int rc = x.need_plan(layer)) return rc;
    BATCH_NEED(num_heads > 0 && num_heads <= x.num_heads && num_heads % x.kv_heads == 0,
               "kv_batch: %d query heads (built for up to %d, %d kv heads)", num_heads,
               x.num_heads, x.kv_heads);
    const bool packed = q_stride_head == x.head_dim &&
                        q_stride_tok == (int64_t)num_heads * x.head_dim &&
                        o_stride_head == x.head_dim &&
                        o_stride_tok == (int64_t)num_heads * x.head_dim;
    if (x.plan_decode && x.plan_private && g_batch_fuse && packed) {
        const int rc = paged_decode_write_kv(
            out, out_dtype, q, x.k_pools[layer], x.v_pools[layer], x.d_tables(), x.max_blocks,
            x.d_lens(), x.plan_n, num_heads, x.kv_heads, x.head_dim, x.block_size, x.num_slots,
            x.plan_max_ctx, scale, x.dtype, x.d_ws, x.ws_bytes, k, v, kv_stride_tok,
            kv_stride_head, x.d_slots(), stream);
        if (rc != FLOUR_ERR_UNSUPPORTED) return rc;
        clear_error();  // nothing launched: the two-launch form
    }
    if (int rc = flour_kv_batch_write_kv(b, layer, k, v, kv_stride_tok, kv_stride_head, stream))
        return rc;
    return flour_kv_batch_attention(b, layer, q, num_heads, q_stride_tok, q_stride_head, out,
                                    out_dtype, o_stride_tok, o_stride_head, scale, stream);
}
extern "C" int flour_kv_batch_pool(const flour_kv_batch* b, int layer, void** k_pool,
                                   void** v_pool, int64_t* num_slots) {
    clear_error();
    BATCH_NEED(b && k_pool && v_pool && num_slots, "kv_batch: bad arguments");
    BATCH_NEED(b->b.device, "kv_batch: no device pool");
    BATCH_NEED(layer >= 0 && layer < b->b.num_layers, "kv_batch: layer %d of %d", layer,
               b->b.num_layers);
    *k_pool = b->b.k_pools[layer];
    *v_pool = b->b.v_pools[layer];
    *num_slots = b->b.num_slots;
    return FLOUR_OK;
}

extern "C" int flour_hip_set_batch_fuse(int on) {
    flour::host::g_batch_fuse = on ? 1 : 0;
    return FLOUR_OK;
}
extern "C" int flour_hip_set_batch_split(int on) {
    flour::host::g_batch_split = on ? 1 : 0;
    return FLOUR_OK;
}
