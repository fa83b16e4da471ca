// kv_cache.cpp — host-side KV-cache bookkeeping over a device pool (include/flour_cache.h).
//
// Restates the reference's per-sequence cache: BlockAllocator and BlockTable
// (src/models/common/paged.rs:7-121), the prefix registry (src/models/common/prefix.rs:1-60)
// and KvCache / Cache (src/models/common/cache.rs:13-165, :429-505), with the pool of
// PagedKvPool::new (paged.rs:138-167) in device memory. The attention call marshals the live
// block table to the device and launches the kernels of flour_hip.h, which replaces
// Cache::kv_blocks + paged_attention (attention.rs:104-109).
//
// The allocator, table and prefix registry are in kv_host.h.
//
// Bundles: export_bundle / import_bundle restate Cache::export_prefix_bundle /
// import_prefix_bundle (cache.rs:166-340) with KvBundleCodec::encode / decode
// (src/kv_cache/bundle.rs:108-214) on the FLKV frame; the payload moves between the device pools
// and the host bytes through a device staging buffer (kv_bundle.hip packs / unpacks it).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <memory>
#include <unordered_map>
#include <vector>

#include "flkv_codec.h"
#include "flour_cache.h"
#include "flour_common.h"
#include "flour_hip.h"
#include "kv_bundle.h"
#include "kv_host.h"

namespace flour {
namespace host {

// ---------------------------------------------------------------- KvCache + device pool
struct KvCacheImpl {
    int num_layers, max_seq_len, num_heads, kv_heads, head_dim, block_size, dtype;
    int num_blocks;
    int64_t num_slots;
    BlockAllocator allocator;
    BlockTable table;
    PrefixRegistry registry;

    bool device = false;
    std::vector<void*> k_pools, v_pools;  // per layer, (kv_heads, num_slots, head_dim)
    // device inputs of the kernels: [0, num_blocks) block table, then kv_len, cu_seqlens (2),
    // then the slot mapping of the current batch (max_seq_len entries)
    int32_t* d_meta = nullptr;
    int32_t* h_meta = nullptr;  // pinned staging of the same layout
    hipEvent_t meta_done = nullptr;
    bool meta_pending = false;
    void* d_ws = nullptr;  // decode split-context partials
    size_t ws_bytes = 0;
    void* d_pf_ws = nullptr;  // prefill V staging copy (long prompts)
    size_t pf_ws_bytes = 0;
    void** d_pool_ptrs = nullptr;  // device copy of the K pool addresses, then the V ones
    void* d_stage = nullptr;       // bundle staging, whole logical blocks (allocated on use)
    size_t stage_bytes = 0;
    uint64_t table_version = 1, uploaded_version = 0;
    int uploaded_len = -1;

    KvCacheImpl(int L, int max_len, int H, int G, int D, int bs, int dt)
        : num_layers(L),
          max_seq_len(max_len),
          num_heads(H),
          kv_heads(G),
          head_dim(D),
          block_size(bs),
          dtype(dt),
          num_blocks((int)(((int64_t)max_len + bs - 1) / bs)),
          num_slots((int64_t)num_blocks * bs),
          allocator(num_blocks),
          table(bs) {}

    int64_t meta_ints() const { return (int64_t)num_blocks + 3 + max_seq_len; }
    int32_t* d_table() const { return d_meta; }
    int32_t* d_kv_len() const { return d_meta + num_blocks; }
    int32_t* d_cu() const { return d_meta + num_blocks + 1; }
    int32_t* d_slots() const { return d_meta + num_blocks + 3; }

    ~KvCacheImpl() {
        if (meta_done) {
            if (meta_pending) (void)hipEventSynchronize(meta_done);
            (void)hipEventDestroy(meta_done);
        }
        for (void* p : k_pools)
            if (p) (void)hipFree(p);
        for (void* p : v_pools)
            if (p) (void)hipFree(p);
        if (d_meta) (void)hipFree(d_meta);
        if (h_meta) (void)hipHostFree(h_meta);
        if (d_ws) (void)hipFree(d_ws);
        if (d_pf_ws) (void)hipFree(d_pf_ws);
        if (d_pool_ptrs) (void)hipFree(d_pool_ptrs);
        if (d_stage) (void)hipFree(d_stage);
    }

    int alloc_device() {
        const size_t pool_bytes = (size_t)kv_heads * num_slots * head_dim * elem_bytes(dtype);
        k_pools.assign(num_layers, nullptr);
        v_pools.assign(num_layers, nullptr);
        for (int l = 0; l < num_layers; l++) {
            if (check_hip(hipMalloc(&k_pools[l], pool_bytes), "kv_cache: pool allocation") ||
                check_hip(hipMalloc(&v_pools[l], pool_bytes), "kv_cache: pool allocation") ||
                check_hip(hipMemset(k_pools[l], 0, pool_bytes), "kv_cache: pool zero fill") ||
                check_hip(hipMemset(v_pools[l], 0, pool_bytes), "kv_cache: pool zero fill"))
                return FLOUR_ERR_HIP;
        }
        const size_t meta_bytes = (size_t)meta_ints() * sizeof(int32_t);
        if (check_hip(hipMalloc(&d_meta, meta_bytes), "kv_cache: table allocation") ||
            check_hip(hipHostMalloc(&h_meta, meta_bytes, hipHostMallocDefault),
                      "kv_cache: pinned staging") ||
            check_hip(hipEventCreateWithFlags(&meta_done, hipEventDisableTiming),
                      "kv_cache: event"))
            return FLOUR_ERR_HIP;
        if (flour_hip_paged_decode_workspace_size(1, num_heads, kv_heads, head_dim, max_seq_len,
                                                  &ws_bytes) != FLOUR_OK)
            return FLOUR_ERR_INVALID_ARGUMENT;
        if (ws_bytes && check_hip(hipMalloc(&d_ws, ws_bytes), "kv_cache: decode workspace"))
            return FLOUR_ERR_HIP;
        if (flour_hip_varlen_prefill_workspace_size(1, num_blocks, block_size, kv_heads, head_dim,
                                                    dtype, &pf_ws_bytes) != FLOUR_OK)
            return FLOUR_ERR_INVALID_ARGUMENT;
        if (pf_ws_bytes &&
            check_hip(hipMalloc(&d_pf_ws, pf_ws_bytes), "kv_cache: prefill workspace"))
            return FLOUR_ERR_HIP;
        std::vector<void*> ptrs(k_pools);
        ptrs.insert(ptrs.end(), v_pools.begin(), v_pools.end());
        if (check_hip(hipMalloc(&d_pool_ptrs, ptrs.size() * sizeof(void*)),
                      "kv_cache: pool address table") ||
            check_hip(hipMemcpy(d_pool_ptrs, ptrs.data(), ptrs.size() * sizeof(void*),
                                hipMemcpyHostToDevice),
                      "kv_cache: pool address table"))
            return FLOUR_ERR_HIP;
        device = true;
        return FLOUR_OK;
    }

    // Wait until the previous upload has read the pinned staging buffer before rewriting it.
    int staging_ready() {
        if (!meta_pending) return FLOUR_OK;
        meta_pending = false;
        return check_hip(hipEventSynchronize(meta_done), "kv_cache: staging wait");
    }

    // Copy ints [first, first + count) of the staging layout to the device on `s`.
    int upload(int first, int count, hipStream_t s) {
        if (check_hip(hipMemcpyAsync(d_meta + first, h_meta + first, count * sizeof(int32_t),
                                     hipMemcpyHostToDevice, s),
                      "kv_cache: table upload") ||
            check_hip(hipEventRecord(meta_done, s), "kv_cache: event record"))
            return FLOUR_ERR_HIP;
        meta_pending = true;
        return FLOUR_OK;
    }

    // Block table, live length and cu_seqlens for an attention call over seq_q rows.
    int upload_table(int seq_q, hipStream_t s) {
        const int len = table.len();
        if (uploaded_version == table_version && uploaded_len == len && h_meta[num_blocks + 2] == seq_q)
            return FLOUR_OK;
        int rc = staging_ready();
        if (rc) return rc;
        const auto& b = table.blocks();
        for (int i = 0; i < (int)b.size(); i++) h_meta[i] = b[i];
        for (int i = (int)b.size(); i < num_blocks; i++) h_meta[i] = 0;
        h_meta[num_blocks] = len;
        h_meta[num_blocks + 1] = 0;
        h_meta[num_blocks + 2] = seq_q;
        rc = upload(0, num_blocks + 3, s);
        if (rc) return rc;
        uploaded_version = table_version;
        uploaded_len = len;
        return FLOUR_OK;
    }

    // ---- KvCache operations
    int allocate_kv(int seq_len) {
        const int64_t end = (int64_t)table.len() + seq_len;
        if (seq_len < 0) {
            set_error("kv_cache: negative seq_len %d", seq_len);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (end > max_seq_len) {
            set_error("paged kv cache overflow: %lld tokens exceeds max_seq_len %d",
                      (long long)end, max_seq_len);
            return FLOUR_ERR_CAPACITY;
        }
        table.reserve_blocks((end + table.block_size() - 1) / table.block_size());
        while (table.capacity() < end) {
            const int id = allocator.allocate();
            if (id < 0) {
                set_error("out of kv blocks");
                return FLOUR_ERR_OUT_OF_BLOCKS;
            }
            table.push_block(id);
            table_version++;
        }
        table.advance(seq_len);
        return FLOUR_OK;
    }

    void reset_sequence() {
        for (int id : table.blocks()) allocator.decref(id);
        table.clear();
        table_version++;
    }

    int match_prefix(const uint32_t* tok, int n) {
        const int bs = table.block_size();
        const int full = n / bs;
        const int reusable = (n % bs == 0) ? (full > 0 ? full - 1 : 0) : full;
        uint64_t parent = PREFIX_SEED;
        int matched = 0;
        table.reserve_blocks(reusable);
        for (int b = 0; b < reusable; b++) {
            const uint32_t* chunk = tok + (int64_t)b * bs;
            const uint64_t h = block_hash(parent, chunk, bs);
            const int id = registry.get(h, chunk, bs);
            if (id < 0) break;
            table.push_block(id);
            allocator.incref(id);
            table_version++;
            matched += bs;
            parent = h;
        }
        table.advance(matched);
        return matched;
    }

    int register_prefix(const uint32_t* tok, int n) {
        const int bs = table.block_size();
        const int full = n / bs;
        if (full > (int)table.blocks().size()) {
            set_error("kv_cache: register_prefix over %d full blocks, the sequence holds %d", full,
                      (int)table.blocks().size());
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        uint64_t parent = PREFIX_SEED;
        for (int b = 0; b < full; b++) {
            const uint32_t* chunk = tok + (int64_t)b * bs;
            const uint64_t h = block_hash(parent, chunk, bs);
            if (!registry.contains(h)) {
                const int id = table.block_at(b);
                registry.insert(h, chunk, bs, id);
                allocator.incref(id);  // the registry holds its own reference
            }
            parent = h;
        }
        return FLOUR_OK;
    }

    void clear_prefix_cache() {
        for (int id : registry.drain_block_ids()) allocator.decref(id);
    }

    // ---- FLKV bundles
    size_t bundle_block_bytes() const {  // one logical block of every layer, K and V
        return (size_t)num_layers * 2 * kv_heads * block_size * head_dim * elem_bytes(dtype);
    }
    static constexpr size_t STAGE_CAP = 64u << 20;  // staging chunk, whole logical blocks
    // Blocks per staging chunk for a bundle of nb logical blocks; grows the buffer on demand.
    int stage_blocks(int nb) {
        const size_t per = bundle_block_bytes();
        const int cb = (int)std::max<size_t>(1, std::min<size_t>(nb, STAGE_CAP / per));
        const size_t need = (size_t)cb * per;
        if (need > stage_bytes) {
            if (d_stage) (void)hipFree(d_stage);
            d_stage = nullptr;
            stage_bytes = 0;
            if (check_hip(hipMalloc(&d_stage, need), "kv bundle: staging allocation")) return -1;
            stage_bytes = need;
        }
        return cb;
    }

    int export_bundle(const char* model_id, const uint32_t* ids, int n_ids, int token_count,
                      void* out, size_t cap, size_t* out_len, hipStream_t s) {
        const int bs = table.block_size();
        if (token_count <= 0 || token_count % bs != 0) {
            set_error("export token_count %d not aligned to block size %d", token_count, bs);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (token_count > table.len()) {
            set_error("export token_count %d exceeds live len %d", token_count, table.len());
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (n_ids < token_count || !ids) {
            set_error("token_ids len %d shorter than token_count %d", ids ? n_ids : 0, token_count);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        flkv::Meta m;
        m.model_id = model_id ? model_id : "";
        m.token_count = (uint64_t)token_count;
        m.token_ids.assign(ids, ids + token_count);
        m.block_size = (uint64_t)bs;
        m.num_layers = (uint64_t)num_layers;
        m.num_kv_heads = (uint64_t)kv_heads;
        m.head_dim = (uint64_t)head_dim;
        m.dtype = dtype;
        const std::string hdr = flkv::encode_header(m);
        const int nb = token_count / bs;
        const size_t per = bundle_block_bytes();
        const size_t head_end = flkv::PREFIX + hdr.size();
        const size_t total = head_end + (size_t)nb * per;
        *out_len = total;
        if (!out) return FLOUR_OK;  // size query
        if (cap < total) {
            set_error("kv bundle: output buffer of %zu bytes, the bundle needs %zu", cap, total);
            return FLOUR_ERR_CAPACITY;
        }
        if (!device) {
            set_error("kv_cache: no device pool");
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        uint8_t* o = static_cast<uint8_t*>(out);
        memcpy(o, flkv::MAGIC, 4);
        o[4] = (uint8_t)(flkv::VERSION & 0xff);
        o[5] = (uint8_t)(flkv::VERSION >> 8);
        const uint32_t hl = (uint32_t)hdr.size();
        for (int i = 0; i < 4; i++) o[6 + i] = (uint8_t)(hl >> (8 * i));
        memcpy(o + flkv::PREFIX, hdr.data(), hdr.size());
        int rc = upload_table(1, s);
        if (rc) return rc;
        const int cb = stage_blocks(nb);
        if (cb < 0) return FLOUR_ERR_HIP;
        for (int b0 = 0; b0 < nb; b0 += cb) {
            const int n = std::min(cb, nb - b0);
            rc = launch_kv_bundle_copy(0, d_stage, d_pool_ptrs, d_table(), b0, n, num_layers,
                                       kv_heads, block_size, head_dim, num_slots,
                                       elem_bytes(dtype), s);
            if (rc) return rc;
            if (check_hip(hipMemcpyAsync(o + head_end + (size_t)b0 * per, d_stage, (size_t)n * per,
                                         hipMemcpyDeviceToHost, s),
                          "kv bundle: device-to-host copy"))
                return FLOUR_ERR_HIP;
        }
        return check_hip(hipStreamSynchronize(s), "kv bundle: export");
    }

    int import_bundle(const void* bytes, size_t len, const uint32_t* prompt, int n_prompt,
                      int* imported, hipStream_t s) {
        // ---- KvBundleCodec::decode (bundle.rs:145-214)
        const uint8_t* p = static_cast<const uint8_t*>(bytes);
        if (!p || len < flkv::PREFIX) {
            set_error("bundle too short: %zu bytes", p ? len : (size_t)0);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (memcmp(p, flkv::MAGIC, 4) != 0) {
            set_error("bad bundle magic");
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        const unsigned version = (unsigned)p[4] | ((unsigned)p[5] << 8);
        if (version != flkv::VERSION) {
            set_error("unsupported bundle version %u", version);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        const size_t hl = (size_t)p[6] | ((size_t)p[7] << 8) | ((size_t)p[8] << 16) |
                          ((size_t)p[9] << 24);
        const size_t head_end = flkv::PREFIX + hl;
        if (len < head_end) {
            set_error("bundle header truncated");
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        flkv::Meta m;
        flkv::Reader rd(reinterpret_cast<const char*>(p + flkv::PREFIX), hl);
        if (!rd.parse(m)) {
            set_error("bundle header: %s", rd.err.c_str());
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (m.block_size == 0) {
            set_error("bundle block_size is zero");
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (m.token_count == 0 || m.token_count % m.block_size != 0) {
            set_error("bundle token_count %llu not block aligned to %llu",
                      (unsigned long long)m.token_count, (unsigned long long)m.block_size);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (m.token_ids.size() != m.token_count) {
            set_error("bundle token_ids len %zu != token_count %llu", m.token_ids.size(),
                      (unsigned long long)m.token_count);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        const uint64_t nb64 = m.token_count / m.block_size;
        // expected payload, with overflow checks (sizes come from the wire)
        unsigned __int128 expected = (unsigned __int128)nb64 * m.num_layers * 2 * m.num_kv_heads *
                                     m.block_size * m.head_dim * flkv::dtype_bytes(m.dtype);
        if (expected != (unsigned __int128)(len - head_end)) {
            set_error("bundle payload length %zu != expected %llu", len - head_end,
                      expected >> 64 ? ~0ull : (unsigned long long)expected);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        // ---- Cache::import_prefix_bundle (cache.rs:238-340)
        const int bs = table.block_size();
        if (m.block_size != (uint64_t)bs) {
            set_error("bundle block_size %llu != cache block_size %d",
                      (unsigned long long)m.block_size, bs);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (m.num_layers != (uint64_t)num_layers) {
            set_error("bundle num_layers %llu != model %d", (unsigned long long)m.num_layers,
                      num_layers);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (m.num_kv_heads != (uint64_t)kv_heads) {
            set_error("bundle num_kv_heads %llu != model %d",
                      (unsigned long long)m.num_kv_heads, kv_heads);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (m.head_dim != (uint64_t)head_dim) {
            set_error("bundle head_dim %llu != model %d", (unsigned long long)m.head_dim,
                      head_dim);
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (m.dtype != dtype) {
            set_error("bundle dtype %s != model dtype", flkv::dtype_name(m.dtype));
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        const uint64_t tc = m.token_count;
        if (!prompt || n_prompt < 0 || (uint64_t)n_prompt < tc ||
            memcmp(prompt, m.token_ids.data(), tc * sizeof(uint32_t)) != 0) {
            set_error("prompt does not start with bundle token ids");
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        if (!device) {
            set_error("kv_cache: no device pool");
            return FLOUR_ERR_INVALID_ARGUMENT;
        }
        const int nb = (int)nb64;
        // start a clean sequence, then make sure every imported block fits
        reset_sequence();
        if (allocator.num_free() < nb) {
            set_error("not enough free kv blocks to import (%d < %d)", allocator.num_free(), nb);
            return FLOUR_ERR_OUT_OF_BLOCKS;
        }
        std::vector<int> allocated;
        allocated.reserve(nb);
        table.reserve_blocks(nb);
        auto roll_back = [&](int rc) {
            for (int id : allocated) allocator.decref(id);
            table.clear();
            table_version++;
            return rc;
        };
        for (int b = 0; b < nb; b++) {
            const int id = allocator.allocate();
            if (id < 0) {
                set_error("out of kv blocks");
                return roll_back(FLOUR_ERR_OUT_OF_BLOCKS);
            }
            allocated.push_back(id);
            table.push_block(id);
        }
        table_version++;
        int rc = upload_table(1, s);
        if (rc) return roll_back(rc);
        const size_t per = bundle_block_bytes();
        const int cb = stage_blocks(nb);
        if (cb < 0) return roll_back(FLOUR_ERR_HIP);
        for (int b0 = 0; b0 < nb; b0 += cb) {
            const int n = std::min(cb, nb - b0);
            if (check_hip(hipMemcpyAsync(d_stage, p + head_end + (size_t)b0 * per, (size_t)n * per,
                                         hipMemcpyHostToDevice, s),
                          "kv bundle: host-to-device copy"))
                return roll_back(FLOUR_ERR_HIP);
            rc = launch_kv_bundle_copy(1, d_stage, d_pool_ptrs, d_table(), b0, n, num_layers,
                                       kv_heads, block_size, head_dim, num_slots,
                                       elem_bytes(dtype), s);
            if (rc) return roll_back(rc);
        }
        if (check_hip(hipStreamSynchronize(s), "kv bundle: import")) return roll_back(FLOUR_ERR_HIP);
        table.advance((int)tc);
        // register the imported blocks like a locally computed prefix (cache.rs:323-337)
        uint64_t parent = PREFIX_SEED;
        for (int b = 0; b < nb; b++) {
            const uint32_t* chunk = m.token_ids.data() + (int64_t)b * bs;
            const uint64_t h = block_hash(parent, chunk, bs);
            if (!registry.contains(h)) {
                const int id = table.block_at(b);
                registry.insert(h, chunk, bs, id);
                allocator.incref(id);
            }
            parent = h;
        }
        *imported = (int)tc;
        return FLOUR_OK;
    }
};

}  // namespace host
}  // namespace flour

using namespace flour;
using namespace flour::host;

struct flour_block_allocator {
    BlockAllocator a;
};
struct flour_block_table {
    BlockTable t;
};
struct flour_kv_cache {
    KvCacheImpl c;
};

#define FLOUR_NEED(cond, ...)                         \
    do {                                              \
        if (!(cond)) {                                \
            set_error(__VA_ARGS__);                   \
            return FLOUR_ERR_INVALID_ARGUMENT;        \
        }                                             \
    } while (0)

// ---------------------------------------------------------------- allocator C-ABI
extern "C" int flour_block_allocator_create(int num_blocks, flour_block_allocator** out) {
    clear_error();
    FLOUR_NEED(out && num_blocks >= 0, "block_allocator: bad arguments");
    return abi_guard("block_allocator", [&]() -> int {
        *out = new flour_block_allocator{BlockAllocator(num_blocks)};
        return FLOUR_OK;
    });
}
extern "C" void flour_block_allocator_destroy(flour_block_allocator* a) { delete a; }
extern "C" int flour_block_allocator_allocate(flour_block_allocator* a) {
    clear_error();
    FLOUR_NEED(a, "block_allocator: null");
    return a->a.allocate();
}
extern "C" int flour_block_allocator_incref(flour_block_allocator* a, int id) {
    clear_error();
    FLOUR_NEED(a && a->a.valid(id), "block_allocator: unknown block %d", id);
    a->a.incref(id);
    return FLOUR_OK;
}
extern "C" int flour_block_allocator_decref(flour_block_allocator* a, int id) {
    clear_error();
    FLOUR_NEED(a && a->a.valid(id), "block_allocator: unknown block %d", id);
    FLOUR_NEED(a->a.ref_count(id) > 0, "decref of unreferenced block %d", id);
    return a->a.decref(id) ? 1 : 0;
}
extern "C" int flour_block_allocator_ref_count(const flour_block_allocator* a, int id) {
    clear_error();
    FLOUR_NEED(a && a->a.valid(id), "block_allocator: unknown block %d", id);
    return a->a.ref_count(id);
}
extern "C" int flour_block_allocator_num_free(const flour_block_allocator* a) {
    clear_error();
    FLOUR_NEED(a, "block_allocator: null");
    return a->a.num_free();
}

// ---------------------------------------------------------------- block table C-ABI
extern "C" int flour_block_table_create(int block_size, flour_block_table** out) {
    clear_error();
    FLOUR_NEED(out && block_size > 0, "block_table: bad arguments");
    return abi_guard("block_table", [&]() -> int {
        *out = new flour_block_table{BlockTable(block_size)};
        return FLOUR_OK;
    });
}
extern "C" void flour_block_table_destroy(flour_block_table* t) { delete t; }
extern "C" int flour_block_table_push_block(flour_block_table* t, int id) {
    clear_error();
    FLOUR_NEED(t && id >= 0, "block_table: bad block id %d", id);
    return abi_guard("block_table", [&]() -> int {
        t->t.push_block(id);
        return FLOUR_OK;
    });
}
extern "C" int flour_block_table_advance(flour_block_table* t, int n) {
    clear_error();
    FLOUR_NEED(t && n >= 0, "block_table: bad advance %d", n);
    t->t.advance(n);
    return FLOUR_OK;
}
extern "C" int flour_block_table_clear(flour_block_table* t) {
    clear_error();
    FLOUR_NEED(t, "block_table: null");
    t->t.clear();
    return FLOUR_OK;
}
extern "C" int flour_block_table_len(const flour_block_table* t) { return t ? t->t.len() : -1; }
extern "C" int flour_block_table_capacity(const flour_block_table* t) {
    return t ? t->t.capacity() : -1;
}
extern "C" int flour_block_table_block_size(const flour_block_table* t) {
    return t ? t->t.block_size() : -1;
}
extern "C" int flour_block_table_blocks(const flour_block_table* t, int32_t* out, int cap,
                                        int* n) {
    clear_error();
    FLOUR_NEED(t && n && (out || cap == 0), "block_table: bad arguments");
    const auto& b = t->t.blocks();
    *n = (int)b.size();
    for (int i = 0; i < (int)b.size() && i < cap; i++) out[i] = b[i];
    return FLOUR_OK;
}
extern "C" int64_t flour_block_table_slot(const flour_block_table* t, int pos) {
    clear_error();
    FLOUR_NEED(t && t->t.backed(pos), "block_table: position %d has no block", pos);
    return t->t.slot(pos);
}
extern "C" int flour_block_table_slots(const flour_block_table* t, int start, int end,
                                       int32_t* out) {
    clear_error();
    FLOUR_NEED(t && out && start >= 0 && end >= start && (end == start || t->t.backed(end - 1)),
               "block_table: slots(%d, %d) outside the mapped blocks", start, end);
    for (int p = start; p < end; p++) out[p - start] = (int32_t)t->t.slot(p);
    return FLOUR_OK;
}

// ---------------------------------------------------------------- kv cache C-ABI
extern "C" int flour_kv_cache_create(int num_layers, int max_seq_len, int num_heads,
                                     int kv_heads, int head_dim, int block_size, int dtype,
                                     int device_pool, flour_kv_cache** out) {
    clear_error();
    FLOUR_NEED(out, "kv_cache: null output");
    *out = nullptr;
    FLOUR_NEED(num_layers > 0 && max_seq_len > 0 && num_heads > 0 && kv_heads > 0 &&
                   num_heads % kv_heads == 0 && head_dim > 0 && block_size > 0 &&
                   valid_dtype(dtype),
               "kv_cache: bad shape (layers=%d max_seq_len=%d heads=%d kv_heads=%d head_dim=%d "
               "block_size=%d dtype=%d)",
               num_layers, max_seq_len, num_heads, kv_heads, head_dim, block_size, dtype);
    const int64_t slots = ((int64_t)max_seq_len + block_size - 1) / block_size * block_size;
    FLOUR_NEED(slots < (1ll << 31), "kv_cache: %lld slots exceed int32 slot ids",
               (long long)slots);
    return abi_guard("kv_cache", [&]() -> int {
        std::unique_ptr<flour_kv_cache> c(new flour_kv_cache{KvCacheImpl(
            num_layers, max_seq_len, num_heads, kv_heads, head_dim, block_size, dtype)});
        if (device_pool) {
            const int rc = c->c.alloc_device();
            if (rc != FLOUR_OK) return rc;
        }
        *out = c.release();
        return FLOUR_OK;
    });
}
extern "C" void flour_kv_cache_destroy(flour_kv_cache* c) { delete c; }

extern "C" int flour_kv_cache_allocate_kv(flour_kv_cache* c, int seq_len) {
    clear_error();
    FLOUR_NEED(c, "kv_cache: null");
    return abi_guard("kv_cache", [&] { return c->c.allocate_kv(seq_len); });
}
extern "C" int flour_kv_cache_len(const flour_kv_cache* c) { return c ? c->c.table.len() : -1; }
extern "C" int flour_kv_cache_capacity(const flour_kv_cache* c) {
    return c ? c->c.table.capacity() : -1;
}
extern "C" int flour_kv_cache_free_blocks(const flour_kv_cache* c) {
    return c ? c->c.allocator.num_free() : -1;
}
extern "C" int flour_kv_cache_ref_count(const flour_kv_cache* c, int id) {
    clear_error();
    FLOUR_NEED(c && c->c.allocator.valid(id), "kv_cache: unknown block %d", id);
    return c->c.allocator.ref_count(id);
}
extern "C" int flour_kv_cache_blocks(const flour_kv_cache* c, int32_t* out, int cap, int* n) {
    clear_error();
    FLOUR_NEED(c && n && (out || cap == 0), "kv_cache: bad arguments");
    const auto& b = c->c.table.blocks();
    *n = (int)b.size();
    for (int i = 0; i < (int)b.size() && i < cap; i++) out[i] = b[i];
    return FLOUR_OK;
}
extern "C" int flour_kv_cache_slots(const flour_kv_cache* c, int start, int end, int32_t* out) {
    clear_error();
    FLOUR_NEED(c && out && start >= 0 && end >= start &&
                   (end == start || c->c.table.backed(end - 1)),
               "kv_cache: slots(%d, %d) outside the mapped blocks", start, end);
    for (int p = start; p < end; p++) out[p - start] = (int32_t)c->c.table.slot(p);
    return FLOUR_OK;
}

extern "C" int flour_kv_cache_write_kv(flour_kv_cache* c, int layer, const void* k,
                                       const void* v, int seq_len, int64_t stride_tok,
                                       int64_t stride_head, void* stream) {
    clear_error();
    FLOUR_NEED(c, "kv_cache: null");
    KvCacheImpl& x = c->c;
    if (!x.device) {
        set_error("kv_cache: write_kv needs a device pool (created with device_pool = 0)");
        return FLOUR_ERR_UNSUPPORTED;
    }
    FLOUR_NEED(layer >= 0 && layer < x.num_layers, "kv_cache: layer %d of %d", layer,
               x.num_layers);
    FLOUR_NEED(seq_len >= 0 && seq_len <= x.table.len(),
               "kv_cache: write of %d tokens, %d are live (allocate_kv first)", seq_len,
               x.table.len());
    if (seq_len == 0) return FLOUR_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = x.staging_ready();
    if (rc) return rc;
    const int end = x.table.len(), start = end - seq_len;
    int32_t* slots = x.h_meta + x.num_blocks + 3;
    for (int p = start; p < end; p++) slots[p - start] = (int32_t)x.table.slot(p);
    rc = x.upload(x.num_blocks + 3, seq_len, s);
    if (rc) return rc;
    return flour_hip_kv_write(k, v, stride_tok, stride_head, x.k_pools[layer], x.v_pools[layer],
                              x.d_slots(), seq_len, x.kv_heads, x.head_dim, x.num_slots, x.dtype,
                              stream);
}

extern "C" int flour_kv_cache_attention(flour_kv_cache* c, int layer, const void* q,
                                        int num_heads, int seq_q, int64_t q_stride_tok,
                                        int64_t q_stride_head, void* out, int out_dtype,
                                        int64_t o_stride_tok, int64_t o_stride_head, float scale,
                                        void* stream) {
    clear_error();
    FLOUR_NEED(c, "kv_cache: null");
    KvCacheImpl& x = c->c;
    if (!x.device) {
        set_error("kv_cache: attention needs a device pool (created with device_pool = 0)");
        return FLOUR_ERR_UNSUPPORTED;
    }
    FLOUR_NEED(layer >= 0 && layer < x.num_layers, "kv_cache: layer %d of %d", layer,
               x.num_layers);
    FLOUR_NEED(num_heads > 0 && num_heads <= x.num_heads && num_heads % x.kv_heads == 0,
               "kv_cache: %d query heads (cache built for up to %d, %d kv heads)", num_heads,
               x.num_heads, x.kv_heads);
    const int len = x.table.len();
    FLOUR_NEED(seq_q >= 1 && seq_q <= len, "kv_cache: %d query rows over %d live positions",
               seq_q, len);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int rc = x.upload_table(seq_q, s);
    if (rc) return rc;
    const int max_blocks = x.num_blocks;
    if (seq_q == 1) {
        FLOUR_NEED(q_stride_head == x.head_dim && o_stride_head == x.head_dim,
                   "kv_cache: decode needs q and out as (num_heads, head_dim) contiguous");
        return flour_hip_paged_decode(out, out_dtype, q, x.k_pools[layer], x.v_pools[layer],
                                      x.d_table(), max_blocks, x.d_kv_len(), 1, num_heads,
                                      x.kv_heads, x.head_dim, x.block_size, x.num_slots, len,
                                      scale, x.dtype, x.d_ws, x.ws_bytes, stream);
    }
    return flour_hip_varlen_prefill_ws(out, out_dtype, o_stride_tok, o_stride_head, q,
                                       q_stride_tok, q_stride_head, x.k_pools[layer],
                                       x.v_pools[layer], x.d_cu(), x.d_kv_len(), x.d_table(),
                                       max_blocks, 1, seq_q, seq_q, num_heads, x.kv_heads,
                                       x.head_dim, x.block_size, x.num_slots, scale, x.dtype,
                                       x.d_pf_ws, x.pf_ws_bytes, stream);
}

extern "C" int flour_kv_cache_reset_sequence(flour_kv_cache* c) {
    clear_error();
    FLOUR_NEED(c, "kv_cache: null");
    c->c.reset_sequence();
    return FLOUR_OK;
}
extern "C" int flour_kv_cache_match_prefix(flour_kv_cache* c, const uint32_t* tokens, int n) {
    clear_error();
    FLOUR_NEED(c && n >= 0 && (tokens || n == 0), "kv_cache: bad token list");
    FLOUR_NEED(c->c.table.blocks().empty() && c->c.table.len() == 0,
               "kv_cache: match_prefix needs a freshly reset sequence");
    return abi_guard("kv_cache", [&] { return c->c.match_prefix(tokens, n); });
}
extern "C" int flour_kv_cache_register_prefix(flour_kv_cache* c, const uint32_t* tokens, int n) {
    clear_error();
    FLOUR_NEED(c && n >= 0 && (tokens || n == 0), "kv_cache: bad token list");
    return abi_guard("kv_cache", [&] { return c->c.register_prefix(tokens, n); });
}
extern "C" int flour_kv_cache_clear_prefix_cache(flour_kv_cache* c) {
    clear_error();
    FLOUR_NEED(c, "kv_cache: null");
    return abi_guard("kv_cache", [&]() -> int {
        c->c.clear_prefix_cache();
        return FLOUR_OK;
    });
}
extern "C" int flour_kv_cache_export_bundle(flour_kv_cache* c, const char* model_id,
                                            const uint32_t* token_ids, int n_ids, int token_count,
                                            void* out, size_t cap, size_t* len, void* stream) {
    clear_error();
    FLOUR_NEED(c && len, "kv_cache: bad arguments");
    return abi_guard("kv bundle export", [&] {
        return c->c.export_bundle(model_id, token_ids, n_ids, token_count, out, cap, len,
                                  static_cast<hipStream_t>(stream));
    });
}
extern "C" int flour_kv_cache_import_bundle(flour_kv_cache* c, const void* bytes, size_t len,
                                            const uint32_t* prompt_tokens, int n_prompt,
                                            int* imported, void* stream) {
    clear_error();
    FLOUR_NEED(c && imported, "kv_cache: bad arguments");
    *imported = 0;
    return abi_guard("kv bundle import", [&] {
        return c->c.import_bundle(bytes, len, prompt_tokens, n_prompt, imported,
                                  static_cast<hipStream_t>(stream));
    });
}
extern "C" int flour_kv_cache_pool(const flour_kv_cache* c, int layer, void** k_pool,
                                   void** v_pool, int64_t* num_slots) {
    clear_error();
    FLOUR_NEED(c && k_pool && v_pool && num_slots, "kv_cache: bad arguments");
    FLOUR_NEED(c->c.device, "kv_cache: no device pool");
    FLOUR_NEED(layer >= 0 && layer < c->c.num_layers, "kv_cache: layer %d of %d", layer,
               c->c.num_layers);
    *k_pool = c->c.k_pools[layer];
    *v_pool = c->c.v_pools[layer];
    *num_slots = c->c.num_slots;
    return FLOUR_OK;
}
