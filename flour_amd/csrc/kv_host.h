// kv_host.h — host-side bookkeeping shared by the cache layers (kv_cache.cpp: one sequence,
// kv_batch.cpp: many sequences over one pool): BlockAllocator and BlockTable
// (src/models/common/paged.rs:7-121) and the prefix registry (src/models/common/prefix.rs:1-60).
//
// Block hashes: a chained 64-bit hash of (parent hash, the block's token ids), so equal
// hashes identify equal full-prefix paths; as in prefix.rs the registry keeps each block's
// tokens and rejects a lookup whose tokens differ (hash collisions never return wrong KV).
// The hash function is this file's own (the reference uses Rust's DefaultHasher); only the
// identity of prefix paths matters, the values are never stored outside the process.
#pragma once

#include <stdint.h>
#include <string.h>

#include <unordered_map>
#include <vector>

namespace flour {
namespace host {

// ---------------------------------------------------------------- BlockAllocator
class BlockAllocator {
  public:
    explicit BlockAllocator(int n) : refs_(n, 0) {
        free_.reserve(n);
        for (int i = n - 1; i >= 0; i--) free_.push_back(i);  // first allocate returns 0
    }
    int allocate() {
        if (free_.empty()) return -1;
        const int id = free_.back();
        free_.pop_back();
        refs_[id] = 1;
        return id;
    }
    bool valid(int id) const { return id >= 0 && id < (int)refs_.size(); }
    void incref(int id) { refs_[id]++; }
    // true when the block reached zero references and returned to the free list
    bool decref(int id) {
        if (--refs_[id] == 0) {
            free_.push_back(id);
            return true;
        }
        return false;
    }
    int ref_count(int id) const { return refs_[id]; }
    int num_free() const { return (int)free_.size(); }
    int num_blocks() const { return (int)refs_.size(); }

  private:
    std::vector<int> free_;
    std::vector<int> refs_;
};

// ---------------------------------------------------------------- BlockTable
class BlockTable {
  public:
    explicit BlockTable(int bs) : bs_(bs) {}
    int len() const { return len_; }
    int block_size() const { return bs_; }
    int capacity() const { return (int)blocks_.size() * bs_; }
    void push_block(int id) { blocks_.push_back(id); }
    // room for n blocks in all, so that the pushes up to n cannot fail (callers reserve
    // before they take references, so a failed allocation changes no reference count)
    void reserve_blocks(int64_t n) { blocks_.reserve((size_t)n); }
    const std::vector<int>& blocks() const { return blocks_; }
    int block_at(int i) const { return blocks_[i]; }
    void clear() {
        blocks_.clear();
        len_ = 0;
    }
    void advance(int n) { len_ += n; }
    int64_t slot(int pos) const { return (int64_t)blocks_[pos / bs_] * bs_ + pos % bs_; }
    bool backed(int pos) const { return pos >= 0 && pos / bs_ < (int)blocks_.size(); }

  private:
    std::vector<int> blocks_;
    int bs_;
    int len_ = 0;
};

// ---------------------------------------------------------------- prefix registry
static constexpr uint64_t PREFIX_SEED = 0;

static inline uint64_t mix64(uint64_t z) {  // splitmix64 finaliser
    z ^= z >> 30;
    z *= 0xbf58476d1ce4e5b9ull;
    z ^= z >> 27;
    z *= 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Chained block hash: identifies the full prefix path ending with this block.
static uint64_t block_hash(uint64_t parent, const uint32_t* tok, int n) {
    uint64_t h = mix64(parent ^ 0x9e3779b97f4a7c15ull) ^ (uint64_t)n;
    for (int i = 0; i < n; i++) h = mix64(h ^ ((uint64_t)tok[i] + 0x632be59bd9b4e019ull));
    return h;
}

struct RegistryEntry {
    std::vector<uint32_t> tokens;
    int block_id;
};

class PrefixRegistry {
  public:
    // block id stored under `h`, only when its tokens equal `tok` (collisions are misses)
    int get(uint64_t h, const uint32_t* tok, int n) const {
        auto it = map_.find(h);
        if (it == map_.end() || (int)it->second.tokens.size() != n ||
            memcmp(it->second.tokens.data(), tok, n * sizeof(uint32_t)) != 0)
            return -1;
        return it->second.block_id;
    }
    bool contains(uint64_t h) const { return map_.count(h) != 0; }
    void insert(uint64_t h, const uint32_t* tok, int n, int id) {
        map_[h] = RegistryEntry{std::vector<uint32_t>(tok, tok + n), id};
    }
    std::vector<int> drain_block_ids() {
        std::vector<int> ids;
        ids.reserve(map_.size());
        for (auto& kv : map_) ids.push_back(kv.second.block_id);
        map_.clear();
        return ids;
    }

  private:
    std::unordered_map<uint64_t, RegistryEntry> map_;
};

}  // namespace host
}  // namespace flour
