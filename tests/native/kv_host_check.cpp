// Checks of the host prefix registry (flour_amd/csrc/kv_host.h) restating the reference's
// prefix.rs tests on this build's hash and registry; built and run by tests/test_kv_host.py.
// Prints "ok" and exits 0 when every check holds; names the failing check otherwise.
#include <stdio.h>

#include "kv_host.h"

using flour::host::block_hash;
using flour::host::PrefixRegistry;

static int failures = 0;
#define CHECK(cond)                                        \
    do {                                                   \
        if (!(cond)) {                                     \
            printf("FAILED: %s (line %d)\n", #cond, __LINE__); \
            failures++;                                    \
        }                                                  \
    } while (0)

int main() {
    const uint64_t seed = 0;  // the root parent of a chain
    // block_hash_is_deterministic_and_parent_sensitive (prefix.rs:64-78)
    const uint32_t toks[3] = {1, 2, 3}, other[3] = {1, 2, 4};
    CHECK(block_hash(seed, toks, 3) == block_hash(seed, toks, 3));
    CHECK(block_hash(seed, toks, 3) != block_hash(42, toks, 3));  // chaining
    CHECK(block_hash(seed, toks, 3) != block_hash(seed, other, 3));
    CHECK(block_hash(seed, toks, 2) != block_hash(seed, toks, 3));  // the length counts too
    // a chain: the hash of block 1 depends on block 0 through its parent
    const uint32_t b0a[2] = {5, 6}, b0b[2] = {5, 7}, b1[2] = {8, 9};
    CHECK(block_hash(block_hash(seed, b0a, 2), b1, 2) != block_hash(block_hash(seed, b0b, 2), b1, 2));

    // registry_get_verifies_tokens_against_collisions (prefix.rs:80-100)
    PrefixRegistry reg;
    const uint32_t t12[2] = {1, 2}, t99[2] = {9, 9}, t34[2] = {3, 4};
    const uint64_t h = block_hash(seed, t12, 2);
    reg.insert(h, t12, 2, 7);
    CHECK(reg.get(h, t12, 2) == 7);  // correct tokens at the stored hash: hit
    CHECK(reg.contains(h));
    CHECK(reg.get(h, t99, 2) == -1);  // same hash, other tokens (a simulated collision): miss
    CHECK(reg.get(h, t12, 1) == -1);  // same hash, a shorter token run: miss
    CHECK(reg.get(block_hash(seed, t34, 2), t34, 2) == -1);  // unknown hash: miss
    const std::vector<int> ids = reg.drain_block_ids();  // the registry's clear
    CHECK(ids.size() == 1 && ids[0] == 7);
    CHECK(!reg.contains(h));
    CHECK(reg.get(h, t12, 2) == -1);

    if (failures == 0) printf("ok\n");
    return failures == 0 ? 0 : 1;
}
