// kv_bundle.h — internal interface between the cache layer (kv_cache.cpp) and the FLKV bundle
// copy kernels (kv_bundle.hip). Not part of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace flour {

// Gather (unpack == 0) or scatter (unpack != 0) the whole (head, block) runs of logical blocks
// [first_block, first_block + num_blocks) between the pools and `stage`, in the FLKV payload
// order: block, layer, K then V, head. d_pools holds the device addresses of the K pools of all
// layers followed by those of the V pools; d_block_ids the physical block of each logical
// block. Element size es bytes.
int launch_kv_bundle_copy(int unpack, void* stage, void* const* d_pools, const int32_t* d_block_ids,
                          int first_block, int num_blocks, int num_layers, int kv_heads,
                          int block_size, int head_dim, int64_t num_slots, int es,
                          hipStream_t stream);

}  // namespace flour
