// kv_bundle.hip — device side of the FLKV bundle export / import over the device pool.
//
// The reference exports a block-aligned prefix of the live sequence as a KvBundle
// (Cache::export_prefix_bundle, src/models/common/cache.rs:166-229) whose payload
// (src/kv_cache/bundle.rs:15-22, written by KvBundleCodec::encode :108-143) is, logical block
// by logical block, for every layer, the K block then the V block, each (kv_heads, block_size,
// head_dim) in the pool's element type; import (cache.rs:238-340) writes each block back into a
// freshly allocated physical block (PagedKvPool::write_block). In the pool (kv_heads, num_slots,
// head_dim) one (head, block) is a contiguous run of block_size * head_dim elements, so the
// payload is a sequence of such runs: this file gathers them into a staging buffer for one
// device-to-host copy (pack) or scatters a staged payload back into the pools (unpack).
//
// One workgroup per run (block_size * head_dim elements, 4 KB at 16 x 128 bf16), 16-byte
// vectors when the run and the pool rows allow them. HBM-bound byte copy; bit-exact.
#include "flour_common.h"
#include "kv_bundle.h"

namespace flour {

template <typename VecT>
__global__ __launch_bounds__(256) void kv_bundle_copy_kernel(
    char* __restrict__ stage, void* const* __restrict__ pools, const int32_t* __restrict__ block_ids,
    int first_block, int num_layers, int kv_heads, int64_t run_bytes, int64_t head_bytes,
    int64_t block_bytes, int unpack) {
    // run r = ((block * num_layers + layer) * 2 + kv) * kv_heads + head, in payload order
    const int64_t r = blockIdx.x;
    const int g = (int)(r % kv_heads);
    const int64_t rk = r / kv_heads;
    const int kv = (int)(rk % 2);
    const int64_t rl = rk / 2;
    const int layer = (int)(rl % num_layers);
    const int b = (int)(rl / num_layers);
    const int64_t phys = block_ids[first_block + b];
    char* pool = static_cast<char*>(pools[kv * num_layers + layer]);
    char* p = pool + (int64_t)g * head_bytes + phys * block_bytes;
    char* s = stage + r * run_bytes;
    const int64_t n = run_bytes / (int64_t)sizeof(VecT);
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        if (unpack)
            reinterpret_cast<VecT*>(p)[i] = reinterpret_cast<const VecT*>(s)[i];
        else
            reinterpret_cast<VecT*>(s)[i] = reinterpret_cast<const VecT*>(p)[i];
    }
}

int launch_kv_bundle_copy(int unpack, void* stage, void* const* d_pools, const int32_t* d_block_ids,
                          int first_block, int num_blocks, int num_layers, int kv_heads,
                          int block_size, int head_dim, int64_t num_slots, int es,
                          hipStream_t stream) {
    if (num_blocks <= 0) return FLOUR_OK;
    const int64_t run_bytes = (int64_t)block_size * head_dim * es;
    const int64_t head_bytes = num_slots * head_dim * es;
    const int64_t block_bytes = run_bytes;  // a physical block's run inside one head's rows
    const int64_t runs = (int64_t)num_blocks * num_layers * 2 * kv_heads;
    if (runs > 0x7fffffff) {
        set_error("kv bundle: %lld runs exceed one launch", (long long)runs);
        return FLOUR_ERR_INVALID_ARGUMENT;
    }
    // staging and pools are allocation bases (256-byte aligned); the run length and the head
    // pitch decide the vector width
    const uint64_t align = (uint64_t)run_bytes | (uint64_t)head_bytes;
    const dim3 grid((unsigned)runs), block(256);
    char* st = static_cast<char*>(stage);
    if ((align & 15) == 0)
        kv_bundle_copy_kernel<u32x4><<<grid, block, 0, stream>>>(
            st, d_pools, d_block_ids, first_block, num_layers, kv_heads, run_bytes, head_bytes,
            block_bytes, unpack);
    else if ((align & 3) == 0)
        kv_bundle_copy_kernel<uint32_t><<<grid, block, 0, stream>>>(
            st, d_pools, d_block_ids, first_block, num_layers, kv_heads, run_bytes, head_bytes,
            block_bytes, unpack);
    else
        kv_bundle_copy_kernel<uint16_t><<<grid, block, 0, stream>>>(
            st, d_pools, d_block_ids, first_block, num_layers, kv_heads, run_bytes, head_bytes,
            block_bytes, unpack);
    return check_hip(hipGetLastError(), unpack ? "kv bundle unpack launch" : "kv bundle pack launch");
}

}  // namespace flour
