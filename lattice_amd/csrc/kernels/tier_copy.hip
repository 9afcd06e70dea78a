// Whole-block moves between HBM and the host swap buffer: the data path of
// eviction and restore (ref src/kcmm/tiering.rs:1207-1406 and 1476-1709, whose
// per-layer gather_kv_layer / scatter_kv_layer launches are
// src/cuda/kernels/kv_gather.cu:9-43).
//
// A block's swap slot holds its page of every region in region order
// ([K layer 0][V layer 0][K layer 1]..., ref tiering.rs:1428-1470), so one
// gather launch covers every layer of a batch of blocks: workgroup (block,
// region) streams one page into device staging laid out exactly like the
// slots, then each block's slot is one contiguous device-to-host copy into
// page-locked host memory.
// Restore runs the same steps backwards.  All work is on the null stream and
// the call returns once it has finished, as the reference's does.
#include <algorithm>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

constexpr int kTierRegions = 64;   // regions per launch
constexpr int kTierBlocks = 64;    // blocks per launch

struct TierBatch {
    uint64_t region[kTierRegions];   // region base addresses
    uint64_t page[kTierBlocks];      // page byte offset of each block (every region)
    uint32_t n_regions;              // regions in this launch
    uint32_t region0;                // index of region[0] among all regions
    uint32_t total_regions;          // regions per block in staging
};

__device__ __forceinline__ uint8_t* staged(uint8_t* staging, const TierBatch& tb, uint32_t b,
                                           uint32_t r, uint32_t block_bytes) {
    return staging + (static_cast<uint64_t>(b) * tb.total_regions + tb.region0 + r) * block_bytes;
}

__global__ __launch_bounds__(256) void tier_gather(TierBatch tb, uint8_t* staging,
                                                   uint32_t block_bytes) {
    const uint32_t b = blockIdx.x / tb.n_regions;
    const uint32_t r = blockIdx.x - b * tb.n_regions;
    const uint8_t* src = reinterpret_cast<const uint8_t*>(tb.region[r]) + tb.page[b];
    uint8_t* dst = staged(staging, tb, b, r, block_bytes);
    for (uint32_t i = threadIdx.x * 16; i < block_bytes; i += 256 * 16)
        *reinterpret_cast<u32x4*>(dst + i) = *reinterpret_cast<const u32x4*>(src + i);
}

__global__ __launch_bounds__(256) void tier_scatter(TierBatch tb, const uint8_t* staging,
                                                    uint32_t block_bytes) {
    const uint32_t b = blockIdx.x / tb.n_regions;
    const uint32_t r = blockIdx.x - b * tb.n_regions;
    const uint8_t* src = staged(const_cast<uint8_t*>(staging), tb, b, r, block_bytes);
    uint8_t* dst = reinterpret_cast<uint8_t*>(tb.region[r]) + tb.page[b];
    for (uint32_t i = threadIdx.x * 16; i < block_bytes; i += 256 * 16)
        *reinterpret_cast<u32x4*>(dst + i) = *reinterpret_cast<const u32x4*>(src + i);
}

// Launches gather (evict) or scatter (restore) for blocks [b0, b0 + nb) of
// the call, every region, in region batches.
bool launch_tier(bool gather, const std::vector<uint64_t>& regions, const uint64_t* pages,
                 size_t nb, uint8_t* staging, uint32_t block_bytes, std::string* err) {
    for (size_t r0 = 0; r0 < regions.size(); r0 += kTierRegions) {
        TierBatch tb{};
        tb.n_regions = static_cast<uint32_t>(std::min<size_t>(kTierRegions, regions.size() - r0));
        tb.region0 = static_cast<uint32_t>(r0);
        tb.total_regions = static_cast<uint32_t>(regions.size());
        for (uint32_t i = 0; i < tb.n_regions; ++i) tb.region[i] = regions[r0 + i];
        for (size_t b = 0; b < nb; ++b) tb.page[b] = pages[b];
        const dim3 grid(static_cast<uint32_t>(nb) * tb.n_regions);
        if (gather)
            hipLaunchKernelGGL(tier_gather, grid, dim3(256), 0, nullptr, tb, staging, block_bytes);
        else
            hipLaunchKernelGGL(tier_scatter, grid, dim3(256), 0, nullptr, tb, staging,
                               block_bytes);
        KCMM_HIP_CHECK(hipGetLastError(), err);
    }
    return true;
}

bool tier_move(bool evict, const std::vector<uint64_t>& regions, const uint64_t* pages,
               uint8_t* const* host, size_t n, uint32_t block_bytes, std::string* err) {
    if (n == 0) return true;
    if (block_bytes % 16 != 0) {
        *err = "page size must be a multiple of 16 bytes";
        return false;
    }
    const size_t per_block = regions.size() * static_cast<size_t>(block_bytes);
    void* ws = nullptr;
    if (!dev::stream_workspace(0, 6, std::min<size_t>(n, kTierBlocks) * per_block, &ws, false,
                               err))
        return false;
    uint8_t* staging = static_cast<uint8_t*>(ws);
    for (size_t b0 = 0; b0 < n; b0 += kTierBlocks) {
        const size_t nb = std::min<size_t>(kTierBlocks, n - b0);
        if (evict) {
            if (!launch_tier(true, regions, pages + b0, nb, staging, block_bytes, err))
                return false;
            for (size_t b = 0; b < nb; ++b)
                KCMM_HIP_CHECK(hipMemcpyAsync(host[b0 + b], staging + b * per_block, per_block,
                                              hipMemcpyDeviceToHost, nullptr),
                               err);
        } else {
            for (size_t b = 0; b < nb; ++b)
                KCMM_HIP_CHECK(hipMemcpyAsync(staging + b * per_block, host[b0 + b], per_block,
                                              hipMemcpyHostToDevice, nullptr),
                               err);
            if (!launch_tier(false, regions, pages + b0, nb, staging, block_bytes, err))
                return false;
        }
        // the staging buffer is reused by the next batch
        KCMM_HIP_CHECK(hipStreamSynchronize(nullptr), err);
    }
    return true;
}

}  // namespace

namespace dev {

bool tier_evict_copy(const std::vector<uint64_t>& regions, const uint64_t* pages,
                     uint8_t* const* host, size_t n, uint32_t block_bytes, std::string* err) {
    return tier_move(true, regions, pages, host, n, block_bytes, err);
}

bool tier_restore_copy(const std::vector<uint64_t>& regions, const uint64_t* pages,
                       uint8_t* const* host, size_t n, uint32_t block_bytes, std::string* err) {
    return tier_move(false, regions, pages, host, n, block_bytes, err);
}

bool host_pinned_alloc(size_t bytes, void** out, std::string* err) {
    *out = nullptr;
    KCMM_HIP_CHECK(hipHostMalloc(out, bytes, hipHostMallocDefault), err);
    return true;
}

void host_pinned_free(void* p) {
    if (p) (void)hipHostFree(p);
}

}  // namespace dev
}  // namespace kcmm
