// Whole-page copies across every layer's K and V region: the copy half of a
// copy-on-write fork (the reference's page-granular copy primitive is
// gather/scatter_kv_layer, ref src/cuda/kernels/kv_gather.cu:9-43; the fork
// itself follows vLLM's copy_blocks, ref patch_vllm.py:1083-1090).  One
// workgroup per (pair, region) streams the page with 16-byte vector copies.
#include <algorithm>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

// One launch carries up to kMaxPairs pairs for up to kMaxRegions regions in
// its kernel arguments (3.6 KB, under the 4 KB argument limit).
constexpr int kMaxRegions = 64;
constexpr int kMaxPairs = 192;

struct CopyBatch {
    uint64_t region[kMaxRegions];
    uint64_t pair[2 * kMaxPairs];  // (src, dst) byte offsets inside each region
    uint32_t n_regions;
};
static_assert(sizeof(CopyBatch) + 8 <= 4096, "page-copy kernel arguments over 4 KB");

__device__ __forceinline__ void copy_page(uint8_t* base, uint64_t src, uint64_t dst,
                                          uint32_t bytes) {
    for (uint32_t i = threadIdx.x * 16; i < bytes; i += 256 * 16)
        *reinterpret_cast<u32x4*>(base + dst + i) = *reinterpret_cast<const u32x4*>(base + src + i);
}

__global__ __launch_bounds__(256) void copy_pages_host(CopyBatch cb, uint32_t block_bytes) {
    const uint32_t pr = blockIdx.x / cb.n_regions;
    const uint32_t rg = blockIdx.x - pr * cb.n_regions;
    copy_page(reinterpret_cast<uint8_t*>(cb.region[rg]), cb.pair[2 * pr], cb.pair[2 * pr + 1],
              block_bytes);
}

// A pair naming an id outside [0, n_ids) is skipped: the offset table is
// never read past the pool's ids, and no page outside the pool is written.
__global__ __launch_bounds__(256) void copy_pages_dev(CopyBatch cb, const int64_t* pairs,
                                                      const uint64_t* offsets_f16,
                                                      uint32_t block_bytes, int64_t n_ids) {
    const uint32_t pr = blockIdx.x / cb.n_regions;
    const uint32_t rg = blockIdx.x - pr * cb.n_regions;
    const int64_t a = pairs[2 * pr], b = pairs[2 * pr + 1];
    if (a < 0 || b < 0 || a >= n_ids || b >= n_ids) return;
    const uint64_t src = offsets_f16[a] * 2ull;
    const uint64_t dst = offsets_f16[b] * 2ull;
    copy_page(reinterpret_cast<uint8_t*>(cb.region[rg]), src, dst, block_bytes);
}

}  // namespace

namespace dev {

bool copy_pages(const std::vector<uint64_t>& regions, const uint64_t* pair_offsets,
                size_t num_pairs, uint32_t block_bytes, uint64_t stream, std::string* err) {
    if (block_bytes % 16 != 0) {
        *err = "page size must be a multiple of 16 bytes";
        return false;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    for (size_t r0 = 0; r0 < regions.size(); r0 += kMaxRegions) {
        CopyBatch cb{};
        cb.n_regions = static_cast<uint32_t>(std::min<size_t>(kMaxRegions, regions.size() - r0));
        for (uint32_t i = 0; i < cb.n_regions; ++i) cb.region[i] = regions[r0 + i];
        for (size_t p0 = 0; p0 < num_pairs; p0 += kMaxPairs) {
            const size_t n = std::min<size_t>(kMaxPairs, num_pairs - p0);
            for (size_t i = 0; i < 2 * n; ++i) cb.pair[i] = pair_offsets[2 * p0 + i];
            hipLaunchKernelGGL(copy_pages_host, dim3(static_cast<unsigned>(n * cb.n_regions)),
                               dim3(256), 0, s, cb, block_bytes);
            KCMM_HIP_CHECK(hipGetLastError(), err);
        }
    }
    return true;
}

bool copy_pages_device(const std::vector<uint64_t>& regions, uint64_t pairs_ptr,
                       uint64_t offsets_f16, size_t num_pairs, uint32_t n_ids,
                       uint32_t block_bytes, uint64_t stream, std::string* err) {
    if (block_bytes % 16 != 0) {
        *err = "page size must be a multiple of 16 bytes";
        return false;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t* pairs = reinterpret_cast<const int64_t*>(pairs_ptr);
    for (size_t r0 = 0; r0 < regions.size(); r0 += kMaxRegions) {
        CopyBatch cb{};
        cb.n_regions = static_cast<uint32_t>(std::min<size_t>(kMaxRegions, regions.size() - r0));
        for (uint32_t i = 0; i < cb.n_regions; ++i) cb.region[i] = regions[r0 + i];
        const size_t grid = num_pairs * cb.n_regions;
        if (grid > 0x7fffffffULL) {
            *err = "too many page pairs for one launch";
            return false;
        }
        hipLaunchKernelGGL(copy_pages_dev, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, cb,
                           pairs, reinterpret_cast<const uint64_t*>(offsets_f16), block_bytes,
                           static_cast<int64_t>(n_ids));
        KCMM_HIP_CHECK(hipGetLastError(), err);
    }
    return true;
}

}  // namespace dev
}  // namespace kcmm
