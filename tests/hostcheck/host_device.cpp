// Device layer of the host-only check build of the KCMM runtime.
//
// libkcmm_hostcheck.so links the product's pool_core.cpp and ffi.cpp against
// this file instead of the HIP device layer, so the CPU test tier exercises
// the exact bookkeeping code that ships (block ids, page offsets, sequences,
// reference counts, error paths).  Regions get distinct fake base addresses
// and superblock mapping is only recorded; every data-path entry point fails
// with "no device" (the tiering moves, which carry no bytes here, aside), so
// nothing here can stand in for the HIP kernels.
#include <cstdint>
#include <cstdlib>
#include <memory>
#include <string>
#include <vector>

#include "../../lattice_amd/csrc/device_api.hpp"

namespace kcmm {
namespace {

class HostBacking final : public PageBacking {
public:
    bool reserve(size_t num_regions, size_t region_bytes, std::string*) override {
        n_ = num_regions;
        bytes_ = region_bytes;
        return true;
    }
    uint64_t region_base(size_t r) const override {
        return 0x100000000000ull + static_cast<uint64_t>(r) * 0x10000000000ull;
    }
    bool map_superblock(size_t sb, std::string* err) override {
        if ((sb + 1) * kSuperblockBytes > bytes_) {
            *err = "superblock beyond the reserved region";
            return false;
        }
        mapped_.push_back(sb);
        return true;
    }
    void release() override { mapped_.clear(); }
    int kind() const override { return 2; }

private:
    size_t n_ = 0, bytes_ = 0;
    std::vector<size_t> mapped_;
};

bool no_device(std::string* err) {
    *err = "no device in the host-check build";
    return false;
}

}  // namespace

namespace dev {

std::unique_ptr<PageBacking> make_backing(int, std::string*) {
    return std::unique_ptr<PageBacking>(new HostBacking());
}
bool set_device(int, std::string*) { return true; }
bool synchronize_device(int, std::string*) { return true; }
bool stream_workspace(uint64_t, int, size_t, void**, bool, std::string* err) {
    return no_device(err);
}
bool attn_decode(const AttnDecodeArgs&, std::string* err) { return no_device(err); }
bool attn_prefill(const AttnPrefillArgs&, std::string* err) { return no_device(err); }
bool kv_write_rows(const KvRowsArgs&, std::string* err) { return no_device(err); }
bool kv_write_device_slots(const KvDeviceSlotsArgs&, std::string* err) { return no_device(err); }
bool copy_pages(const std::vector<uint64_t>&, const uint64_t*, size_t, uint32_t, uint64_t,
                std::string* err) {
    return no_device(err);
}
bool copy_pages_device(const std::vector<uint64_t>&, uint64_t, uint64_t, size_t, uint32_t,
                       uint32_t, uint64_t, std::string* err) {
    return no_device(err);
}
bool gemm_bf16(uint64_t, uint64_t, uint64_t, uint32_t, uint32_t, uint32_t, uint64_t,
               std::string* err, uint64_t) {
    return no_device(err);
}
bool rmsnorm_bf16(uint64_t, uint64_t, uint64_t, uint32_t, uint32_t, float, uint64_t,
                  std::string* err) {
    return no_device(err);
}
bool rope_append_bf16(const RopeAppendArgs&, std::string* err) { return no_device(err); }
bool silu_mul_bf16(uint64_t, uint64_t, uint32_t, uint32_t, uint64_t, std::string* err) {
    return no_device(err);
}
bool gemm_bf16_rope_append(uint64_t, uint64_t, uint32_t, uint32_t, const RopeAppendArgs&,
                           std::string* err) {
    return no_device(err);
}
bool gemm_bf16_swiglu(uint64_t, uint64_t, uint64_t, uint32_t, uint32_t, uint32_t, uint64_t,
                      std::string* err) {
    return no_device(err);
}
bool gemm_bf16_tiled(uint64_t, uint64_t, uint64_t, uint32_t, uint32_t, uint32_t, uint64_t, uint64_t,
                     std::string* err) {
    return no_device(err);
}
bool gemm_split_reduce_launch(const float*, uint16_t*, const uint16_t*, int, int, uint64_t,
                              std::string* err) {
    return no_device(err);
}
// The host-check backing has no page memory (fake region addresses), so the
// tiering moves carry no bytes here: they succeed, and the CPU tier checks
// the bookkeeping around them (victims, swap slots, locations, new pages).
// The bytes are checked on the GPU (tests/test_gpu_tiering.py).
bool tier_evict_copy(const std::vector<uint64_t>&, const uint64_t*, uint8_t* const*, size_t,
                     uint32_t, std::string*) {
    return true;
}
bool tier_restore_copy(const std::vector<uint64_t>&, const uint64_t*, uint8_t* const*, size_t,
                       uint32_t, std::string*) {
    return true;
}
bool host_pinned_alloc(size_t bytes, void** out, std::string* err) {
    *out = std::malloc(bytes);
    if (*out == nullptr) {
        *err = "host allocation failed";
        return false;
    }
    return true;
}
void host_pinned_free(void* p) { std::free(p); }
bool gemm_bf16_partials(uint64_t, uint64_t, uint32_t, uint32_t, uint32_t, uint64_t, float**, int*,
                        std::string* err) {
    return no_device(err);
}
bool rope_append_from_partials(const RopeAppendArgs&, const float*, int, std::string* err) {
    return no_device(err);
}
bool residual_rmsnorm_from_partials(const float*, int, uint64_t, uint64_t, uint64_t, uint32_t,
                                    uint32_t, float, uint64_t, std::string* err) {
    return no_device(err);
}

}  // namespace dev
}  // namespace kcmm
