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
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../lattice_amd/csrc/device_api.hpp"
#include "../../lattice_amd/csrc/vmm_backing.hpp"

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

// Recording stand-in for the HIP VMM calls (KCMM_BACKING=vmm in this build
// only): fake addresses, live-resource counts, one injected failure
// (operation, n-th call) at a time, and every call checked against the
// preconditions the VMM API documents (CUDA's cuMem* and HIP's hipMem*
// pages); a call that breaks one counts a violation:
//  * sizes, addresses and alignments are multiples of the allocation
//    granularity (the mock's minimum granularity is 64 KiB, below the 2 MiB
//    superblock, and a reservation with alignment 0 comes back aligned to
//    that granularity only, not to 2 MiB);
//  * a mapping lies inside one live reservation, overlaps no other mapping,
//    and maps a live handle that no other mapping uses;
//  * access is set on a range inside one live mapping;
//  * an unmap names exactly one mapping (its address and size);
//  * a handle is released once, when it is no longer mapped;
//  * a reservation is freed with exactly its base and size, with nothing
//    mapped inside it.
struct VmmMock {
    static constexpr uint64_t kGran = 64 * 1024;
    std::mutex mu;
    int64_t reservations = 0, handles = 0, mappings = 0, violations = 0;
    int64_t calls[5] = {0, 0, 0, 0, 0};   // reserve, create, map, set_access, granularity
    int fail_op = -1;
    int64_t fail_at = -1;
    uint64_t next_va = 0x200000000000ull + kGran, next_handle = 0;
    struct Mapping {
        uint64_t bytes, handle;
    };
    std::map<uint64_t, Mapping> mapped;           // address -> mapping
    std::map<uint64_t, uint64_t> reserved;        // base -> bytes
    std::map<uint64_t, uint64_t> live_handles;    // handle -> bytes
    bool fail(int op) { return ++calls[op] == fail_at && op == fail_op; }
    void check(bool ok) { if (!ok) ++violations; }
    bool in_one_reservation(uint64_t a, uint64_t n) const {
        auto it = reserved.upper_bound(a);
        if (it == reserved.begin()) return false;
        --it;
        return a >= it->first && a + n <= it->first + it->second;
    }
    bool overlaps_mapping(uint64_t a, uint64_t n) const {
        for (const auto& m : mapped)
            if (a < m.first + m.second.bytes && m.first < a + n) return true;
        return false;
    }
} g_vmm;

struct MockVmmOps {
    using Handle = uint64_t;
    bool granularity(size_t* g, std::string* err) {
        std::lock_guard<std::mutex> lk(g_vmm.mu);
        if (g_vmm.fail(4)) { *err = "mock: granularity failed"; return false; }
        *g = VmmMock::kGran;
        return true;
    }
    bool reserve(size_t bytes, size_t align, void** va, std::string* err) {
        std::lock_guard<std::mutex> lk(g_vmm.mu);
        if (g_vmm.fail(0)) { *err = "mock: reserve failed"; return false; }
        g_vmm.check(bytes > 0 && bytes % VmmMock::kGran == 0);
        g_vmm.check(align == 0 || (align % VmmMock::kGran == 0 && (align & (align - 1)) == 0));
        uint64_t base = g_vmm.next_va;
        if (align != 0) base = (base + align - 1) / align * align;
        *va = reinterpret_cast<void*>(base);
        g_vmm.reserved[base] = bytes;
        // the next reservation starts one granule past a 2 MiB boundary
        g_vmm.next_va = (base + bytes + kSuperblockBytes) / kSuperblockBytes * kSuperblockBytes +
                        VmmMock::kGran;
        ++g_vmm.reservations;
        return true;
    }
    bool create(size_t bytes, Handle* h, std::string* err) {
        std::lock_guard<std::mutex> lk(g_vmm.mu);
        if (g_vmm.fail(1)) { *err = "mock: create failed"; return false; }
        g_vmm.check(bytes > 0 && bytes % VmmMock::kGran == 0);
        *h = ++g_vmm.next_handle;
        g_vmm.live_handles[*h] = bytes;
        ++g_vmm.handles;
        return true;
    }
    bool map(void* at, size_t bytes, Handle h, std::string* err) {
        std::lock_guard<std::mutex> lk(g_vmm.mu);
        if (g_vmm.fail(2)) { *err = "mock: map failed"; return false; }
        const uint64_t a = reinterpret_cast<uint64_t>(at);
        g_vmm.check(a % VmmMock::kGran == 0 && bytes % VmmMock::kGran == 0);
        g_vmm.check(g_vmm.in_one_reservation(a, bytes));
        g_vmm.check(!g_vmm.overlaps_mapping(a, bytes));
        auto hs = g_vmm.live_handles.find(h);
        g_vmm.check(hs != g_vmm.live_handles.end() && hs->second == bytes);
        for (const auto& m : g_vmm.mapped) g_vmm.check(m.second.handle != h);
        g_vmm.mapped[a] = VmmMock::Mapping{bytes, h};
        ++g_vmm.mappings;
        return true;
    }
    bool set_access(void* at, size_t bytes, std::string* err) {
        std::lock_guard<std::mutex> lk(g_vmm.mu);
        if (g_vmm.fail(3)) { *err = "mock: set_access failed"; return false; }
        const uint64_t a = reinterpret_cast<uint64_t>(at);
        bool inside = false;
        for (const auto& m : g_vmm.mapped)
            inside |= a >= m.first && a + bytes <= m.first + m.second.bytes;
        g_vmm.check(inside && bytes > 0 && bytes % VmmMock::kGran == 0);
        return true;
    }
    void unmap(void* at, size_t bytes) {
        std::lock_guard<std::mutex> lk(g_vmm.mu);
        auto it = g_vmm.mapped.find(reinterpret_cast<uint64_t>(at));
        if (it == g_vmm.mapped.end() || it->second.bytes != bytes) {
            ++g_vmm.violations;
            return;
        }
        g_vmm.mapped.erase(it);
        --g_vmm.mappings;
    }
    void release(Handle h) {
        std::lock_guard<std::mutex> lk(g_vmm.mu);
        for (const auto& m : g_vmm.mapped) g_vmm.check(m.second.handle != h);   // still mapped
        if (g_vmm.live_handles.erase(h) == 0) {
            ++g_vmm.violations;
            return;
        }
        --g_vmm.handles;
    }
    void free_va(void* va, size_t bytes) {
        std::lock_guard<std::mutex> lk(g_vmm.mu);
        const uint64_t a = reinterpret_cast<uint64_t>(va);
        auto it = g_vmm.reserved.find(a);
        if (it == g_vmm.reserved.end() || it->second != bytes) {
            ++g_vmm.violations;
            return;
        }
        g_vmm.check(!g_vmm.overlaps_mapping(a, bytes));
        g_vmm.reserved.erase(it);
        --g_vmm.reservations;
    }
};

bool no_device(std::string* err) {
    *err = "no device in the host-check build";
    return false;
}

}  // namespace

namespace dev {

std::unique_ptr<PageBacking> make_backing(int, std::string*) {
    const char* env = std::getenv("KCMM_BACKING");
    if (env != nullptr && std::strcmp(env, "vmm") == 0)
        return std::unique_ptr<PageBacking>(new VmmBacking<MockVmmOps>(MockVmmOps()));
    return std::unique_ptr<PageBacking>(new HostBacking());
}
bool set_device(int, std::string*) { return true; }
bool synchronize_device(int, std::string*) { return true; }
bool stream_workspace(uint64_t, int, size_t, void**, bool, std::string* err) {
    return no_device(err);
}
bool release_orphaned_workspaces(std::string*) { return true; }
size_t orphaned_workspaces() { return 0; }
bool attn_decode(const AttnDecodeArgs&, std::string* err) { return no_device(err); }
bool attn_stream_timing_start(uint32_t, std::string* err) { return no_device(err); }
bool attn_stream_timing_stop(double*, uint32_t*, std::string* err) { return no_device(err); }
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
bool embed_bf16(uint64_t, uint64_t, uint64_t, uint32_t, uint32_t, uint32_t, uint64_t,
                std::string* err) {
    return no_device(err);
}
bool silu_mul_bf16(uint64_t, uint64_t, uint32_t, uint32_t, uint64_t, std::string* err) {
    return no_device(err);
}
bool gemm_bf16_rope_append(uint64_t, uint64_t, uint32_t, uint32_t, const RopeAppendArgs&,
                           std::string* err, uint64_t) {
    return no_device(err);
}
bool gemm_bf16_swiglu(uint64_t, uint64_t, uint64_t, uint32_t, uint32_t, uint32_t, uint64_t,
                      std::string* err, uint64_t) {
    return no_device(err);
}
bool gemm_bf16_tiled(uint64_t, uint64_t, uint64_t, uint32_t, uint32_t, uint32_t, uint64_t, uint64_t,
                     std::string* err) {
    return no_device(err);
}
bool gemm_fp8w_bf16(uint64_t, uint64_t, uint64_t, uint64_t, uint32_t, uint32_t, uint32_t, uint64_t,
                    std::string* err, uint64_t) {
    return no_device(err);
}
bool gemm_split_reduce_launch(const float*, uint16_t*, const uint16_t*, int, int, uint64_t,
                              std::string* err) {
    return no_device(err);
}
void gemm_tiled_plan(uint32_t, uint32_t, uint32_t, int* splits, int* tile) {
    *splits = 1;
    *tile = -1;
}
bool gemm_plan(uint32_t, uint32_t, uint32_t, bool, GemmPlan*, std::string* err) {
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
                        std::string* err, uint64_t) {
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

// Test hooks of the mock VMM (host-check build only): reset the counters and
// arm one failure (op 0 reserve, 1 create, 2 map, 3 set_access, 4
// granularity; at = 1-based call index, -1 none); read reservations,
// handles, mappings, violations.
extern "C" void kcmm_hostcheck_vmm_reset(int fail_op, int64_t fail_at) {
    std::lock_guard<std::mutex> lk(kcmm::g_vmm.mu);
    std::memset(kcmm::g_vmm.calls, 0, sizeof(kcmm::g_vmm.calls));
    kcmm::g_vmm.violations = 0;
    kcmm::g_vmm.fail_op = fail_op;
    kcmm::g_vmm.fail_at = fail_at;
}
extern "C" void kcmm_hostcheck_vmm_state(int64_t* out) {
    std::lock_guard<std::mutex> lk(kcmm::g_vmm.mu);
    out[0] = kcmm::g_vmm.reservations;
    out[1] = kcmm::g_vmm.handles;
    out[2] = kcmm::g_vmm.mappings;
    out[3] = kcmm::g_vmm.violations;
}
