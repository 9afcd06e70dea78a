// Grow-on-demand page backing over a virtual-memory API (the reference's
// CUDA-VMM design, ref src/cache/cuda_vmm.rs:6-234 with the per-superblock
// mapping of ref pool.rs:211-221,287-322): one virtual-address reservation
// for the whole pool, carved into its regions (region r at base + r *
// region_bytes; the reference reserves one range per region), requested
// with alignment 0 as the reference does (ref cuda_vmm.rs:63-69); at growth
// one 2 MiB physical chunk is created and mapped at byte sb * 2 MiB of every
// region.  Region offsets, block ids and page offsets do not depend on where
// the range lies.
//
// The bookkeeping is written once over an `Ops` type that issues the driver
// calls, so that the HIP build (Ops = HIP VMM calls) and the host-check build
// (Ops = a recording mock with fault injection) run the same code:
//   bool granularity(size_t* g, std::string* err);
//   bool reserve(size_t bytes, size_t align, void** va, std::string* err);
//   bool create(size_t bytes, Handle* h, std::string* err);
//   bool map(void* at, size_t bytes, Handle h, std::string* err);
//   bool set_access(void* at, size_t bytes, std::string* err);
//   void unmap(void* at, size_t bytes);
//   void release(Handle h);
//   void free_va(void* va, size_t bytes);
// A superblock is mapped in every region or in none: a failure partway
// unmaps and releases what that superblock had mapped, so the pool's
// superblock count stays right and a later growth maps the same range again.
#pragma once

#include <cstddef>
#include <string>
#include <utility>
#include <vector>

#include "pool_core.hpp"

namespace kcmm {

template <class Ops>
class VmmBacking final : public PageBacking {
public:
    using Handle = typename Ops::Handle;

    explicit VmmBacking(Ops ops) : ops_(std::move(ops)) {}
    ~VmmBacking() override { release(); }

    bool reserve(size_t num_regions, size_t region_bytes, std::string* err) override {
        size_t gran = 0;
        if (!ops_.granularity(&gran, err)) return false;
        if (gran == 0 || kSuperblockBytes % gran != 0) {
            *err = "VMM granularity does not divide the 2 MiB superblock";
            return false;
        }
        if (region_bytes % gran != 0 || num_regions == 0) {
            *err = "VMM region size is not a multiple of the granularity";
            return false;
        }
        region_bytes_ = region_bytes;
        va_bytes_ = num_regions * region_bytes;
        void* va = nullptr;
        if (!ops_.reserve(va_bytes_, 0, &va, err)) {
            va_bytes_ = 0;
            return false;
        }
        va_ = va;
        for (size_t r = 0; r < num_regions; ++r)
            bases_.push_back(static_cast<char*>(va) + r * region_bytes);
        return true;
    }

    uint64_t region_base(size_t r) const override {
        return reinterpret_cast<uint64_t>(bases_[r]);
    }

    bool map_superblock(size_t sb, std::string* err) override {
        if ((sb + 1) * kSuperblockBytes > region_bytes_) {
            *err = "superblock beyond the reserved region";
            return false;
        }
        const size_t first = mapped_.size();
        for (void* base : bases_) {
            char* at = static_cast<char*>(base) + sb * kSuperblockBytes;
            Handle h{};
            if (!ops_.create(kSuperblockBytes, &h, err)) return rollback(first);
            if (!ops_.map(at, kSuperblockBytes, h, err)) {
                ops_.release(h);
                return rollback(first);
            }
            mapped_.push_back({at, h});
            if (!ops_.set_access(at, kSuperblockBytes, err)) return rollback(first);
        }
        return true;
    }

    // Unmap, then release the physical chunks, then free the reservation.
    void release() override {
        rollback(0);
        if (va_ != nullptr) ops_.free_va(va_, va_bytes_);
        va_ = nullptr;
        va_bytes_ = 0;
        bases_.clear();
    }

    int kind() const override { return 0; }

    const Ops& ops() const { return ops_; }

private:
    // Undo the mappings from index `first` on (newest first); returns false.
    bool rollback(size_t first) {
        while (mapped_.size() > first) {
            ops_.unmap(mapped_.back().first, kSuperblockBytes);
            ops_.release(mapped_.back().second);
            mapped_.pop_back();
        }
        return false;
    }

    Ops ops_;
    size_t region_bytes_ = 0;
    void* va_ = nullptr;        // the pool's one reservation
    size_t va_bytes_ = 0;
    std::vector<void*> bases_;
    std::vector<std::pair<void*, Handle>> mapped_;
};

}  // namespace kcmm
