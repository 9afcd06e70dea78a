// Tiering bookkeeping of a KCMM pool: the eviction policies and the host
// swap-slot allocator (ref src/kcmm/tiering.rs:25-643).  Pure C++17, linked
// into libkcmm.so and into the host-only check library.
//
// Handles are physical page handles (superblock, index).  The reference
// stamps LRU / FIFO / sink-window entries with Instant::now(); here a logical
// clock ticks once per event, which gives the same order without ties.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <utility>
#include <vector>

namespace kcmm {

using PageHandle = std::pair<uint32_t, uint32_t>;

enum class PolicyKind : int { kLru = 0, kLfu = 1, kFifo = 2, kArc = 3, kSinkWindow = 4 };

// One eviction policy (ref tiering.rs:32-545).
//  * lru: last allocate/access time, oldest first (:60-106)
//  * lfu: access count (1 at allocate, +1 per access), least first (:113-162)
//  * fifo: allocate time only, earliest first (:169-216)
//  * arc: T1/T2 recency lists with B1/B2 ghosts and adaptive target p
//    (:218-430); select ranks T1 from its LRU end, then T2, then untracked
//  * sink_window: LRU among blocks outside a sequence's first / last blocks;
//    the reference pool never registers block positions (register_block is
//    only called from its tests), so it selects exactly as LRU (:432-545)
// select_victims keeps the candidates' order among equal keys (stable sort)
// and, except under arc, drops candidates the policy does not track.
class EvictionPolicy {
public:
    EvictionPolicy(PolicyKind kind, size_t arc_capacity);

    void on_allocate(PageHandle h);
    void on_access(PageHandle h);
    void on_evict(PageHandle h);
    std::vector<PageHandle> select_victims(const std::vector<PageHandle>& candidates,
                                           size_t count) const;
    PolicyKind kind() const { return kind_; }
    const char* name() const;

private:
    void arc_replace();

    PolicyKind kind_;
    uint64_t clock_ = 0;
    std::map<PageHandle, uint64_t> key_;     // time (lru/fifo/sink) or count (lfu)
    std::vector<PageHandle> t1_, t2_, b1_, b2_;   // arc; index 0 = most recent
    size_t arc_p_ = 0;
    size_t arc_cap_ = 1;
};

// Best-fit byte-range allocator of the swap buffer (ref tiering.rs:547-643):
// the smallest free range that fits, shrunk from its start; frees merge with
// both neighbours.
class SwapSlots {
public:
    explicit SwapSlots(uint64_t total = 0);
    bool allocate(uint64_t size, uint64_t* offset);
    void free(uint64_t offset, uint64_t size);
    const std::vector<std::pair<uint64_t, uint64_t>>& ranges() const { return free_; }

private:
    std::vector<std::pair<uint64_t, uint64_t>> free_;   // [start, end), sorted
};

}  // namespace kcmm
