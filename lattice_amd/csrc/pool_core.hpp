// Host bookkeeping of a KCMM pool: the 2 MiB superblock page allocator, the
// logical block-id table, sequences and their block tables, reference counts
// for copy-on-write sharing.  Pure C++17 -- no HIP types -- so the exact same
// code is linked into libkcmm.so and into the host-only check library the CPU
// tests load.  Device memory is reached only through PageBacking.
//
// Allocation rules restated from the reference (all must hold bit-exactly):
//   block_bytes        = kv_heads*block_size*head_dim*elem  (ref pool.rs:203-204)
//   blocks/superblock  = floor(2 MiB / block_bytes), tail is padding
//                                                        (ref superblock.rs:55-70,139-141)
//   new superblock     pushes handles 0..bps-1, allocation pops (LIFO)
//                                                        (ref superblock.rs:95-116)
//   growth             only when the free list is empty; capacity
//                      ceil(max_blocks_total/bps)*bps    (ref pool.rs:323-337,1145-1152)
//   superblock s       mapped at byte s*2MiB of every layer's K and V region
//                                                        (ref pool.rs:287-322)
//   block id           LIFO pop of recycled ids, else len(block_info)
//                                                        (ref pool.rs:412-454)
//   va offset          s*2MiB + index*block_bytes        (ref pool.rs:404-407)
//   free order         handles and ids returned in table order
//                                                        (ref pool.rs:478-549)
//   sequence ids       len(sequences), never reused      (ref pool.rs:551-572)
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <deque>
#include <vector>

#include "tiering.hpp"

namespace kcmm {

constexpr size_t kSuperblockBytes = 2u * 1024u * 1024u;

enum KvDtype : int32_t { kF16 = 0, kBF16 = 1, kFP8 = 2, kF32 = 3 };

// Maps 2 MiB superblocks into 2*num_layers device VA regions (layer l: K at
// region 2l, V at region 2l+1).  Implemented over HIP VMM / hipMalloc in the
// product library and over host memory in the CPU check library.
class PageBacking {
public:
    virtual ~PageBacking() = default;
    virtual bool reserve(size_t num_regions, size_t region_bytes, std::string* err) = 0;
    virtual uint64_t region_base(size_t region) const = 0;
    virtual bool map_superblock(size_t sb_idx, std::string* err) = 0;
    virtual void release() = 0;
    virtual int kind() const = 0;
};

struct PoolGeometry {
    size_t block_size = 16;
    size_t num_layers = 0;
    size_t kv_heads = 0;
    size_t head_dim = 0;
    size_t max_batch = 0;
    size_t max_seq_len = 0;
    int32_t dtype = kF16;

    size_t elem_bytes = 2;          // bytes per K/V element
    size_t row_bytes = 0;           // one token row of a page: kv_heads*head_dim*elem
    size_t data_bytes = 0;          // block_size*row_bytes
    size_t block_bytes = 0;         // data_bytes (+ fp8 scale footer, 256-B padded)
    size_t blocks_per_superblock = 0;
    size_t max_blocks_per_seq = 0;
    size_t max_blocks_total = 0;
    size_t max_physical_blocks = 0; // ceil(max_blocks_total/bps)*bps
    size_t region_bytes = 0;        // VA reserved per region

    // Returns false with a message when the shape cannot form a pool.
    bool compute(std::string* err);
};

// Where a block's data is (kcmm.h kcmm_block_location_t, ref pool.rs:30-45).
enum BlockLoc : int { kLocGpu = 0, kLocCpu = 1, kLocEvicting = 3, kLocRestoring = 4 };

struct BlockInfo {
    uint64_t va_offset = 0;
    uint32_t superblock_idx = 0;
    uint32_t block_index = 0;
    bool in_use = false;
    int location = kLocGpu;
    uint64_t cpu_offset = 0;   // swap offset while kLocCpu / kLocEvicting
};

// One block moving between HBM and the host swap buffer: its page offset in
// every region (the old one when evicting, the new one when restoring) and
// its swap offset.
struct TierMove {
    uint32_t block;
    uint64_t va_offset;
    uint64_t cpu_offset;
};

struct SequenceState {
    // The block table: with base >= 0 it is the shared base's ids followed by
    // `table`, else `table` alone.
    std::vector<uint32_t> table;
    int32_t base = -1;
    uint32_t seq_len = 0;
    bool active = true;
    int priority = 2;  // Evictable 0, Low 1, Normal 2, High 3 (ref pool.rs:69-86)
};

struct Stats {
    uint32_t blocks_in_use, total_blocks, total_physical_blocks, free_physical_blocks;
    uint32_t active_sequences, num_layers, blocks_per_superblock, superblock_count;
    uint32_t block_size, max_blocks_per_seq, block_bytes;
    float physical_idle_ratio;
};

struct Metrics {
    float ifr, pme, bu, rfi;
    uint64_t gpu_blocks;
};

// One destination row of a KV write, resolved on the host.
struct RowDst {
    uint32_t src_row;      // row of the [batch][row] source
    uint64_t page_offset;  // byte offset of the page inside each region
    uint32_t slot;         // token offset inside the page
};

// Chained content hashes of the full blocks of a token sequence (the keys of
// the prefix cache): hash i covers tokens [0, (i+1) * block_size) through
// hash i-1.  Writes min(n_tokens / block_size, max_out) hashes, returns that.
size_t prefix_hash_blocks(const int32_t* tokens, size_t n_tokens, size_t block_size,
                          uint64_t seed, uint64_t* out, size_t max_out);

class PoolCore {
public:
    PoolCore(const PoolGeometry& g, std::unique_ptr<PageBacking> backing);
    ~PoolCore();

    const PoolGeometry& geo() const { return geo_; }
    uint64_t va_k(size_t layer) const { return backing_->region_base(2 * layer); }
    uint64_t va_v(size_t layer) const { return backing_->region_base(2 * layer + 1); }
    int backing_kind() const { return backing_->kind(); }

    // Allocation (ref pool.rs:456-476).  On failure nothing stays allocated.
    bool alloc_blocks(uint32_t n, uint32_t* out, std::string* err);
    // Decrement and release at zero, in table order (ref pool.rs:478-549).
    void free_blocks(const uint32_t* ids, size_t n);

    uint32_t register_sequence(const uint32_t* table, size_t n);
    void unregister_sequence(uint32_t seq);
    void touch(uint32_t seq);
    void cool(uint32_t seq);
    void set_priority(uint32_t seq, int prio);
    bool has_sequence(uint32_t seq);
    void update_seq_len(uint32_t seq, uint32_t len);
    uint32_t get_seq_len(uint32_t seq);
    bool append_block_to_sequence(uint32_t seq, uint32_t block);
    bool get_block_table(uint32_t seq, std::vector<uint32_t>* out);

    bool block_va_offset(uint32_t block, uint64_t* out);  // false if not in use
    std::vector<uint64_t> all_offsets_f16();
    std::vector<uint8_t> all_valid_flags();
    bool table_va_offsets(uint32_t seq, std::vector<uint64_t>* out);
    uint32_t refcount(uint32_t block);

    // Copy-on-write support.
    bool fork_sequence(uint32_t src, uint32_t* out_seq, std::string* err);
    bool share_prefix(uint32_t src, uint32_t dst, uint32_t n, uint32_t* out, std::string* err);

    // Prefix cache: the reference's SharingManager contract (content hash ->
    // the blocks of a prefix, with a reference held for sharing; ref
    // src/kcmm/sharing.rs:9-65, a placeholder there).  Keys are the chained
    // per-block content hashes of prefix_hash_blocks; every entry holds one
    // reference on its block, so a cached prefix outlives the sequence that
    // registered it.
    // Cache the first n blocks of seq under hashes[0..n) (full blocks only:
    // n * block_size <= seq_len).  Existing keys are left as they are; each
    // new entry takes a reference.  *added = entries created.
    bool prefix_register(uint32_t seq, const uint64_t* hashes, uint32_t n, uint32_t* added,
                         std::string* err);
    // Longest cached run hashes[0..m) -> blocks[0..m); marks those entries as
    // used now.  Returns m.
    uint32_t prefix_match(const uint64_t* hashes, uint32_t n, uint32_t* blocks);
    // prefix_match, then append the m blocks to dst's table, one reference
    // each (as share_prefix).  blocks may be null.
    bool prefix_attach(uint32_t dst, const uint64_t* hashes, uint32_t n, uint32_t* blocks,
                       uint32_t* matched, std::string* err);
    // Drop up to n entries, least recently used first (the deepest first
    // among entries used together), releasing their references.  Returns
    // the number dropped.
    uint32_t prefix_evict(uint32_t n);
    uint32_t prefix_entries();
    int cow_block_for_append(uint32_t seq, uint32_t logical, uint32_t* src, uint32_t* dst,
                             std::string* err);
    // Beam fork of a decode step: for each parent, width - 1 children, each
    // forked and then made private at the page of its next token (logical
    // block seq_len / block_size, when allocated).  Appends the (src, dst)
    // page copies to *pairs and the children (parent-major) to children.
    // All or nothing: parents, pages and capacity are checked before any
    // state changes, so a failed call leaves the pool as it was.
    bool fork_beams(const uint32_t* parents, uint32_t n, uint32_t width, uint32_t* children,
                    std::vector<uint32_t>* pairs, std::string* err);
    // Byte offsets of the pages of (src, dst) pairs; false if an id is not in use.
    bool resolve_pairs(const uint32_t* pairs, size_t n, std::vector<uint64_t>* out,
                       std::string* err);

    // KV-write destination resolution (ref ffi.rs:1088-1200, 1217-1383).  Every
    // row is validated before anything is returned (no partial writes).
    bool resolve_positions(const uint32_t* seqs, const uint32_t* pos, uint32_t batch,
                           std::vector<RowDst>* out, std::string* err);
    bool resolve_slots(const int64_t* slots, uint32_t batch, std::vector<RowDst>* out,
                       std::string* err);

    // ---- tiering (ref tiering.rs, pool.rs:824-1002, ffi.rs:1900-2008) ----
    // Policy 0 lru, 1 lfu, 2 fifo (anything else lru, ref ffi.rs:425-432);
    // the swap buffer holds max_blocks blocks of every layer's K and V.
    void enable_tiering(int policy, size_t max_blocks, size_t max_batch_blocks);
    bool tiering_enabled();
    bool set_eviction_policy(const std::string& name);   // lru lfu fifo arc sink_window
    std::string eviction_policy_name();
    uint64_t swap_bytes() const { return swap_bytes_; }
    uint64_t block_swap_bytes() const { return block_swap_bytes_; }
    size_t max_batch_blocks() const { return max_batch_; }
    int block_location(uint32_t block);   // -1 when not in use
    // The hint / protect path: on_access of the block's handle; false when
    // the block is not in use.
    bool policy_access(uint32_t block);
    // Eviction in two steps around the data copy: victims chosen by the
    // policy among GPU-resident blocks (in id order), each given a swap slot
    // and marked evicting; then, once copied, the page handle goes back to
    // the free list and the block is swapped out (copied == false rolls back).
    std::vector<TierMove> begin_evict(uint32_t count);
    void end_evict(const std::vector<TierMove>& moves, bool copied);
    // Restore in two steps: ids validated (out of bounds, not in use or in
    // transit: error, nothing done), swapped-out ids (each once) given a new
    // page by the allocation rule and marked restoring; fewer than 8 stop at
    // the first allocation failure, 8 or more skip it (*partial set, *err
    // says why).  Then, once copied, each block is GPU-resident, its swap
    // slot free and the policy told of an access.
    bool begin_restore(const uint32_t* ids, size_t n, std::vector<TierMove>* moves,
                       bool* partial, std::string* err);
    void end_restore(const std::vector<TierMove>& moves, bool copied);

    Stats stats();
    Metrics metrics();
    bool below_low_watermark(float threshold);
    bool has_free_blocks();
    uint32_t blocks_in_use();
    uint32_t total_blocks();
    uint32_t free_physical_blocks();
    uint32_t active_sequences();
    uint64_t epoch();

private:
    bool ensure_capacity_locked(std::string* err);
    bool alloc_one_locked(uint32_t* id, std::string* err);
    void release_locked(const uint32_t* ids, size_t n);
    uint32_t blocks_in_use_locked() const;

    PoolGeometry geo_;
    std::unique_ptr<PageBacking> backing_;
    std::mutex mu_;
    // Physical page handles (superblock, index) -- one list for all 2*L
    // regions, which the reference keeps identical by construction
    // ("lockstep", ref pool.rs:364-410).
    std::vector<std::pair<uint32_t, uint32_t>> free_handles_;
    size_t superblock_count_ = 0;
    std::vector<BlockInfo> blocks_;
    // Reference count per block id, beside blocks_ (kept out of BlockInfo so
    // the fork and release passes over a table touch 4 bytes per entry).
    std::vector<uint32_t> rc_;
    std::vector<uint32_t> free_ids_;
    // Sequence indices are never reused, so a serving loop that forks keeps
    // appending; a deque never moves the sequences it already holds.
    std::deque<SequenceState> seqs_;
    // Block-table buffers of unregistered sequences, kept (emptied) for the
    // next sequence that needs one, so that forks and registrations of a
    // steady serving loop do not go to the heap for every table.
    static constexpr size_t kMaxSpareTables = 1024;
    std::vector<std::vector<uint32_t>> spare_tables_;
    std::vector<uint32_t> take_table_locked();

    // Shared table bases of beam forks.  fork_beams moves a parent's table
    // up to its next-token page into a base that the parent and its
    // children all start with, so a child costs its short tail, not a copy
    // of the table.  The base's references are counted lazily: rc_ holds
    // (holders - lazy) references per base id and `lazy` holders own theirs
    // only through the base, so a fork adds holders in O(1) and a holder
    // that leaves while lazy > 0 just decrements lazy (no block of the base
    // can reach zero then).  The count an id would have with eager counting
    // is rc_ + the lazy counts of the bases that list it; every path that
    // needs it exactly (a refcount query, a release or privacy check of an
    // id that rc_ alone puts at 1) first makes all bases eager
    // (flush_lazy_locked), which is rare in a beam loop.  A base one of
    // whose ids is freed while it lives (a caller freeing a block a table
    // still holds) stays eager for good.
    struct SharedBase {
        std::vector<uint32_t> ids;
        uint32_t holders = 0;
        uint32_t lazy = 0;
        bool eager_only = false;
    };
    std::vector<SharedBase> bases_;
    std::vector<int32_t> free_bases_;
    std::vector<uint32_t> in_base_;     // per block id: how many bases list it
    uint64_t lazy_total_ = 0;           // sum of lazy over the bases
    static constexpr size_t kMaxSharedTail = 64;

    size_t table_size(const SequenceState& s) const {
        return (s.base >= 0 ? bases_[s.base].ids.size() : 0) + s.table.size();
    }
    uint32_t table_at(const SequenceState& s, size_t i) const {
        if (s.base >= 0) {
            const auto& b = bases_[s.base].ids;
            if (i < b.size()) return b[i];
            return s.table[i - b.size()];
        }
        return s.table[i];
    }
    template <typename F>
    void for_each_id(const SequenceState& s, F&& f) const {
        if (s.base >= 0)
            for (uint32_t id : bases_[s.base].ids) f(id);
        for (uint32_t id : s.table) f(id);
    }
    void flush_lazy_locked();
    // make sure rc_[id] is the exact count of an id that rc_ puts at 1
    void exact_rc_locked(uint32_t id) {
        if (lazy_total_ != 0 && id < in_base_.size() && in_base_[id] != 0 && rc_[id] == 1)
            flush_lazy_locked();
    }
    int32_t new_base_locked(SequenceState& s, size_t cut);
    // the sequence stops using its base: keep_refs moves the base's ids into
    // its own table (references kept), else its references are released
    void leave_base_locked(SequenceState& s, bool keep_refs);
    void poison_bases_locked(uint32_t id);
    struct PrefixEntry {
        uint32_t block;
        uint32_t depth;       // position in the prefix it was registered at
        uint64_t last_use;    // prefix_tick_ when registered or last matched
    };
    std::unordered_map<uint64_t, PrefixEntry> prefix_;
    uint64_t prefix_tick_ = 0;
    uint32_t prefix_match_locked(const uint64_t* hashes, uint32_t n, uint32_t* blocks);
    uint64_t epoch_ = 0;
    // tiering (null policy: disabled)
    std::unique_ptr<EvictionPolicy> policy_;
    std::unique_ptr<SwapSlots> slots_;
    uint64_t swap_bytes_ = 0, block_swap_bytes_ = 0;
    size_t max_batch_ = 0;
};

}  // namespace kcmm
