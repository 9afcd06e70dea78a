// Host bookkeeping of a KCMM pool.  The allocation rules this file must keep
// bit-exact are listed in pool_core.hpp with their reference lines.
#include "pool_core.hpp"

#include <algorithm>
#include <cstdio>
#include <map>

namespace kcmm {

namespace {

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

std::string fmt(const char* f, unsigned long long a = 0, unsigned long long b = 0,
                unsigned long long c = 0, unsigned long long d = 0) {
    char buf[512];
    std::snprintf(buf, sizeof(buf), f, a, b, c, d);
    return buf;
}

}  // namespace

bool PoolGeometry::compute(std::string* err) {
    if (num_layers == 0 || kv_heads == 0 || head_dim == 0 || block_size == 0) {
        *err = "pool geometry: num_layers, kv_heads, head_dim and block_size must be positive";
        return false;
    }
    switch (dtype) {
        case kF16:
        case kBF16: elem_bytes = 2; break;
        case kFP8: elem_bytes = 1; break;
        case kF32: elem_bytes = 4; break;
        default: *err = "pool geometry: unknown kv dtype"; return false;
    }
    row_bytes = kv_heads * head_dim * elem_bytes;
    data_bytes = block_size * row_bytes;
    // fp8 pages carry their per-kv-head fp32 scales in a footer; the page is
    // padded to 256 B so every page starts on a 256-B boundary.
    block_bytes = dtype == kFP8 ? align_up(data_bytes + kv_heads * 4, 256) : data_bytes;
    blocks_per_superblock = kSuperblockBytes / block_bytes;
    if (blocks_per_superblock == 0) {
        *err = fmt("pool geometry: block_bytes (%llu) too large for a 2 MiB superblock",
                   (unsigned long long)block_bytes);
        return false;
    }
    // ref pool.rs:206-207
    max_blocks_per_seq = (max_seq_len + block_size - 1) / block_size;
    max_blocks_total = max_batch * max_blocks_per_seq;
    if (max_blocks_total == 0) {
        *err = "pool geometry: max_batch and max_seq_len must be positive";
        return false;
    }
    // ref pool.rs:1145-1152
    const size_t sbs = (max_blocks_total + blocks_per_superblock - 1) / blocks_per_superblock;
    max_physical_blocks = sbs * blocks_per_superblock;
    // The reference reserves align_up(max_blocks_total*block_bytes, 2 MiB)
    // (ref pool.rs:211-212), which can be one superblock short of its own
    // capacity limit when block_bytes does not divide 2 MiB; reserve enough
    // for every superblock the capacity rule admits.
    region_bytes = std::max(align_up(max_blocks_total * block_bytes, kSuperblockBytes),
                            sbs * kSuperblockBytes);
    return true;
}

PoolCore::PoolCore(const PoolGeometry& g, std::unique_ptr<PageBacking> backing)
    : geo_(g), backing_(std::move(backing)) {}

PoolCore::~PoolCore() {
    if (backing_) backing_->release();
}

bool PoolCore::ensure_capacity_locked(std::string* err) {
    if (!free_handles_.empty()) return true;
    const size_t bps = geo_.blocks_per_superblock;
    const size_t total = superblock_count_ * bps;
    if (total >= geo_.max_physical_blocks) {
        // ref pool.rs:328-337 (same wording)
        *err = fmt("KCMM physical block capacity exhausted: total_physical_blocks=%llu "
                   "max_physical_blocks_per_layer=%llu max_blocks_total=%llu "
                   "blocks_per_superblock=%llu",
                   total, geo_.max_physical_blocks, geo_.max_blocks_total, bps);
        return false;
    }
    if (!backing_->map_superblock(superblock_count_, err)) return false;
    const uint32_t sb = static_cast<uint32_t>(superblock_count_);
    for (size_t i = 0; i < bps; ++i) free_handles_.emplace_back(sb, static_cast<uint32_t>(i));
    ++superblock_count_;
    ++epoch_;
    return true;
}

bool PoolCore::alloc_one_locked(uint32_t* id_out, std::string* err) {
    if (!ensure_capacity_locked(err)) return false;
    const auto h = free_handles_.back();
    free_handles_.pop_back();
    BlockInfo bi;
    bi.va_offset = static_cast<uint64_t>(h.first) * kSuperblockBytes +
                   static_cast<uint64_t>(h.second) * geo_.block_bytes;
    bi.superblock_idx = h.first;
    bi.block_index = h.second;
    bi.in_use = true;
    bi.location = kLocGpu;
    uint32_t id;
    if (!free_ids_.empty()) {
        id = free_ids_.back();
        free_ids_.pop_back();
        blocks_[id] = bi;
    } else {
        id = static_cast<uint32_t>(blocks_.size());
        blocks_.push_back(bi);
        rc_.push_back(0);
        in_base_.push_back(0);
    }
    rc_[id] = 1;
    ++epoch_;
    *id_out = id;
    if (policy_) policy_->on_allocate(h);   // ref pool.rs:446-449
    return true;
}

bool PoolCore::alloc_blocks(uint32_t n, uint32_t* out, std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    const size_t ids_before = blocks_.size();
    for (uint32_t i = 0; i < n; ++i) {
        if (!alloc_one_locked(&out[i], err)) {
            // Undo this call's allocations in reverse so the free lists are
            // exactly as before (superblocks mapped meanwhile stay mapped).
            for (uint32_t j = i; j-- > 0;) {
                BlockInfo& bi = blocks_[out[j]];
                free_handles_.emplace_back(bi.superblock_idx, bi.block_index);
                if (out[j] >= ids_before) {
                    blocks_.pop_back();
                    rc_.pop_back();
                    in_base_.pop_back();
                } else {
                    bi = BlockInfo{};
                    free_ids_.push_back(out[j]);
                }
            }
            ++epoch_;
            return false;
        }
    }
    return true;
}

void PoolCore::release_locked(const uint32_t* ids, size_t n) {
    std::vector<uint32_t> recycled;
    for (size_t i = 0; i < n; ++i) {
        const uint32_t id = ids[i];
        if (id >= blocks_.size()) continue;
        BlockInfo& bi = blocks_[id];
        if (!bi.in_use) continue;
        exact_rc_locked(id);
        if (rc_[id] > 1) {
            --rc_[id];
            continue;
        }
        // ref pool.rs:491-545: a swapped-out block gives back its swap slot,
        // one in transit is left alone
        if (bi.location == kLocEvicting || bi.location == kLocRestoring) continue;
        bi.in_use = false;
        rc_[id] = 0;
        if (in_base_[id] != 0) poison_bases_locked(id);
        if (bi.location == kLocCpu) {
            if (slots_) slots_->free(bi.cpu_offset, block_swap_bytes_);
        } else {
            free_handles_.emplace_back(bi.superblock_idx, bi.block_index);
        }
        bi.location = kLocGpu;
        recycled.push_back(id);
    }
    if (!recycled.empty()) {
        ++epoch_;
        free_ids_.insert(free_ids_.end(), recycled.begin(), recycled.end());
    }
}

void PoolCore::free_blocks(const uint32_t* ids, size_t n) {
    std::lock_guard<std::mutex> lk(mu_);
    release_locked(ids, n);
}

std::vector<uint32_t> PoolCore::take_table_locked() {
    std::vector<uint32_t> t;
    if (!spare_tables_.empty()) {
        t.swap(spare_tables_.back());
        spare_tables_.pop_back();
    }
    return t;
}

uint32_t PoolCore::register_sequence(const uint32_t* table, size_t n) {
    std::lock_guard<std::mutex> lk(mu_);
    SequenceState s;
    s.table = take_table_locked();
    s.table.assign(table, table + n);
    seqs_.push_back(std::move(s));
    return static_cast<uint32_t>(seqs_.size() - 1);
}

void PoolCore::unregister_sequence(uint32_t seq) {
    std::lock_guard<std::mutex> lk(mu_);
    if (seq >= seqs_.size()) return;
    // table order: the shared base's ids, then the sequence's own
    if (seqs_[seq].base >= 0) leave_base_locked(seqs_[seq], false);
    std::vector<uint32_t> table;
    table.swap(seqs_[seq].table);
    seqs_[seq].seq_len = 0;
    if (!table.empty()) release_locked(table.data(), table.size());
    if (table.capacity() != 0 && spare_tables_.size() < kMaxSpareTables) {
        table.clear();
        spare_tables_.push_back(std::move(table));
    }
}

void PoolCore::touch(uint32_t seq) {
    std::lock_guard<std::mutex> lk(mu_);
    if (seq < seqs_.size()) seqs_[seq].active = true;
}

void PoolCore::cool(uint32_t seq) {
    std::lock_guard<std::mutex> lk(mu_);
    if (seq < seqs_.size()) seqs_[seq].active = false;
}

void PoolCore::set_priority(uint32_t seq, int prio) {
    std::lock_guard<std::mutex> lk(mu_);
    if (seq < seqs_.size()) seqs_[seq].priority = prio;
}

bool PoolCore::has_sequence(uint32_t seq) {
    std::lock_guard<std::mutex> lk(mu_);
    return seq < seqs_.size();
}

void PoolCore::update_seq_len(uint32_t seq, uint32_t len) {
    std::lock_guard<std::mutex> lk(mu_);
    if (seq < seqs_.size()) seqs_[seq].seq_len = len;
}

uint32_t PoolCore::get_seq_len(uint32_t seq) {
    std::lock_guard<std::mutex> lk(mu_);
    return seq < seqs_.size() ? seqs_[seq].seq_len : 0;
}

bool PoolCore::append_block_to_sequence(uint32_t seq, uint32_t block) {
    std::lock_guard<std::mutex> lk(mu_);
    if (seq >= seqs_.size()) return false;
    seqs_[seq].table.push_back(block);
    return true;
}

bool PoolCore::get_block_table(uint32_t seq, std::vector<uint32_t>* out) {
    std::lock_guard<std::mutex> lk(mu_);
    if (seq >= seqs_.size()) return false;
    out->clear();
    out->reserve(table_size(seqs_[seq]));
    for_each_id(seqs_[seq], [out](uint32_t id) { out->push_back(id); });
    return true;
}

bool PoolCore::block_va_offset(uint32_t block, uint64_t* out) {
    std::lock_guard<std::mutex> lk(mu_);
    if (block >= blocks_.size() || !blocks_[block].in_use) return false;
    *out = blocks_[block].va_offset;
    return true;
}

std::vector<uint64_t> PoolCore::all_offsets_f16() {
    std::lock_guard<std::mutex> lk(mu_);
    std::vector<uint64_t> v(blocks_.size());
    for (size_t i = 0; i < blocks_.size(); ++i)
        v[i] = blocks_[i].in_use ? blocks_[i].va_offset / 2 : 0;
    return v;
}

std::vector<uint8_t> PoolCore::all_valid_flags() {
    std::lock_guard<std::mutex> lk(mu_);
    std::vector<uint8_t> v(blocks_.size());
    for (size_t i = 0; i < blocks_.size(); ++i) v[i] = blocks_[i].in_use ? 1 : 0;
    return v;
}

bool PoolCore::table_va_offsets(uint32_t seq, std::vector<uint64_t>* out) {
    std::lock_guard<std::mutex> lk(mu_);
    if (seq >= seqs_.size()) return false;
    out->clear();
    const SequenceState& s = seqs_[seq];
    for (size_t i = 0, n = table_size(s); i < n; ++i) {
        const uint32_t id = table_at(s, i);
        if (id >= blocks_.size() || !blocks_[id].in_use) return false;
        out->push_back(blocks_[id].va_offset);
    }
    return true;
}

uint32_t PoolCore::refcount(uint32_t block) {
    std::lock_guard<std::mutex> lk(mu_);
    if (block >= blocks_.size() || !blocks_[block].in_use) return 0;
    if (lazy_total_ != 0 && in_base_[block] != 0) flush_lazy_locked();
    return rc_[block];
}

bool PoolCore::fork_sequence(uint32_t src, uint32_t* out_seq, std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    if (src >= seqs_.size()) {
        *err = fmt("kcmm_fork_sequence: seq_idx %llu out of bounds", src);
        return false;
    }
    SequenceState s;
    s.table = take_table_locked();
    s.table.reserve(table_size(seqs_[src]));
    for_each_id(seqs_[src], [&s](uint32_t id) { s.table.push_back(id); });
    s.seq_len = seqs_[src].seq_len;
    for (uint32_t id : s.table)
        if (id < blocks_.size() && blocks_[id].in_use) ++rc_[id];
    seqs_.push_back(std::move(s));
    *out_seq = static_cast<uint32_t>(seqs_.size() - 1);
    return true;
}

bool PoolCore::share_prefix(uint32_t src, uint32_t dst, uint32_t n, uint32_t* out,
                            std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    if (src >= seqs_.size() || dst >= seqs_.size()) {
        *err = fmt("kcmm_share_prefix: sequence index out of bounds (src %llu, dst %llu)", src,
                   dst);
        return false;
    }
    const SequenceState& st = seqs_[src];
    if (table_size(st) < n) {
        *err = fmt("kcmm_share_prefix: src seq %llu holds %llu blocks, %llu requested", src,
                   table_size(st), n);
        return false;
    }
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t id = table_at(st, i);
        if (id >= blocks_.size() || !blocks_[id].in_use) {
            *err = fmt("kcmm_share_prefix: block %llu not in use", id);
            return false;
        }
    }
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t id = table_at(seqs_[src], i);
        ++rc_[id];
        seqs_[dst].table.push_back(id);
        out[i] = id;
    }
    return true;
}

// FNV-1a (64-bit) over the little-endian bytes of the previous block's hash
// (the seed for block 0) followed by the block's token ids (int32, LE).
size_t prefix_hash_blocks(const int32_t* tokens, size_t n_tokens, size_t block_size,
                          uint64_t seed, uint64_t* out, size_t max_out) {
    const size_t nb = block_size ? n_tokens / block_size : 0;
    uint64_t prev = seed;
    size_t i = 0;
    for (; i < nb && i < max_out; ++i) {
        uint64_t h = 0xcbf29ce484222325ull;
        auto mix = [&h](uint32_t b) {
            h ^= b;
            h *= 0x100000001b3ull;
        };
        for (int k = 0; k < 8; ++k) mix(static_cast<uint32_t>((prev >> (8 * k)) & 0xFF));
        for (size_t t = 0; t < block_size; ++t) {
            const uint32_t v = static_cast<uint32_t>(tokens[i * block_size + t]);
            for (int k = 0; k < 4; ++k) mix((v >> (8 * k)) & 0xFF);
        }
        out[i] = h;
        prev = h;
    }
    return i;
}

bool PoolCore::prefix_register(uint32_t seq, const uint64_t* hashes, uint32_t n,
                               uint32_t* added, std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    *added = 0;
    if (seq >= seqs_.size()) {
        *err = fmt("kcmm_prefix_register: seq_idx %llu out of bounds", seq);
        return false;
    }
    const SequenceState& s = seqs_[seq];
    if (n > table_size(s)) {
        *err = fmt("kcmm_prefix_register: seq %llu holds %llu blocks, %llu requested", seq,
                   table_size(s), n);
        return false;
    }
    if (static_cast<uint64_t>(n) * geo_.block_size > s.seq_len) {
        *err = fmt("kcmm_prefix_register: only full blocks are cached (%llu blocks of %llu "
                   "tokens > seq_len %llu)", n, geo_.block_size, s.seq_len);
        return false;
    }
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t id = table_at(s, i);
        if (id >= blocks_.size() || !blocks_[id].in_use) {
            *err = fmt("kcmm_prefix_register: block %llu not in use", id);
            return false;
        }
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (prefix_.count(hashes[i])) continue;
        const uint32_t id = table_at(s, i);
        prefix_.emplace(hashes[i], PrefixEntry{id, i, ++prefix_tick_});
        ++rc_[id];
        ++*added;
    }
    return true;
}

uint32_t PoolCore::prefix_match_locked(const uint64_t* hashes, uint32_t n, uint32_t* blocks) {
    const uint64_t now = ++prefix_tick_;
    uint32_t m = 0;
    for (; m < n; ++m) {
        auto it = prefix_.find(hashes[m]);
        if (it == prefix_.end()) break;
        it->second.last_use = now;
        if (blocks) blocks[m] = it->second.block;
    }
    return m;
}

uint32_t PoolCore::prefix_match(const uint64_t* hashes, uint32_t n, uint32_t* blocks) {
    std::lock_guard<std::mutex> lk(mu_);
    return prefix_match_locked(hashes, n, blocks);
}

bool PoolCore::prefix_attach(uint32_t dst, const uint64_t* hashes, uint32_t n, uint32_t* blocks,
                             uint32_t* matched, std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    *matched = 0;
    if (dst >= seqs_.size()) {
        *err = fmt("kcmm_prefix_attach: seq_idx %llu out of bounds", dst);
        return false;
    }
    std::vector<uint32_t> ids(n);
    const uint32_t m = prefix_match_locked(hashes, n, ids.data());
    for (uint32_t i = 0; i < m; ++i) {
        ++rc_[ids[i]];
        seqs_[dst].table.push_back(ids[i]);
        if (blocks) blocks[i] = ids[i];
    }
    *matched = m;
    return true;
}

uint32_t PoolCore::prefix_evict(uint32_t n) {
    std::lock_guard<std::mutex> lk(mu_);
    std::vector<std::pair<uint64_t, const PrefixEntry*>> order;
    order.reserve(prefix_.size());
    for (const auto& kv : prefix_) order.emplace_back(kv.first, &kv.second);
    std::sort(order.begin(), order.end(), [](const auto& a, const auto& b) {
        if (a.second->last_use != b.second->last_use) return a.second->last_use < b.second->last_use;
        return a.second->depth > b.second->depth;
    });
    const uint32_t k = static_cast<uint32_t>(std::min<size_t>(n, order.size()));
    std::vector<uint64_t> keys(k);
    std::vector<uint32_t> ids(k);
    for (uint32_t i = 0; i < k; ++i) {
        keys[i] = order[i].first;
        ids[i] = order[i].second->block;
    }
    for (uint32_t i = 0; i < k; ++i) prefix_.erase(keys[i]);
    if (k) release_locked(ids.data(), k);     // in eviction order
    return k;
}

uint32_t PoolCore::prefix_entries() {
    std::lock_guard<std::mutex> lk(mu_);
    return static_cast<uint32_t>(prefix_.size());
}

void PoolCore::flush_lazy_locked() {
    for (SharedBase& b : bases_) {
        if (b.lazy == 0) continue;
        for (uint32_t id : b.ids) rc_[id] += b.lazy;   // every id of such a base is in use
        lazy_total_ -= b.lazy;
        b.lazy = 0;
    }
}

int32_t PoolCore::new_base_locked(SequenceState& s, size_t cut) {
    int32_t idx;
    if (!free_bases_.empty()) {
        idx = free_bases_.back();
        free_bases_.pop_back();
    } else {
        idx = static_cast<int32_t>(bases_.size());
        bases_.emplace_back();
    }
    SharedBase& b = bases_[idx];
    b.ids = std::move(s.table);
    s.table = take_table_locked();
    s.table.assign(b.ids.begin() + cut, b.ids.end());
    b.ids.resize(cut);
    b.holders = 1;
    b.lazy = 0;
    b.eager_only = false;
    for (uint32_t id : b.ids) {
        if (id < in_base_.size()) ++in_base_[id];
        if (id >= blocks_.size() || !blocks_[id].in_use) b.eager_only = true;
    }
    s.base = idx;
    return idx;
}

void PoolCore::leave_base_locked(SequenceState& s, bool keep_refs) {
    const int32_t idx = s.base;
    s.base = -1;
    SharedBase& b = bases_[idx];
    if (keep_refs) {
        if (b.lazy > 0) {   // this holder's references become counted ones
            --b.lazy;
            --lazy_total_;
            for (uint32_t id : b.ids) ++rc_[id];
        }
        std::vector<uint32_t> t = take_table_locked();
        t.reserve(b.ids.size() + s.table.size());
        t.assign(b.ids.begin(), b.ids.end());
        t.insert(t.end(), s.table.begin(), s.table.end());
        s.table.swap(t);
        if (t.capacity() != 0 && spare_tables_.size() < kMaxSpareTables) {
            t.clear();
            spare_tables_.push_back(std::move(t));
        }
    } else if (b.lazy > 0) {
        --b.lazy;           // (every id keeps a count of 2 or more: nothing is freed)
        --lazy_total_;
    } else {
        release_locked(b.ids.data(), b.ids.size());
    }
    if (--b.holders == 0) {
        for (uint32_t id : b.ids)
            if (id < in_base_.size()) --in_base_[id];
        b.ids.clear();
        if (b.ids.capacity() != 0 && spare_tables_.size() < kMaxSpareTables) {
            spare_tables_.push_back(std::move(b.ids));
            b.ids = std::vector<uint32_t>();
        }
        free_bases_.push_back(idx);
    }
}

void PoolCore::poison_bases_locked(uint32_t id) {
    for (SharedBase& b : bases_) {
        if (b.holders == 0 || b.eager_only) continue;
        if (std::find(b.ids.begin(), b.ids.end(), id) != b.ids.end()) b.eager_only = true;
    }
}

bool PoolCore::fork_beams(const uint32_t* parents, uint32_t n, uint32_t width,
                          uint32_t* children, std::vector<uint32_t>* pairs, std::string* err) {
    if (width == 0) {
        *err = "kcmm_fork_beams: beam width must be at least 1";
        return false;
    }
    const uint32_t bs = static_cast<uint32_t>(geo_.block_size);
    const uint32_t forks = width - 1;
    std::lock_guard<std::mutex> lk(mu_);
    // Everything that can fail is checked before any state changes: the
    // parents, the page each child makes private, and the capacity for them.
    // Every child needs its own copy of that page: after the forks it is
    // shared by the parent and all the children still to be made private.
    size_t needed = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (parents[i] >= seqs_.size()) {
            *err = fmt("kcmm_fork_beams: parent seq_idx %llu out of bounds", parents[i]);
            return false;
        }
        const SequenceState& ps = seqs_[parents[i]];
        const uint32_t logical = ps.seq_len / bs;
        if (forks == 0 || logical >= table_size(ps)) continue;   // the next token opens a new page
        const uint32_t id = table_at(ps, logical);
        if (id >= blocks_.size() || !blocks_[id].in_use) {
            *err = fmt("kcmm_fork_beams: block %llu of parent %llu not in use", id, parents[i]);
            return false;
        }
        if (blocks_[id].location != kLocGpu) {
            *err = fmt("kcmm_fork_beams: block %llu is not resident in HBM (restore it first)", id);
            return false;
        }
        needed += forks;
    }
    const size_t grow = geo_.max_physical_blocks - superblock_count_ * geo_.blocks_per_superblock;
    if (needed > free_handles_.size() + grow) {
        *err = fmt("kcmm_fork_beams: %llu new pages needed, %llu free within the pool's capacity",
                   needed, free_handles_.size() + grow);
        return false;
    }
    if (forks == 0) return true;
    const size_t seqs0 = seqs_.size(), pairs0 = pairs->size();
    pairs->reserve(pairs0 + 2 * needed);
    // parents whose forks' references are taken: (parent, through its base)
    std::vector<std::pair<uint32_t, bool>> done;
    done.reserve(n);
    auto add_refs = [&](const std::vector<uint32_t>& ids, int64_t d) {
        for (uint32_t id : ids)
            if (id < rc_.size() && rc_[id] != 0)   // in use <=> rc > 0
                rc_[id] = static_cast<uint32_t>(static_cast<int64_t>(rc_[id]) + d);
    };
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t p = parents[i];
        SequenceState& ps = seqs_[p];
        const size_t total = table_size(ps);
        const uint32_t logical = ps.seq_len / bs;
        // The table up to the next-token page is shared through a base (made
        // from the parent's own table the first time; remade when the parent
        // has grown far past it); what follows is copied into each child.
        const size_t cut = std::min<size_t>(logical, total);
        if (ps.base >= 0 && !bases_[ps.base].eager_only &&
            (bases_[ps.base].ids.size() > cut || cut - bases_[ps.base].ids.size() > kMaxSharedTail))
            leave_base_locked(ps, true);
        if (ps.base < 0 && cut > 0) new_base_locked(ps, cut);
        const bool shared = ps.base >= 0 && !bases_[ps.base].eager_only;
        if (shared) {
            // the forks' references: through the base (counted lazily) and,
            // for the parent's own entries, one each
            SharedBase& b = bases_[ps.base];
            b.holders += forks;
            b.lazy += forks;
            lazy_total_ += forks;
            add_refs(ps.table, forks);
        } else {
            for_each_id(ps, [&](uint32_t id) {
                if (id < rc_.size() && rc_[id] != 0) rc_[id] += forks;
            });
        }
        done.emplace_back(p, shared);
        const size_t bl = shared ? bases_[ps.base].ids.size() : 0;
        for (uint32_t c = 0; c < forks; ++c) {
            SequenceState s;
            s.table = take_table_locked();
            if (shared) {
                s.base = ps.base;
                s.table.assign(ps.table.begin(), ps.table.end());
            } else {
                s.table.reserve(total);
                for_each_id(ps, [&s](uint32_t id) { s.table.push_back(id); });
            }
            s.seq_len = ps.seq_len;
            seqs_.push_back(std::move(s));
            const uint32_t child = static_cast<uint32_t>(seqs_.size() - 1);
            children[static_cast<size_t>(i) * forks + c] = child;
            if (logical >= total) continue;
            // (logical >= bl: the base ends at the next-token page)
            const uint32_t old_id = seqs_[child].table[logical - bl];
            uint32_t new_id = 0;
            if (!alloc_one_locked(&new_id, err)) {
                // Only a page backing that fails to map memory gets here.
                // Undo the call: new pages back in reverse order (the free
                // list is LIFO), references and children removed (the
                // parents keep their bases: the same tables).
                for (size_t q = pairs->size(); q > pairs0; q -= 2) {
                    const uint32_t nid = (*pairs)[q - 1];
                    rc_[nid] = 1;
                    release_locked(&nid, 1);
                    ++rc_[(*pairs)[q - 2]];
                }
                pairs->resize(pairs0);
                for (const auto& d : done) {
                    SequenceState& q = seqs_[d.first];
                    if (d.second) {
                        SharedBase& b = bases_[q.base];
                        b.holders -= forks;
                        b.lazy -= forks;
                        lazy_total_ -= forks;
                        add_refs(q.table, -static_cast<int64_t>(forks));
                    } else {
                        for_each_id(q, [&](uint32_t id) {
                            if (id < rc_.size() && rc_[id] != 0) rc_[id] -= forks;
                        });
                    }
                }
                while (seqs_.size() > seqs0) seqs_.pop_back();
                return false;
            }
            seqs_[child].table[logical - bl] = new_id;
            --rc_[old_id];
            pairs->push_back(old_id);
            pairs->push_back(new_id);
        }
    }
    return true;
}

int PoolCore::cow_block_for_append(uint32_t seq, uint32_t logical, uint32_t* src,
                                   uint32_t* dst, std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    if (seq >= seqs_.size()) {
        *err = fmt("kcmm_cow_block_for_append: seq_idx %llu out of bounds", seq);
        return -1;
    }
    SequenceState& s = seqs_[seq];
    if (logical >= table_size(s)) {
        *err = fmt("kcmm_cow_block_for_append: logical block %llu >= allocated %llu", logical,
                   table_size(s));
        return -1;
    }
    const uint32_t old_id = table_at(s, logical);
    if (old_id >= blocks_.size() || !blocks_[old_id].in_use) {
        *err = fmt("kcmm_cow_block_for_append: block %llu not in use", old_id);
        return -1;
    }
    exact_rc_locked(old_id);
    if (rc_[old_id] <= 1) return 0;
    if (blocks_[old_id].location != kLocGpu) {
        *err = fmt("kcmm_cow_block_for_append: block %llu is not resident in HBM "
                   "(restore it first)", old_id);
        return -1;
    }
    uint32_t new_id;
    if (!alloc_one_locked(&new_id, err)) return -1;
    if (s.base >= 0 && logical < bases_[s.base].ids.size()) leave_base_locked(s, true);
    const size_t bl = s.base >= 0 ? bases_[s.base].ids.size() : 0;
    s.table[logical - bl] = new_id;
    --rc_[old_id];
    *src = old_id;
    *dst = new_id;
    return 1;
}

bool PoolCore::resolve_pairs(const uint32_t* pairs, size_t n, std::vector<uint64_t>* out,
                             std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    out->resize(2 * n);
    for (size_t i = 0; i < 2 * n; ++i) {
        const uint32_t id = pairs[i];
        if (id >= blocks_.size() || !blocks_[id].in_use) {
            *err = fmt("kcmm_copy_blocks: block %llu not in use", id);
            return false;
        }
        if (blocks_[id].location != kLocGpu) {
            *err = fmt("kcmm_copy_blocks: block %llu is not resident in HBM", id);
            return false;
        }
        (*out)[i] = blocks_[id].va_offset;
    }
    return true;
}

bool PoolCore::resolve_positions(const uint32_t* seqs, const uint32_t* pos, uint32_t batch,
                                 std::vector<RowDst>* out, std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    out->clear();
    out->reserve(batch);
    for (uint32_t b = 0; b < batch; ++b) {
        if (seqs[b] >= seqs_.size()) {
            *err = fmt("kcmm_append_kv_step: seq_idx %llu out of bounds", seqs[b]);
            return false;
        }
        const SequenceState& sq = seqs_[seqs[b]];
        const size_t lb = pos[b] / geo_.block_size;
        const size_t off = pos[b] % geo_.block_size;
        if (lb >= table_size(sq)) {
            *err = fmt("kcmm_append_kv_step: logical_block %llu >= allocated %llu for seq %llu",
                       lb, table_size(sq), seqs[b]);
            return false;
        }
        const uint32_t id = table_at(sq, lb);
        if (id >= blocks_.size() || !blocks_[id].in_use) {
            *err = fmt("kcmm_append_kv_step: block_idx %llu not in use", id);
            return false;
        }
        exact_rc_locked(id);
        if (rc_[id] > 1) {
            if (lazy_total_ != 0 && in_base_[id] != 0) flush_lazy_locked();   // exact count
            *err = fmt("kcmm_append_kv_step: block_idx %llu is shared (refcount %llu); "
                       "make it private with kcmm_cow_block_for_append first",
                       id, rc_[id]);
            return false;
        }
        if (blocks_[id].location != kLocGpu) {
            *err = fmt("kcmm_append_kv_step: block_idx %llu is not resident in HBM "
                       "(restore it first)", id);
            return false;
        }
        out->push_back(RowDst{b, blocks_[id].va_offset, static_cast<uint32_t>(off)});
    }
    return true;
}

bool PoolCore::resolve_slots(const int64_t* slots, uint32_t batch, std::vector<RowDst>* out,
                             std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    out->clear();
    out->reserve(batch);
    for (uint32_t b = 0; b < batch; ++b) {
        if (slots[b] < 0) continue;  // padding row (ref ffi.rs:1327)
        const uint64_t s = static_cast<uint64_t>(slots[b]);
        const uint64_t id = s / geo_.block_size;
        const uint32_t off = static_cast<uint32_t>(s % geo_.block_size);
        if (id >= blocks_.size() || !blocks_[id].in_use) {
            *err = fmt("kcmm_append_kv_slots: block_idx %llu from slot %llu not in use", id,
                       s);
            return false;
        }
        exact_rc_locked(static_cast<uint32_t>(id));
        if (rc_[id] > 1) {
            if (lazy_total_ != 0 && in_base_[id] != 0) flush_lazy_locked();   // exact count
            *err = fmt("kcmm_append_kv_slots: block_idx %llu is shared (refcount %llu)", id,
                       rc_[id]);
            return false;
        }
        if (blocks_[id].location != kLocGpu) {
            *err = fmt("kcmm_append_kv_slots: block_idx %llu is not resident in HBM "
                       "(restore it first)", id);
            return false;
        }
        out->push_back(RowDst{b, blocks_[id].va_offset, off});
    }
    return true;
}

// ---- tiering ------------------------------------------------------------------

void PoolCore::enable_tiering(int policy, size_t max_blocks, size_t max_batch_blocks) {
    std::lock_guard<std::mutex> lk(mu_);
    block_swap_bytes_ = static_cast<uint64_t>(geo_.num_layers) * 2 * geo_.block_bytes;
    swap_bytes_ = static_cast<uint64_t>(max_blocks) * block_swap_bytes_;
    max_batch_ = max_batch_blocks;
    const PolicyKind k = policy == 1 ? PolicyKind::kLfu
                         : policy == 2 ? PolicyKind::kFifo
                                       : PolicyKind::kLru;
    policy_.reset(new EvictionPolicy(k, max_blocks));
    slots_.reset(new SwapSlots(swap_bytes_));
}

bool PoolCore::tiering_enabled() {
    std::lock_guard<std::mutex> lk(mu_);
    return policy_ != nullptr;
}

// ref tiering.rs:851-875: a fresh policy, arc sized from the swap buffer
bool PoolCore::set_eviction_policy(const std::string& name) {
    std::lock_guard<std::mutex> lk(mu_);
    if (!policy_) return false;
    PolicyKind k;
    size_t cap = 1;
    if (name == "lru") k = PolicyKind::kLru;
    else if (name == "lfu") k = PolicyKind::kLfu;
    else if (name == "fifo") k = PolicyKind::kFifo;
    else if (name == "sink_window") k = PolicyKind::kSinkWindow;
    else if (name == "arc") {
        k = PolicyKind::kArc;
        cap = static_cast<size_t>(swap_bytes_ / std::max<size_t>(max_batch_, 1));
    } else {
        return false;
    }
    policy_.reset(new EvictionPolicy(k, cap));
    return true;
}

std::string PoolCore::eviction_policy_name() {
    std::lock_guard<std::mutex> lk(mu_);
    return policy_ ? policy_->name() : "";
}

int PoolCore::block_location(uint32_t block) {
    std::lock_guard<std::mutex> lk(mu_);
    if (block >= blocks_.size() || !blocks_[block].in_use) return -1;
    return blocks_[block].location;
}

bool PoolCore::policy_access(uint32_t block) {
    std::lock_guard<std::mutex> lk(mu_);
    if (block >= blocks_.size() || !blocks_[block].in_use) return false;
    if (policy_) policy_->on_access({blocks_[block].superblock_idx, blocks_[block].block_index});
    return true;
}

std::vector<TierMove> PoolCore::begin_evict(uint32_t count) {
    std::lock_guard<std::mutex> lk(mu_);
    std::vector<TierMove> moves;
    if (!policy_ || count == 0) return moves;
    std::vector<PageHandle> cands;
    std::map<PageHandle, uint32_t> owner;
    for (uint32_t i = 0; i < blocks_.size(); ++i) {
        const BlockInfo& b = blocks_[i];
        if (!b.in_use || b.location != kLocGpu) continue;
        const PageHandle h{b.superblock_idx, b.block_index};
        cands.push_back(h);
        owner.emplace(h, i);
    }
    for (const PageHandle& h : policy_->select_victims(cands, count)) {
        const uint32_t id = owner.at(h);
        uint64_t off;
        if (!slots_->allocate(block_swap_bytes_, &off)) continue;   // swap full: skipped
        BlockInfo& b = blocks_[id];
        b.location = kLocEvicting;
        b.cpu_offset = off;
        moves.push_back(TierMove{id, b.va_offset, off});
    }
    if (!moves.empty()) ++epoch_;
    return moves;
}

void PoolCore::end_evict(const std::vector<TierMove>& moves, bool copied) {
    std::lock_guard<std::mutex> lk(mu_);
    for (const TierMove& m : moves) {
        BlockInfo& b = blocks_[m.block];
        if (copied) {
            // ref tiering.rs:995-1010, 1172-1176: the page handle returns to
            // the free list, the policy forgets it
            free_handles_.emplace_back(b.superblock_idx, b.block_index);
            b.location = kLocCpu;
            policy_->on_evict({b.superblock_idx, b.block_index});
        } else {
            slots_->free(m.cpu_offset, block_swap_bytes_);
            b.location = kLocGpu;
            b.cpu_offset = 0;
        }
    }
    if (!moves.empty()) ++epoch_;
}

bool PoolCore::begin_restore(const uint32_t* ids, size_t n, std::vector<TierMove>* moves,
                             bool* partial, std::string* err) {
    std::lock_guard<std::mutex> lk(mu_);
    moves->clear();
    *partial = false;
    if (!policy_) {
        *err = "tiering is disabled; cannot restore evicted blocks";
        return false;
    }
    // ref pool.rs:905-931: every id checked before anything changes
    for (size_t i = 0; i < n; ++i) {
        if (ids[i] >= blocks_.size()) {
            *err = fmt("block_idx %llu out of bounds", ids[i]);
            return false;
        }
        const BlockInfo& b = blocks_[ids[i]];
        if (!b.in_use) {
            *err = fmt("block_idx %llu is not in use", ids[i]);
            return false;
        }
        if (b.location == kLocEvicting || b.location == kLocRestoring) {
            *err = fmt(b.location == kLocEvicting
                           ? "block %llu is in transit (Evicting); cannot restore"
                           : "block %llu is in transit (Restoring); cannot restore",
                       ids[i]);
            return false;
        }
    }
    std::vector<uint32_t> todo;
    for (size_t i = 0; i < n; ++i)
        if (blocks_[ids[i]].location == kLocCpu &&
            std::find(todo.begin(), todo.end(), ids[i]) == todo.end())
            todo.push_back(ids[i]);
    // ref tiering.rs:1711-1745: fewer than 8 one at a time (the first
    // failure ends the call), 8 or more as a batch (failures skipped)
    const bool one_by_one = todo.size() < 8;
    size_t failed = 0;
    std::string alloc_err;
    for (uint32_t id : todo) {
        if (!ensure_capacity_locked(&alloc_err)) {
            ++failed;
            if (one_by_one) break;
            continue;
        }
        const auto h = free_handles_.back();
        free_handles_.pop_back();
        BlockInfo& b = blocks_[id];
        b.superblock_idx = h.first;
        b.block_index = h.second;
        b.va_offset = static_cast<uint64_t>(h.first) * kSuperblockBytes +
                      static_cast<uint64_t>(h.second) * geo_.block_bytes;
        b.location = kLocRestoring;
        moves->push_back(TierMove{id, b.va_offset, b.cpu_offset});
    }
    if (!moves->empty()) ++epoch_;
    if (failed > 0) {
        *partial = true;
        if (one_by_one)
            *err = alloc_err;
        else if (moves->empty())
            *err = fmt("batched restore could not allocate GPU physical blocks for any of %llu "
                       "requested blocks", todo.size());
        else
            *err = fmt("batched restore only restored %llu of %llu requested blocks",
                       moves->size(), todo.size());
    }
    return true;
}

void PoolCore::end_restore(const std::vector<TierMove>& moves, bool copied) {
    std::lock_guard<std::mutex> lk(mu_);
    for (const TierMove& m : moves) {
        BlockInfo& b = blocks_[m.block];
        if (copied) {
            // ref tiering.rs:1860-1885
            b.location = kLocGpu;
            slots_->free(m.cpu_offset, block_swap_bytes_);
            b.cpu_offset = 0;
            policy_->on_access({b.superblock_idx, b.block_index});
        } else {
            free_handles_.emplace_back(b.superblock_idx, b.block_index);
            b.location = kLocCpu;
        }
    }
    if (!moves.empty()) ++epoch_;
}

uint32_t PoolCore::blocks_in_use_locked() const {
    uint32_t n = 0;
    for (const auto& b : blocks_) n += b.in_use ? 1 : 0;
    return n;
}

Stats PoolCore::stats() {
    std::lock_guard<std::mutex> lk(mu_);
    Stats s{};
    s.blocks_in_use = blocks_in_use_locked();
    s.total_blocks = static_cast<uint32_t>(blocks_.size());
    s.total_physical_blocks = static_cast<uint32_t>(superblock_count_ * geo_.blocks_per_superblock);
    s.free_physical_blocks = static_cast<uint32_t>(free_handles_.size());
    s.active_sequences = static_cast<uint32_t>(seqs_.size());
    s.num_layers = static_cast<uint32_t>(geo_.num_layers);
    s.blocks_per_superblock = static_cast<uint32_t>(geo_.blocks_per_superblock);
    s.superblock_count = static_cast<uint32_t>(superblock_count_);
    s.block_size = static_cast<uint32_t>(geo_.block_size);
    s.max_blocks_per_seq = static_cast<uint32_t>(geo_.max_blocks_per_seq);
    s.block_bytes = static_cast<uint32_t>(geo_.block_bytes);
    // ref pool.rs:1160-1172
    s.physical_idle_ratio = 0.0f;
    if (superblock_count_ > 0) {
        const uint64_t total = static_cast<uint64_t>(superblock_count_) * kSuperblockBytes *
                               geo_.num_layers * 2;
        const uint64_t used = static_cast<uint64_t>(s.blocks_in_use) * geo_.block_bytes *
                              geo_.num_layers * 2;
        if (used < total)
            s.physical_idle_ratio = static_cast<float>(total - used) / static_cast<float>(total);
    }
    return s;
}

Metrics PoolCore::metrics() {
    // ref pool.rs:1179-1240 (collect_metrics) and metrics.rs:142-162, computed
    // in f32 exactly as the reference does.
    std::lock_guard<std::mutex> lk(mu_);
    Metrics m{};
    const uint64_t total_physical = superblock_count_ * geo_.blocks_per_superblock;
    const uint64_t in_use = blocks_in_use_locked();
    uint64_t blocks_used = 0, tokens = 0;
    for (const auto& s : seqs_) {
        blocks_used += table_size(s);
        tokens += s.seq_len;
    }
    const uint64_t layers2 = geo_.num_layers * 2;
    const uint64_t actual_physical = superblock_count_ * kSuperblockBytes * layers2;
    const uint64_t slots = blocks_used * geo_.block_size;
    m.ifr = slots > 0 ? static_cast<float>(static_cast<int64_t>(slots) -
                                           static_cast<int64_t>(tokens)) /
                            static_cast<float>(slots)
                      : 0.0f;
    m.bu = total_physical > 0
               ? static_cast<float>(in_use) / static_cast<float>(total_physical)
               : 0.0f;
    // The reference multiplies tokens by elements (not bytes) per token here.
    const uint64_t bpt_all = geo_.kv_heads * geo_.head_dim * layers2;
    const uint64_t ideal = tokens * bpt_all;
    m.pme = actual_physical > 0
                ? static_cast<float>(ideal) / static_cast<float>(actual_physical)
                : 1.0f;
    const uint64_t bps = geo_.blocks_per_superblock;
    const uint64_t active_sb = (in_use + bps - 1) / bps;
    const uint64_t actual_active = active_sb * kSuperblockBytes * layers2;
    m.rfi = actual_active > 0
                ? 1.0f - static_cast<float>(ideal) / static_cast<float>(actual_active)
                : 0.0f;
    m.gpu_blocks = in_use;
    return m;
}

bool PoolCore::below_low_watermark(float threshold) {
    std::lock_guard<std::mutex> lk(mu_);
    const size_t total = superblock_count_ * geo_.blocks_per_superblock;
    if (total == 0) return false;
    return static_cast<float>(free_handles_.size()) / static_cast<float>(total) < threshold;
}

bool PoolCore::has_free_blocks() {
    std::lock_guard<std::mutex> lk(mu_);
    return !free_handles_.empty();
}

uint32_t PoolCore::blocks_in_use() {
    std::lock_guard<std::mutex> lk(mu_);
    return blocks_in_use_locked();
}

uint32_t PoolCore::total_blocks() {
    std::lock_guard<std::mutex> lk(mu_);
    return static_cast<uint32_t>(blocks_.size());
}

uint32_t PoolCore::free_physical_blocks() {
    std::lock_guard<std::mutex> lk(mu_);
    return static_cast<uint32_t>(free_handles_.size());
}

uint32_t PoolCore::active_sequences() {
    std::lock_guard<std::mutex> lk(mu_);
    return static_cast<uint32_t>(seqs_.size());
}

uint64_t PoolCore::epoch() {
    std::lock_guard<std::mutex> lk(mu_);
    return epoch_;
}

}  // namespace kcmm
