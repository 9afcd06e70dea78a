// Eviction policies and swap slots (ref src/kcmm/tiering.rs:25-643).
#include "tiering.hpp"

#include <algorithm>

namespace kcmm {

namespace {

long find(const std::vector<PageHandle>& l, PageHandle h) {
    auto it = std::find(l.begin(), l.end(), h);
    return it == l.end() ? -1 : static_cast<long>(it - l.begin());
}

// distance of the last occurrence from the end (a handle re-allocated while
// still listed appears twice; ref tiering.rs:355-356 ranks by iter().rev())
long rpos(const std::vector<PageHandle>& l, PageHandle h) {
    for (size_t j = l.size(); j-- > 0;)
        if (l[j] == h) return static_cast<long>(l.size() - 1 - j);
    return -1;
}

// append at the LRU end, dropping the oldest entries beyond cap
// (ref tiering.rs:276-279, 286-289)
void push_bounded(std::vector<PageHandle>& l, PageHandle h, size_t cap) {
    l.push_back(h);
    while (l.size() > cap) l.erase(l.begin());
}

}  // namespace

EvictionPolicy::EvictionPolicy(PolicyKind kind, size_t arc_capacity)
    : kind_(kind), arc_cap_(arc_capacity > 0 ? arc_capacity : 1) {}

const char* EvictionPolicy::name() const {
    switch (kind_) {
        case PolicyKind::kLfu: return "lfu";
        case PolicyKind::kFifo: return "fifo";
        case PolicyKind::kArc: return "arc";
        case PolicyKind::kSinkWindow: return "sink_window";
        default: return "lru";
    }
}

// ref tiering.rs:269-296
void EvictionPolicy::arc_replace() {
    if (!t1_.empty() && (t1_.size() > arc_p_ || t2_.empty())) {
        const PageHandle v = t1_.back();
        t1_.pop_back();
        push_bounded(b1_, v, arc_cap_);
    } else if (!t2_.empty()) {
        const PageHandle v = t2_.back();
        t2_.pop_back();
        push_bounded(b2_, v, arc_cap_);
    }
}

void EvictionPolicy::on_allocate(PageHandle h) {
    switch (kind_) {
        case PolicyKind::kLfu:
            key_[h] = 1;
            break;
        case PolicyKind::kArc: {
            // ref tiering.rs:299-337: a ghost hit moves the target and
            // enters T2, anything else enters T1; then trim to capacity
            const long i1 = find(b1_, h);
            if (i1 >= 0) b1_.erase(b1_.begin() + i1);
            const long i2 = find(b2_, h);
            if (i2 >= 0) b2_.erase(b2_.begin() + i2);
            if (i1 >= 0) {
                const size_t d = std::max<size_t>(
                    std::max<size_t>(b2_.size(), 1) / std::max<size_t>(b1_.size(), 1), 1);
                arc_p_ = std::min(arc_p_ + d, arc_cap_);
                t2_.insert(t2_.begin(), h);
            } else if (i2 >= 0) {
                const size_t d = std::max<size_t>(
                    std::max<size_t>(b1_.size(), 1) / std::max<size_t>(b2_.size(), 1), 1);
                arc_p_ = arc_p_ > d ? arc_p_ - d : 0;
                t2_.insert(t2_.begin(), h);
            } else {
                t1_.insert(t1_.begin(), h);
            }
            while (t1_.size() + t2_.size() > arc_cap_) arc_replace();
            break;
        }
        default:  // lru, fifo, sink_window: allocation time
            key_[h] = ++clock_;
            break;
    }
}

void EvictionPolicy::on_access(PageHandle h) {
    switch (kind_) {
        case PolicyKind::kFifo:
            break;  // the allocation time is the only key (ref tiering.rs:203-206)
        case PolicyKind::kLfu:
            ++key_[h];  // or_insert(0) += 1 (ref tiering.rs:147-150)
            break;
        case PolicyKind::kArc: {
            // ref tiering.rs:376-393: T1 -> head of T2; T2 -> head of T2
            const long i1 = find(t1_, h);
            if (i1 >= 0) {
                t1_.erase(t1_.begin() + i1);
                t2_.insert(t2_.begin(), h);
                break;
            }
            const long i2 = find(t2_, h);
            if (i2 >= 0) {
                t2_.erase(t2_.begin() + i2);
                t2_.insert(t2_.begin(), h);
            }
            break;
        }
        default:
            key_[h] = ++clock_;
            break;
    }
}

void EvictionPolicy::on_evict(PageHandle h) {
    if (kind_ != PolicyKind::kArc) {
        key_.erase(h);
        return;
    }
    // ref tiering.rs:395-424: the entry becomes a ghost of its list
    const long i1 = find(t1_, h);
    if (i1 >= 0) {
        t1_.erase(t1_.begin() + i1);
        if (find(b1_, h) < 0) push_bounded(b1_, h, arc_cap_);
        return;
    }
    const long i2 = find(t2_, h);
    if (i2 >= 0) {
        t2_.erase(t2_.begin() + i2);
        if (find(b2_, h) < 0) push_bounded(b2_, h, arc_cap_);
    }
}

std::vector<PageHandle> EvictionPolicy::select_victims(const std::vector<PageHandle>& cands,
                                                       size_t count) const {
    std::vector<std::pair<PageHandle, uint64_t>> scored;
    if (cands.empty() || count == 0) return {};
    scored.reserve(cands.size());
    for (const PageHandle& h : cands) {
        if (kind_ == PolicyKind::kArc) {
            // ref tiering.rs:339-374: position from the LRU end of T1, then T2
            const long p1 = rpos(t1_, h);
            const long p2 = p1 < 0 ? rpos(t2_, h) : -1;
            uint64_t score;
            if (p1 >= 0) score = static_cast<uint64_t>(p1);
            else if (p2 >= 0) score = t1_.size() + static_cast<uint64_t>(p2);
            else score = t1_.size() + t2_.size() + 1;
            scored.emplace_back(h, score);
        } else {
            auto it = key_.find(h);
            if (it != key_.end()) scored.emplace_back(h, it->second);
        }
    }
    std::stable_sort(scored.begin(), scored.end(),
                     [](const auto& a, const auto& b) { return a.second < b.second; });
    if (scored.size() > count) scored.resize(count);
    std::vector<PageHandle> out;
    out.reserve(scored.size());
    for (const auto& s : scored) out.push_back(s.first);
    return out;
}

SwapSlots::SwapSlots(uint64_t total) {
    if (total > 0) free_.emplace_back(0, total);
}

// ref tiering.rs:578-605
bool SwapSlots::allocate(uint64_t size, uint64_t* offset) {
    if (size == 0 || free_.empty()) return false;
    size_t best = free_.size();
    uint64_t best_len = UINT64_MAX;
    for (size_t i = 0; i < free_.size(); ++i) {
        const uint64_t len = free_[i].second - free_[i].first;
        if (len >= size && len < best_len) {
            best_len = len;
            best = i;
        }
    }
    if (best == free_.size()) return false;
    *offset = free_[best].first;
    if (best_len == size) free_.erase(free_.begin() + static_cast<long>(best));
    else free_[best].first += size;
    return true;
}

// ref tiering.rs:607-642
void SwapSlots::free(uint64_t offset, uint64_t size) {
    if (size == 0) return;
    const uint64_t end = offset + size;
    size_t at = 0;
    while (at < free_.size() && free_[at].first <= offset) ++at;
    const bool prev = at > 0 && free_[at - 1].second == offset;
    const bool next = at < free_.size() && free_[at].first == end;
    if (prev && next) {
        free_[at - 1].second = free_[at].second;
        free_.erase(free_.begin() + static_cast<long>(at));
    } else if (prev) {
        free_[at - 1].second = end;
    } else if (next) {
        free_[at].first = offset;
    } else {
        free_.insert(free_.begin() + static_cast<long>(at), {offset, end});
    }
}

}  // namespace kcmm
