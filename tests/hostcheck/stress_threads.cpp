// Concurrency stress of the pool core, host only: T threads share one
// PoolCore (the C ABI promises that every call is thread-safe and that a pool
// handle may be shared across threads, include/kcmm.h) and each runs random
// operations on sequences of its own: alloc + register, grow, seq_len
// updates, single forks, beam forks (fork_beams, whose children share the
// parent's pages through a lazily counted base), copy-on-write for append,
// share_prefix, cached prefixes under keys only this thread uses, prefix
// attach, unregister.  Blocks of one thread's sequences are referenced only
// by that thread's sequences and cache entries, so each thread can predict
// every table and every refcount of its own blocks while the others run, and
// checks them (refcount queries also settle the lazy counts of the bases).
// At the end every sequence is unregistered and every cached entry evicted,
// and no block may remain in use; the allocator then hands out every id
// exactly once.  Built with -fsanitize=thread by tests/test_pool_threads.py.
//
// usage: stress_threads THREADS STEPS SEED    (exit 0 and "ok" on success)
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <random>
#include <set>
#include <string>
#include <thread>
#include <vector>

#include "../../lattice_amd/csrc/pool_core.hpp"

using namespace kcmm;

namespace {

struct NullBacking : PageBacking {
    bool reserve(size_t, size_t, std::string*) override { return true; }
    uint64_t region_base(size_t r) const override { return 0x1000000000ull * (r + 1); }
    bool map_superblock(size_t, std::string*) override { return true; }
    void release() override {}
    int kind() const override { return 2; }
};

std::atomic<int> g_fail{0};

#define CHECK(cond, ...)                                              \
    do {                                                              \
        if (!(cond)) {                                                \
            std::fprintf(stderr, "thread %d step %ld line %d: ", tid, step, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);                        \
            std::fprintf(stderr, "\n");                               \
            g_fail = 1;                                               \
            return false;                                             \
        }                                                             \
    } while (0)

constexpr uint32_t kBs = 4;

struct Worker {
    PoolCore* core;
    int tid;
    std::mt19937_64 rng;
    long step = 0;
    std::map<uint32_t, std::vector<uint32_t>> seqs;   // live sequence -> expected table
    std::map<uint32_t, uint32_t> lens;                // live sequence -> seq_len
    std::map<uint64_t, uint32_t> cached;              // this thread's key -> block
    std::vector<uint64_t> chains;                     // key chains registered: first keys
    uint64_t next_key;

    Worker(PoolCore* c, int t, uint64_t seed)
        : core(c), tid(t), rng(seed * 1000003u + t), next_key((static_cast<uint64_t>(t) + 1) << 40) {}

    uint32_t rnd(uint32_t n) { return n ? static_cast<uint32_t>(rng() % n) : 0; }

    uint32_t pick() {
        auto it = seqs.begin();
        std::advance(it, rnd(static_cast<uint32_t>(seqs.size())));
        return it->first;
    }

    // expected refcount of b: occurrences in this thread's tables + cache
    uint32_t expect_rc(uint32_t b) {
        uint32_t n = 0;
        for (auto& kv : seqs)
            for (uint32_t x : kv.second) n += x == b;
        for (auto& kv : cached) n += kv.second == b;
        return n;
    }

    bool check_seq(uint32_t s) {
        std::vector<uint32_t> got;
        CHECK(core->get_block_table(s, &got), "seq %u missing", s);
        CHECK(got == seqs[s], "table of seq %u differs (%zu vs %zu blocks)", s, got.size(),
              seqs[s].size());
        CHECK(core->get_seq_len(s) == lens[s], "seq_len of %u", s);
        return true;
    }

    bool check_refcounts() {
        std::set<uint32_t> ids;
        for (auto& kv : seqs) ids.insert(kv.second.begin(), kv.second.end());
        for (auto& kv : cached) ids.insert(kv.second);
        for (uint32_t b : ids) {
            const uint32_t got = core->refcount(b), want = expect_rc(b);
            CHECK(got == want, "refcount of block %u: %u, expected %u", b, got, want);
        }
        return true;
    }

    bool op_new() {
        if (seqs.size() >= 24) return true;
        const uint32_t n = 1 + rnd(6);
        std::vector<uint32_t> ids(n);
        std::string err;
        if (!core->alloc_blocks(n, ids.data(), &err)) return true;   // pool full: fine
        const uint32_t s = core->register_sequence(ids.data(), n);
        CHECK(s != UINT32_MAX, "register failed");
        for (uint32_t b : ids) CHECK(expect_rc(b) == 0, "fresh block %u already held", b);
        seqs[s] = ids;
        lens[s] = n * kBs - rnd(kBs);
        core->update_seq_len(s, lens[s]);
        return true;
    }

    bool op_grow() {
        if (seqs.empty()) return true;
        const uint32_t s = pick();
        uint32_t b;
        std::string err;
        if (!core->alloc_blocks(1, &b, &err)) return true;
        CHECK(expect_rc(b) == 0, "fresh block %u already held", b);
        CHECK(core->append_block_to_sequence(s, b), "append to %u", s);
        seqs[s].push_back(b);
        lens[s] = static_cast<uint32_t>(seqs[s].size()) * kBs - rnd(kBs);
        core->update_seq_len(s, lens[s]);
        return true;
    }

    bool op_fork() {
        if (seqs.empty() || seqs.size() >= 24) return true;
        const uint32_t s = pick();
        uint32_t c;
        std::string err;
        if (!core->fork_sequence(s, &c, &err)) return true;
        seqs[c] = seqs[s];
        lens[c] = lens[s];
        return check_seq(c);
    }

    bool op_beams() {
        if (seqs.empty() || seqs.size() >= 20) return true;
        std::vector<uint32_t> parents;
        const uint32_t np = 1 + rnd(2);
        std::set<uint32_t> used;
        for (uint32_t i = 0; i < np; ++i) {
            const uint32_t s = pick();
            if (used.insert(s).second) parents.push_back(s);
        }
        const uint32_t width = 2 + rnd(2);
        std::vector<uint32_t> children(parents.size() * (width - 1));
        std::vector<uint32_t> pairs;
        std::string err;
        if (!core->fork_beams(parents.data(), static_cast<uint32_t>(parents.size()), width,
                              children.data(), &pairs, &err))
            return true;   // capacity: all or nothing, nothing changed
        // each child: the parent's table, made private at its next token's
        // page when that page exists (a (src, dst) pair per such child)
        size_t pi = 0;
        for (size_t p = 0; p < parents.size(); ++p) {
            const std::vector<uint32_t> pt = seqs[parents[p]];
            const uint32_t logical = lens[parents[p]] / kBs;
            for (uint32_t k = 0; k + 1 < width; ++k) {
                const uint32_t c = children[p * (width - 1) + k];
                std::vector<uint32_t> t = pt;
                if (logical < t.size()) {
                    CHECK(pi + 1 < pairs.size(), "missing copy pair");
                    CHECK(pairs[pi] == t[logical], "pair source %u, page %u", pairs[pi], t[logical]);
                    t[logical] = pairs[pi + 1];
                    pi += 2;
                }
                seqs[c] = t;
                lens[c] = lens[parents[p]];
                if (!check_seq(c)) return false;
            }
        }
        CHECK(pi == pairs.size(), "%zu pairs, %zu used", pairs.size(), pi);
        return true;
    }

    bool op_cow() {
        if (seqs.empty()) return true;
        const uint32_t s = pick();
        if (seqs[s].empty()) return true;
        const uint32_t logical = rnd(static_cast<uint32_t>(seqs[s].size()));
        uint32_t src = 0, dst = 0;
        std::string err;
        const int r = core->cow_block_for_append(s, logical, &src, &dst, &err);
        if (r < 0) return true;   // capacity
        if (r == 1) {
            CHECK(src == seqs[s][logical], "cow source %u, page %u", src, seqs[s][logical]);
            CHECK(expect_rc(dst) == 0, "cow target %u already held", dst);
            seqs[s][logical] = dst;
        } else {
            CHECK(expect_rc(seqs[s][logical]) == 1, "page %u shared but no copy",
                  seqs[s][logical]);
        }
        return check_seq(s);
    }

    bool op_share() {
        if (seqs.size() < 2) return true;
        const uint32_t a = pick(), b = pick();
        if (a == b || seqs[a].empty()) return true;
        const uint32_t n = 1 + rnd(static_cast<uint32_t>(seqs[a].size()));
        std::vector<uint32_t> out(n);
        std::string err;
        if (!core->share_prefix(a, b, n, out.data(), &err)) return true;
        for (uint32_t i = 0; i < n; ++i) {
            CHECK(out[i] == seqs[a][i], "shared block %u", i);
            seqs[b].push_back(seqs[a][i]);
        }
        return check_seq(b);
    }

    bool op_cache() {
        if (seqs.empty()) return true;
        const uint32_t s = pick();
        const uint32_t full = lens[s] / kBs;
        if (full == 0) return true;
        const uint32_t n = 1 + rnd(full);
        std::vector<uint64_t> keys(n);
        for (uint32_t i = 0; i < n; ++i) keys[i] = next_key + i;
        uint32_t added = 0;
        std::string err;
        CHECK(core->prefix_register(s, keys.data(), n, &added, &err), "prefix_register: %s",
              err.c_str());
        CHECK(added == n, "added %u of %u fresh keys", added, n);
        for (uint32_t i = 0; i < n; ++i) cached[keys[i]] = seqs[s][i];
        chains.push_back(next_key);
        next_key += n + 1;   // a gap: chains never run into each other
        return true;
    }

    bool op_attach() {
        if (seqs.empty() || chains.empty()) return true;
        const uint32_t dst = pick();
        const uint64_t k0 = chains[rnd(static_cast<uint32_t>(chains.size()))];
        std::vector<uint64_t> keys;
        for (uint64_t k = k0; cached.count(k); ++k) keys.push_back(k);
        if (keys.empty()) return true;
        std::vector<uint32_t> blocks(keys.size());
        uint32_t matched = 0;
        std::string err;
        if (!core->prefix_attach(dst, keys.data(), static_cast<uint32_t>(keys.size()),
                                 blocks.data(), &matched, &err))
            return true;   // the table is full
        CHECK(matched == keys.size(), "matched %u of %zu own keys", matched, keys.size());
        for (uint32_t i = 0; i < matched; ++i) {
            CHECK(blocks[i] == cached[keys[i]], "attached block %u", i);
            seqs[dst].push_back(blocks[i]);
        }
        return check_seq(dst);
    }

    bool op_unregister() {
        if (seqs.empty()) return true;
        const uint32_t s = pick();
        core->unregister_sequence(s);
        seqs.erase(s);
        lens.erase(s);
        // (sequence indices are not reused: has_sequence stays true for an
        // index once handed out, registered or not)
        return true;
    }

    bool run(long steps) {
        for (step = 0; step < steps && !g_fail; ++step) {
            bool ok = true;
            switch (rnd(20)) {
                case 0: case 1: case 2: ok = op_new(); break;
                case 3: case 4: ok = op_grow(); break;
                case 5: case 6: ok = op_fork(); break;
                case 7: case 8: case 9: ok = op_beams(); break;
                case 10: case 11: ok = op_cow(); break;
                case 12: ok = op_share(); break;
                case 13: ok = op_cache(); break;
                case 14: ok = op_attach(); break;
                case 15: case 16: case 17: ok = op_unregister(); break;
                case 18: if (!seqs.empty()) ok = check_seq(pick()); break;
                default: ok = rnd(4) == 0 ? check_refcounts() : true; break;
            }
            if (!ok) return false;
        }
        if (!check_refcounts()) return false;
        for (auto& kv : seqs) core->unregister_sequence(kv.first);
        seqs.clear();
        lens.clear();
        for (auto& kv : cached) CHECK(core->refcount(kv.second) >= 1, "cached block %u freed", kv.second);
        return true;
    }
};

}  // namespace

int main(int argc, char** argv) {
    const int threads = argc > 1 ? std::atoi(argv[1]) : 8;
    const long steps = argc > 2 ? std::atol(argv[2]) : 2000;
    const uint64_t seed = argc > 3 ? std::strtoull(argv[3], nullptr, 10) : 1;
    PoolGeometry g;
    g.block_size = kBs;
    g.num_layers = 1;
    g.kv_heads = 1;
    g.head_dim = 8;
    g.max_batch = 1024;
    g.max_seq_len = 4096;
    g.dtype = kBF16;
    std::string err;
    if (!g.compute(&err)) {
        std::fprintf(stderr, "geometry: %s\n", err.c_str());
        return 2;
    }
    PoolCore core(g, std::unique_ptr<PageBacking>(new NullBacking()));
    std::vector<Worker> workers;
    for (int t = 0; t < threads; ++t) workers.emplace_back(&core, t, seed);
    // all threads start together, so their calls interleave from the first
    std::atomic<int> ready{0};
    std::vector<std::thread> th;
    for (int t = 0; t < threads; ++t)
        th.emplace_back([&, t] {
            ready.fetch_add(1);
            while (ready.load() < threads) std::this_thread::yield();
            workers[t].run(steps);
        });
    for (auto& x : th) x.join();
    if (g_fail) return 1;
    // every cached entry released: nothing may remain in use
    while (core.prefix_evict(1u << 20) > 0) {}
    if (core.blocks_in_use() != 0) {
        std::fprintf(stderr, "after teardown: %u blocks in use\n", core.blocks_in_use());
        return 1;
    }
    // the free list holds every id exactly once
    const uint32_t total = core.total_blocks();
    std::vector<uint32_t> ids(total);
    if (total && !core.alloc_blocks(total, ids.data(), &err)) {
        std::fprintf(stderr, "cannot allocate all %u blocks: %s\n", total, err.c_str());
        return 1;
    }
    std::set<uint32_t> uniq(ids.begin(), ids.end());
    if (uniq.size() != total) {
        std::fprintf(stderr, "free list: %zu distinct of %u\n", uniq.size(), total);
        return 1;
    }
    std::printf("ok %d threads x %ld steps, %u blocks\n", threads, steps, total);
    return 0;
}
