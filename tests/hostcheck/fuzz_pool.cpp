// Differential fuzz of the pool core's block tables and reference counts
// against the oracle pool (oracle/oracle.c), host only.  Random sequences of
// alloc / register / append / seq_len updates / beam forks (fork_beams, which
// shares a parent's table through a lazily counted base) / single forks /
// copy-on-write / unregister / frees (also of blocks a table still holds) /
// share_prefix / cached-prefix references / append privacy checks, with the
// block tables compared after every step and every refcount, the next ids
// the allocator hands out and the privacy verdicts compared at random
// points (a refcount query makes the lazy counts exact, so checks are kept
// sparse to leave the lazy state in place between them).
//
// usage: fuzz_pool SEED STEPS    (exit 0 and "ok" on agreement)
#include <cstdio>
#include <cstdlib>
#include <random>
#include <set>
#include <string>
#include <vector>

#include "../../lattice_amd/csrc/pool_core.hpp"
#include "../../oracle/oracle.h"

using namespace kcmm;

namespace {

struct NullBacking : PageBacking {
    bool reserve(size_t, size_t, std::string*) override { return true; }
    uint64_t region_base(size_t r) const override { return 0x1000000000ull * (r + 1); }
    bool map_superblock(size_t, std::string*) override { return true; }
    void release() override {}
    int kind() const override { return 2; }
};

int g_fail = 0;
#define CHECK(cond, ...)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            std::fprintf(stderr, "MISMATCH line %d: ", __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);             \
            std::fprintf(stderr, "\n");                    \
            g_fail = 1;                                    \
            return;                                        \
        }                                                  \
    } while (0)

struct Fuzz {
    static constexpr size_t kBs = 4;
    PoolGeometry g;
    PoolCore* core = nullptr;
    OPool* op = nullptr;
    std::mt19937_64 rng;
    uint32_t nseqs = 0;
    std::vector<uint32_t> live;            // registered and not unregistered
    std::set<uint64_t> cached_keys;
    uint64_t next_key = 1;
    long step = 0;

    explicit Fuzz(uint64_t seed) : rng(seed) {
        g.block_size = kBs;
        g.num_layers = 1;
        g.kv_heads = 1;
        g.head_dim = 8;
        g.max_batch = 64;
        g.max_seq_len = 2048;
        g.dtype = kBF16;
        std::string err;
        if (!g.compute(&err)) {
            std::fprintf(stderr, "geometry: %s\n", err.c_str());
            std::exit(2);
        }
        core = new PoolCore(g, std::unique_ptr<PageBacking>(new NullBacking()));
        op = opool_new(kBs, 1, 1, 8, 64, 2048, 1, 1);
    }
    ~Fuzz() {
        delete core;
        opool_delete(op);
    }

    uint32_t rnd(uint32_t n) { return n ? static_cast<uint32_t>(rng() % n) : 0; }

    std::vector<uint32_t> tbuf = std::vector<uint32_t>(1 << 16);
    std::vector<uint32_t> otable(uint32_t s) {
        uint32_t cnt = 0;
        if (opool_block_table(op, s, tbuf.data(), static_cast<uint32_t>(tbuf.size()), &cnt))
            return {};
        return std::vector<uint32_t>(tbuf.begin(), tbuf.begin() + cnt);
    }

    std::vector<uint32_t> ids_in_use() {
        std::vector<uint32_t> v;
        const uint32_t n = core->total_blocks();
        for (uint32_t i = 0; i < n; ++i)
            if (opool_refcount(op, i) > 0) v.push_back(i);
        return v;
    }

    void check_tables() {   // the live sequences, and a few released ones
        std::vector<uint32_t> which = live;
        for (int i = 0; i < 4 && nseqs; ++i) which.push_back(rnd(nseqs));
        for (uint32_t s : which) {
            std::vector<uint32_t> a;
            core->get_block_table(s, &a);
            CHECK(a == otable(s), "step %ld: table of seq %u differs", step, s);
            CHECK(core->get_seq_len(s) == opool_seq_len(op, s), "step %ld: seq_len of %u", step, s);
        }
    }

    void check_refcounts() {
        const uint32_t n = core->total_blocks();
        for (uint32_t i = 0; i < n + 2; ++i)
            CHECK(core->refcount(i) == opool_refcount(op, i), "step %ld: refcount of %u: %u vs %u",
                  step, i, core->refcount(i), opool_refcount(op, i));
    }

    void check_free_order() {
        const uint32_t k = 1 + rnd(3);
        std::vector<uint32_t> a(k), b(k);
        std::string err;
        const bool ca = core->alloc_blocks(k, a.data(), &err);
        const bool cb = opool_alloc(op, k, b.data()) == 0;
        CHECK(ca == cb, "step %ld: probe alloc outcome", step);
        if (!ca) return;
        CHECK(a == b, "step %ld: probe alloc ids differ", step);
        core->free_blocks(a.data(), k);
        opool_release(op, b.data(), k);
    }

    uint32_t pick_live() { return live[rnd(static_cast<uint32_t>(live.size()))]; }

    void op_alloc_register() {
        const uint32_t n = 1 + rnd(12);
        std::vector<uint32_t> a(n), b(n);
        std::string err;
        const bool ca = core->alloc_blocks(n, a.data(), &err);
        const bool cb = opool_alloc(op, n, b.data()) == 0;
        CHECK(ca == cb, "step %ld: alloc outcome", step);
        if (!ca) return;
        CHECK(a == b, "step %ld: alloc ids differ", step);
        const uint32_t s = core->register_sequence(a.data(), n);
        const uint32_t t = opool_register(op, b.data(), n);
        CHECK(s == t, "step %ld: register idx %u vs %u", step, s, t);
        const uint32_t len = static_cast<uint32_t>(n * kBs - rnd(kBs));
        core->update_seq_len(s, len);
        opool_update_seq_len(op, s, len);
        live.push_back(s);
        ++nseqs;
    }

    void op_set_len() {   // any length within the table, shorter ones included
        const uint32_t s = pick_live();
        const uint32_t len = rnd(static_cast<uint32_t>(otable(s).size() * kBs) + 1);
        core->update_seq_len(s, len);
        opool_update_seq_len(op, s, len);
    }

    void op_grow() {   // a sequence appends tokens, opening pages as it goes
        const uint32_t s = pick_live();
        const uint32_t add = rnd(10) == 0 ? kBs * (40 + rnd(60)) : 1 + rnd(3 * kBs);
        uint32_t len = core->get_seq_len(s) + add;
        std::vector<uint32_t> t;
        core->get_block_table(s, &t);
        while (t.size() * kBs < len) {
            uint32_t a = 0, b = 0;
            std::string err;
            const bool ca = core->alloc_blocks(1, &a, &err);
            const bool cb = opool_alloc(op, 1, &b) == 0;
            CHECK(ca == cb && (!ca || a == b), "step %ld: grow alloc", step);
            if (!ca) {
                len = static_cast<uint32_t>(t.size() * kBs);
                break;
            }
            core->append_block_to_sequence(s, a);
            opool_append_block(op, s, b);
            t.push_back(a);
        }
        core->update_seq_len(s, len);
        opool_update_seq_len(op, s, len);
    }

    void op_beam_fork() {
        // Parents whose tables hold only blocks in use: a table that still
        // lists a freed block (a caller's misuse) would see it reallocated as
        // a child's new page within the call, and the batched fork takes its
        // references before any page is allocated while fork + CoW one child
        // at a time would count the reallocated block for the later children.
        std::vector<uint32_t> ok_parents;
        for (uint32_t s : live) {
            bool clean = true;
            for (uint32_t id : otable(s)) clean &= opool_refcount(op, id) > 0;
            if (clean) ok_parents.push_back(s);
        }
        if (ok_parents.empty()) return;
        const uint32_t np = 1 + rnd(std::min<uint32_t>(6, static_cast<uint32_t>(ok_parents.size())));
        std::vector<uint32_t> parents;
        for (uint32_t i = 0; i < np; ++i)
            parents.push_back(ok_parents[rnd(static_cast<uint32_t>(ok_parents.size()))]);
        const uint32_t width = 1 + rnd(4), forks = width - 1;
        // a parent whose next-token page was freed under it is refused
        bool refused = false;
        for (uint32_t p : parents) {
            const std::vector<uint32_t> t = otable(p);
            const uint32_t logical = opool_seq_len(op, p) / kBs;
            if (forks > 0 && logical < t.size() && opool_refcount(op, t[logical]) == 0) refused = true;
        }
        std::vector<uint32_t> children(np * forks + 1), pairs;
        std::string err;
        if (std::getenv("FUZZ_TRACE")) {
            std::fprintf(stderr, "  beam fork width %u parents:", width);
            for (uint32_t p : parents) {
                std::fprintf(stderr, " %u(len %u:", p, opool_seq_len(op, p));
                for (uint32_t id : otable(p)) std::fprintf(stderr, " %u", id);
                std::fprintf(stderr, ")");
            }
            std::fprintf(stderr, "\n  rc before (core/oracle):");
            for (uint32_t id : otable(parents.back()))
                std::fprintf(stderr, " %u:%u/%u", id, core->refcount(id), opool_refcount(op, id));
            std::fprintf(stderr, "\n");
        }
        const bool ok = core->fork_beams(parents.data(), np, width, children.data(), &pairs, &err);
        if (std::getenv("FUZZ_TRACE")) {
            std::fprintf(stderr, "  pairs:");
            for (size_t q = 0; q < pairs.size(); q += 2) std::fprintf(stderr, " %u->%u", pairs[q], pairs[q + 1]);
            std::fprintf(stderr, "\n");
        }
        CHECK(ok != refused, "step %ld: fork_beams outcome %d (%s)", step, ok, err.c_str());
        if (!ok) return;
        std::vector<uint32_t> och, opairs;
        for (uint32_t p : parents) {
            for (uint32_t c = 0; c < forks; ++c) {
                uint32_t ch = 0;
                opool_fork(op, p, &ch);
                och.push_back(ch);
                const uint32_t logical = opool_seq_len(op, ch) / kBs;
                if (logical < otable(ch).size()) {
                    uint32_t a = 0, b = 0;
                    const int r = opool_cow(op, ch, logical, &a, &b);
                    if (r == 1) {
                        opairs.push_back(a);
                        opairs.push_back(b);
                    }
                }
            }
        }
        children.resize(np * forks);
        if (std::getenv("FUZZ_TRACE")) {
            std::fprintf(stderr, "  oracle pairs:");
            for (size_t q = 0; q < opairs.size(); q += 2) std::fprintf(stderr, " %u->%u", opairs[q], opairs[q + 1]);
            std::fprintf(stderr, "\n  rc after (core/oracle):");
            for (uint32_t id : otable(parents.back()))
                std::fprintf(stderr, " %u:%u/%u", id, core->refcount(id), opool_refcount(op, id));
            std::fprintf(stderr, "\n");
        }
        CHECK(children == och, "step %ld: children differ", step);
        CHECK(pairs == opairs, "step %ld: CoW pairs differ (%zu vs %zu)", step, pairs.size(),
              opairs.size());
        nseqs += np * forks;
        for (uint32_t c : children) live.push_back(c);
    }

    void op_fork_one() {
        const uint32_t s = pick_live();
        uint32_t a = 0, b = 0;
        std::string err;
        core->fork_sequence(s, &a, &err);
        opool_fork(op, s, &b);
        CHECK(a == b, "step %ld: fork_sequence idx", step);
        live.push_back(a);
        ++nseqs;
    }

    void op_cow() {
        const uint32_t s = pick_live();
        const uint32_t n = static_cast<uint32_t>(otable(s).size());
        const uint32_t logical = rnd(n + 1);
        uint32_t a0 = 0, a1 = 0, b0 = 0, b1 = 0;
        std::string err;
        const int ra = core->cow_block_for_append(s, logical, &a0, &a1, &err);
        const int rb = opool_cow(op, s, logical, &b0, &b1);
        CHECK(ra == rb, "step %ld: cow result %d vs %d", step, ra, rb);
        if (ra == 1) CHECK(a0 == b0 && a1 == b1, "step %ld: cow pair", step);
    }

    void op_unregister() {
        const uint32_t i = rnd(static_cast<uint32_t>(live.size()));
        const uint32_t s = live[i];
        core->unregister_sequence(s);
        opool_unregister(op, s);
        live.erase(live.begin() + i);
    }

    void op_free() {   // frees that may hit blocks a table still holds
        std::vector<uint32_t> use = ids_in_use();
        if (use.empty()) return;
        const uint32_t k = 1 + rnd(3);
        std::vector<uint32_t> ids;
        for (uint32_t i = 0; i < k; ++i) ids.push_back(use[rnd(static_cast<uint32_t>(use.size()))]);
        core->free_blocks(ids.data(), ids.size());
        opool_release(op, ids.data(), static_cast<uint32_t>(ids.size()));
    }

    void op_share_prefix() {
        const uint32_t src = pick_live(), dst = pick_live();
        const uint32_t n = rnd(static_cast<uint32_t>(otable(src).size()) + 1);
        std::vector<uint32_t> a(n + 1), b(n + 1);
        std::string err;
        const bool ca = core->share_prefix(src, dst, n, a.data(), &err);
        const bool cb = opool_share_prefix(op, src, dst, n, b.data()) == 0;
        CHECK(ca == cb, "step %ld: share_prefix outcome", step);
        if (ca) CHECK(std::vector<uint32_t>(a.begin(), a.begin() + n) ==
                          std::vector<uint32_t>(b.begin(), b.begin() + n),
                      "step %ld: share_prefix ids", step);
    }

    void op_prefix_ref() {   // cached-prefix references (one per new key)
        const uint32_t s = pick_live();
        const std::vector<uint32_t> t = otable(s);
        const uint32_t full = opool_seq_len(op, s) / kBs;
        const uint32_t n = rnd(std::min<uint32_t>(full, static_cast<uint32_t>(t.size())) + 1);
        bool all_in_use = true;
        for (uint32_t i = 0; i < n; ++i) all_in_use &= opool_refcount(op, t[i]) > 0;
        std::vector<uint64_t> keys;
        for (uint32_t i = 0; i < n; ++i) keys.push_back(next_key++);
        uint32_t added = 0;
        std::string err;
        const bool ok = core->prefix_register(s, keys.data(), n, &added, &err);
        CHECK(ok == all_in_use, "step %ld: prefix_register outcome", step);
        if (!ok) return;
        for (uint32_t i = 0; i < n; ++i) opool_incref(op, t[i]);
        CHECK(added == n, "step %ld: prefix entries added", step);
    }

    void op_append_check() {   // is the next-token page private?
        const uint32_t s = pick_live();
        const std::vector<uint32_t> t = otable(s);
        const uint32_t pos = rnd(static_cast<uint32_t>(t.size() * kBs) + 1);
        std::vector<RowDst> out;
        std::string err;
        const bool ok = core->resolve_positions(&s, &pos, 1, &out, &err);
        const uint32_t lb = pos / kBs;
        const bool want = lb < t.size() && opool_refcount(op, t[lb]) == 1;
        CHECK(ok == want, "step %ld: append privacy of seq %u pos %u: %d vs %d", step, s, pos,
              ok, want);
    }

    void run(long steps) {
        for (step = 0; step < steps && !g_fail; ++step) {
            const uint32_t r = rnd(100);
            if (live.size() < 3 || r < 10) op_alloc_register();
            else if (r < 20) op_grow();
            else if (r < 22) op_set_len();
            else if (r < 44) op_beam_fork();
            else if (r < 48) op_fork_one();
            else if (r < 56) op_cow();
            else if (r < 72) op_unregister();
            else if (r < 76) op_free();
            else if (r < 80) op_share_prefix();
            else if (r < 84) op_prefix_ref();
            else op_append_check();
            if (g_fail) break;
            if (std::getenv("FUZZ_TRACE")) std::fprintf(stderr, "step %ld op %u\n", step, r);
            check_tables();
            if (std::getenv("FUZZ_FULL") || rnd(8) == 0) check_refcounts();
            if (rnd(16) == 0) check_free_order();
            // keep the pool from filling: drop a few sequences now and then
            while (live.size() > 40 && !g_fail) op_unregister();
        }
        if (!g_fail) {
            check_refcounts();
            check_free_order();
        }
    }
};

}  // namespace

int main(int argc, char** argv) {
    const uint64_t seed = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1;
    const long steps = argc > 2 ? std::strtol(argv[2], nullptr, 10) : 2000;
    Fuzz f(seed);
    f.run(steps);
    if (g_fail) return 1;
    std::printf("ok seed %llu steps %ld seqs %u\n", static_cast<unsigned long long>(seed), steps,
                f.nseqs);
    return 0;
}
