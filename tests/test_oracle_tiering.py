"""The oracle's tiering restatement pinned to the reference's own unit tests:
eviction policies (ref tiering.rs:2106-2465, 3796-4025), the swap-slot
allocator (ref tiering.rs:2575-2738) and the pool-level evict / restore
transitions (ref tiering.rs:2743-3420, pool.rs:2120-2175), each with the
reference test it restates named in the docstring.  Timestamps are the
oracle's logical clock, so the reference's sleeps between events are not
needed."""
import oracle as O


def h(i, sb=0):
    return (sb, i)


# ---- LRU (ref tiering.rs:2106-2231) ----

def test_lru_oldest_first():
    p = O.OracleTier("lru")
    for i in range(3):
        p.on_allocate(h(i))
    assert p.select_victims([h(0), h(1), h(2)], 2) == [h(0), h(1)]   # :2174-2190


def test_lru_respects_count_and_candidates():
    p = O.OracleTier("lru")
    for i in range(10):
        p.on_allocate(h(i))
    assert p.select_victims([h(i) for i in range(10)], 3) == [h(0), h(1), h(2)]   # :2193-2206
    q = O.OracleTier("lru")
    q.on_allocate(h(0))
    q.on_allocate(h(1))
    assert len(q.select_victims([h(0), h(1)], 10)) == 2                           # :2209-2216


def test_lru_untracked_skipped_and_access_refreshes():
    p = O.OracleTier("lru")
    p.on_allocate(h(0))
    assert p.select_victims([h(0), h(1)], 2) == [h(0)]                             # :2219-2228
    p.on_allocate(h(1))
    p.on_access(h(0))                                                             # :2137-2146
    assert p.select_victims([h(0), h(1)], 2) == [h(1), h(0)]
    p.on_evict(h(1))                                                              # :2149-2156
    assert p.select_victims([h(0), h(1)], 2) == [h(0)]
    assert p.select_victims([], 5) == [] and p.select_victims([h(0)], 0) == []     # :2159-2171


def test_lru_on_access_inserts_untracked():
    p = O.OracleTier("lru")
    p.on_access(h(4))                                                             # :2129-2134
    assert p.select_victims([h(4)], 1) == [h(4)]


# ---- LFU (ref tiering.rs:2233-2350) ----

def test_lfu_least_frequent_first():
    p = O.OracleTier("lfu")
    p.on_access(h(0))
    for _ in range(3):
        p.on_access(h(1))
    for _ in range(2):
        p.on_access(h(2))
    assert p.select_victims([h(0), h(1), h(2)], 3) == [h(0), h(2), h(1)]          # :2287-2309


def test_lfu_allocate_sets_one_access_increments():
    p = O.OracleTier("lfu")
    p.on_allocate(h(0))                                                           # :2242-2248
    p.on_allocate(h(1))
    p.on_access(h(0))                                                             # :2250-2259
    assert p.select_victims([h(0), h(1)], 2) == [h(1), h(0)]
    # equal counts keep candidate order
    p.on_access(h(1))
    assert p.select_victims([h(1), h(0)], 2) == [h(1), h(0)]
    p.on_evict(h(0))                                                              # :2262-2271
    assert p.select_victims([h(0), h(1)], 2) == [h(1)]


# ---- FIFO (ref tiering.rs:2352-2465) ----

def test_fifo_earliest_allocated_and_access_is_noop():
    p = O.OracleTier("fifo")
    p.on_access(h(9))                                                             # :2368-2374
    assert p.select_victims([h(9)], 1) == []
    for i in range(3):
        p.on_allocate(h(i))
    p.on_access(h(0))                                                             # :2376-2385
    assert p.select_victims([h(0), h(1), h(2)], 2) == [h(0), h(1)]                # :2410-2426
    p.on_evict(h(0))                                                              # :2387-2394
    assert p.select_victims([h(0), h(1), h(2)], 3) == [h(1), h(2)]


# ---- ARC (ref tiering.rs:3796-3911) ----

def test_arc_first_access_t1_second_t2():
    p = O.OracleTier("arc", arc_capacity=10)
    p.on_allocate(h(0))
    assert p.select_victims([h(0)], 1) == [h(0)]                                  # :3802-3810
    assert p.arc_list("t1") == [h(0)]
    p.on_access(h(0))                                                             # :3813-3823
    assert p.arc_list("t1") == [] and p.arc_list("t2") == [h(0)]
    assert p.select_victims([], 1) == []


def test_arc_t1_before_t2():
    p = O.OracleTier("arc", arc_capacity=10)
    p.on_allocate(h(0))
    p.on_allocate(h(1))
    p.on_access(h(1))
    p.on_allocate(h(2))
    assert p.select_victims([h(0), h(1), h(2)], 1) == [h(0)]                      # :3826-3844
    assert p.select_victims([h(0), h(1), h(2)], 3) == [h(0), h(2), h(1)]


def test_arc_evict_populates_ghost():
    p = O.OracleTier("arc", arc_capacity=3)
    p.on_allocate(h(0))
    p.on_allocate(h(1))
    p.on_access(h(1))
    p.on_allocate(h(2))
    assert p.arc_list("t1") == [h(2), h(0)] and p.arc_list("t2") == [h(1)]        # :3853-3857
    p.on_evict(h(0))
    assert p.arc_list("b1") == [h(0)]
    p.on_allocate(h(0))                                                           # B1 ghost hit
    assert p.arc_list("b1") == [] and p.arc_list("t2") == [h(0), h(1)]
    assert p.arc_p() == 1
    assert len(p.select_victims([h(0)], 1)) == 1                                  # :3847-3868


def test_arc_capacity_enforcement():
    p = O.OracleTier("arc", arc_capacity=2)
    for i in range(3):
        p.on_allocate(h(i))
    assert p.arc_list("b1") == [h(0)] and p.arc_list("t1") == [h(2), h(1)]
    v = p.select_victims([h(0), h(1), h(2)], 3)                                   # :3871-3887
    assert len(v) == 3 and v[2] == h(0)
    assert p.select_victims([h(0)], 0) == []                                      # :3897-3903


def test_sink_window_without_registrations_is_lru():
    """The reference pool never registers block positions with the
    sink-window policy (register_block appears only in its tests), so through
    the pool it ranks exactly as LRU (ref tiering.rs:492-528)."""
    a, b = O.OracleTier("sink_window"), O.OracleTier("lru")
    for p in (a, b):
        for i in range(5):
            p.on_allocate(h(i))
        p.on_access(h(1))
        p.on_evict(h(3))
    c = [h(i) for i in range(5)]
    assert a.select_victims(c, 4) == b.select_victims(c, 4) == [h(0), h(2), h(4), h(1)]


# ---- swap-slot allocator (ref tiering.rs:2575-2738) ----

def test_slots_basic():
    assert O.OracleTier(swap_size=0).free_ranges() == []                         # :2582-2586
    s = O.OracleTier(swap_size=1024)
    assert s.free_ranges() == [(0, 1024)]                                         # :2589-2593
    assert s.allocate(1024) == 0 and s.free_ranges() == []                        # :2596-2601
    s = O.OracleTier(swap_size=1024)
    assert s.allocate(256) == 0 and s.free_ranges() == [(256, 1024)]              # :2604-2610
    s = O.OracleTier(swap_size=1024)
    assert s.allocate(0) is None and s.free_ranges() == [(0, 1024)]               # :2613-2619
    s = O.OracleTier(swap_size=64)
    s.allocate(64)
    assert s.allocate(1) is None                                                  # :2622-2626


def test_slots_best_fit():
    # free ranges [0..64, 128..256, 320..640] (ref :2629-2640), built by allocations
    s = O.OracleTier(swap_size=640)
    offs = [s.allocate(n) for n in (64, 64, 128, 64, 320)]
    assert offs == [0, 64, 128, 256, 320]
    for o, n in ((0, 64), (128, 128), (320, 320)):
        s.free(o, n)
    assert s.free_ranges() == [(0, 64), (128, 256), (320, 640)]
    assert s.allocate(48) == 0 and s.free_ranges()[0] == (48, 64)


def test_slots_merging():
    s = O.OracleTier(swap_size=1024)
    a, b = s.allocate(256), s.allocate(256)
    s.free(a, 256)
    assert s.free_ranges() == [(0, 256), (512, 1024)]                              # :2654-2667
    s.free(b, 256)
    assert s.free_ranges() == [(0, 1024)]
    s = O.OracleTier(swap_size=1024)
    s.allocate(256), s.allocate(256)
    c = s.allocate(256)
    s.free(c, 256)
    assert s.free_ranges() == [(512, 1024)]                                       # :2670-2681
    s = O.OracleTier(swap_size=1024)
    o1, o2, o3 = s.allocate(256), s.allocate(256), s.allocate(256)
    s.free(o1, 256)
    s.free(o3, 256)
    assert s.free_ranges() == [(0, 256), (512, 1024)]                             # :2684-2702
    s.free(o2, 256)
    assert s.free_ranges() == [(0, 1024)]
    s.free(100, 0)
    assert s.free_ranges() == [(0, 1024)]                                         # :2705-2710


def test_slots_sequential_and_reuse():
    s = O.OracleTier(swap_size=1024)
    assert [s.allocate(n) for n in (128, 256, 512)] == [0, 128, 384]              # :2713-2723
    assert s.free_ranges() == [(896, 1024)]
    s = O.OracleTier(swap_size=1024)
    a, b = s.allocate(512), s.allocate(512)
    assert (a, b) == (0, 512) and s.free_ranges() == []
    s.free(a, 512)
    assert s.allocate(256) == 0 and s.free_ranges() == [(256, 512)]               # :2726-2737


# ---- pool-level evict / restore (ref tiering.rs:2743-3420, pool.rs:2120-2175) ----

def pool(policy=0, **kw):
    # ref tiering.rs:2749-2778: 2 layers, 4 kv heads, head_dim 64, 4 x 64 tokens,
    # max_blocks 256, lru
    p = O.OraclePool(16, kw.get("layers", 2), 4, 64, kw.get("max_batch", 4), kw.get("max_seq", 64))
    assert p.enable_tiering(policy, kw.get("max_blocks", 256), kw.get("max_batch_blocks", 64))
    return p


def test_pool_evict_single_block():
    p = pool()
    [b] = p.alloc(1)
    assert p.location(b) == 0
    assert p.evict(1) == [b]                                                      # :2783-2820
    assert p.location(b) == 1 and p.cpu_offset(b) == 0
    assert p.offsets_f16()[b] == p.block_offset(b) // 2   # table unchanged (pool.rs:724-737)


def test_pool_evict_offsets_sequential():
    p = pool()
    t = p.alloc(3)
    per = 2 * 2 * p.stats()["block_bytes"]
    ev = p.evict(3)                                                               # :2823-2875
    assert sorted(ev) == sorted(t)
    assert sorted(p.cpu_offset(b) for b in t) == [0, per, 2 * per]
    assert p.evict(0) == []                                                       # :2887-2908
    q = pool()
    q.alloc(2)
    assert len(q.evict(10)) == 2                                                  # :2911-2924


def test_pool_evict_keeps_physical_total():
    p = pool()
    p.alloc(2)
    before = p.stats()
    p.evict(2)                                                                    # :2927-2948
    after = p.stats()
    assert after["total_physical_blocks"] == before["total_physical_blocks"]
    assert after["free_physical_blocks"] == before["free_physical_blocks"] + 2
    assert after["blocks_in_use"] == before["blocks_in_use"]


def test_pool_restore_transitions():
    p = pool()
    [b] = p.alloc(1)
    va0 = p.block_offset(b)
    assert p.restore_one(b) == va0                                                # GPU: no-op (:3134-3157)
    p.evict(1)
    va = p.restore_one(b)                                                         # :3098-3131
    assert va is not None and va > 0 and p.location(b) == 0
    assert p.cpu_offset(b) is None
    # its swap slot is free again: the next eviction lands at offset 0 (:3194-3222)
    p.evict(1)
    assert p.cpu_offset(b) == 0
    assert p.restore([b]) and p.location(b) == 0                                  # :3225-3263
    assert p.evict(1) == [b] and p.location(b) == 1


def test_pool_restore_errors():
    p = pool()
    assert p.restore_one(999) is None                                             # :3349-3357
    [b] = p.alloc(1)
    p.release([b])
    assert p.restore_one(b) is None and not p.restore([b])
    q = O.OraclePool(16, 2, 4, 64, 4, 64)
    [c] = q.alloc(1)
    assert q.restore_one(c) is None and q.evict(1) == []   # tiering disabled


def test_pool_evict_policy_forgets_and_restore_touches():
    """ref tiering.rs:3266-3298: after eviction the old handle is not tracked;
    after restore the new handle is.  Through the pool: a restored block is
    the most recently used, so LRU evicts the others first."""
    p = pool()
    t = p.alloc(3)
    assert p.evict(1) == [t[0]]          # oldest allocation first
    p.restore([t[0]])
    assert p.evict(3) == [t[1], t[2], t[0]]


def test_pool_free_swapped_block_returns_slot():
    """ref pool.rs:2120-2172: freeing a swapped-out block releases its swap
    slot, not a page handle."""
    p = pool()
    t = p.alloc(2)
    free_before = p.stats()["free_physical_blocks"]
    p.evict(1)
    p.release([t[0]])
    st = p.stats()
    assert st["free_physical_blocks"] == free_before + 1 and st["blocks_in_use"] == 1
    p.evict(1)
    assert p.cpu_offset(t[1]) == 0       # the freed slot is reused


def test_pool_restore_allocation_rule_and_growth():
    """A restored block takes the next page by the allocation rule (LIFO pop,
    a new superblock when none is free)."""
    p = pool(max_batch=64, max_seq=1024)
    bps = p.stats()["blocks_per_superblock"]
    t = p.alloc(bps)                     # fills superblock 0
    ev = p.evict(2)
    assert ev == t[:2]
    u = p.alloc(2)                       # takes the two freed pages
    assert p.stats()["superblock_count"] == 1
    assert p.restore(ev)                 # none free: superblock 1 is mapped
    assert p.stats()["superblock_count"] == 2
    assert [p.block_offset(b) // (2 * 1024 * 1024) for b in ev] == [1, 1]
    assert len(set(p.block_offset(b) for b in t + u)) == len(t) + len(u)


def test_pool_set_policy_starts_fresh():
    """ref tiering.rs:851-875: a new policy has no history, so until blocks
    are allocated or accessed nothing is selected (LRU / LFU / FIFO)."""
    p = pool()
    t = p.alloc(3)
    assert p.set_policy("lfu") and p.policy_name() == "lfu"
    assert p.evict(3) == []
    p.access(t[2])
    assert p.evict(3) == [t[2]]
    assert p.set_policy("arc") and p.evict(1) == [t[0]]   # arc ranks untracked last, in order
    assert not p.set_policy("nope") and p.policy_name() == "arc"
