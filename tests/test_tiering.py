"""Tiering bookkeeping of the product (libkcmm's pool code through the
host-check build of the C ABI) against the oracle: the reference's
pool-level evict / restore expectations (ref tiering.rs:2743-3420,
pool.rs:2120-2175) run on both, then randomized sequences of allocation,
free, eviction, restore, hints, protection and policy changes compared on
every observable (locations, page offsets, offset table, stats).  The bytes
moved are checked on the GPU (tests/test_gpu_tiering.py)."""
import random

import pytest

from lattice_amd.bindings import KcmmError, make_config
from tests.poolapi import OracleAdapter, ProductAdapter

SB = 2 * 1024 * 1024


@pytest.fixture(params=["oracle", "product"])
def make(request, hostcheck_lib, oracle_lib):
    made = []

    def factory(**kw):
        kw.setdefault("tiering", True)
        if request.param == "oracle":
            a = OracleAdapter(**kw)
        else:
            a = ProductAdapter(hostcheck_lib, **kw)
            made.append(a)
        return a

    yield factory
    for a in made:
        a.close()


def geo(**kw):
    # ref tiering.rs:2749-2778
    d = dict(block_size=16, num_layers=2, kv_heads=4, head_dim=64, max_batch=4, max_seq_len=64,
             max_blocks=256)
    d.update(kw)
    return d


def test_evict_restore_transitions(make):
    p = make(**geo())
    [b] = p.alloc(1)
    va0 = p.block_offset(b)
    assert p.location(b) == 0
    assert p.restore_one(b) == va0            # GPU-resident: returns its offset
    assert p.evict(1) == 1 and p.location(b) == 1
    assert p.offsets_f16()[b] == va0 // 2      # the table keeps the last offset
    va = p.restore_one(b)
    assert va == va0 and p.location(b) == 0   # the same page comes back (LIFO)
    assert p.evict(0) == 0
    assert p.evict(10) == 1 and p.restore([b, b]) and p.location(b) == 0


def test_evict_keeps_physical_total_and_frees_pages(make):
    p = make(**geo())
    p.alloc(2)
    before = p.stats()
    assert p.evict(2) == 2
    after = p.stats()
    assert after["total_physical_blocks"] == before["total_physical_blocks"]
    assert after["free_physical_blocks"] == before["free_physical_blocks"] + 2
    assert after["blocks_in_use"] == before["blocks_in_use"] == 2


def test_lru_order_and_restore_touch(make):
    p = make(**geo())
    t = p.alloc(3)
    assert p.evict(1) == 1 and [p.location(b) for b in t] == [1, 0, 0]
    assert p.restore([t[0]])
    assert p.evict(2) == 2 and [p.location(b) for b in t] == [0, 1, 1]


def test_policies_by_config(make):
    # ffi.rs:425-432: 0 lru, 1 lfu, 2 fifo, anything else lru
    for code, name in ((0, "lru"), (1, "lfu"), (2, "fifo"), (7, "lru")):
        p = make(**geo(), policy=code)
        assert p.policy_name() == name


def test_protect_and_hint_shape_lru(make):
    p = make(**geo())
    t = p.alloc(4)
    s = p.register(t[:2])
    assert p.protect([t[0]], 0)               # never-evict: refreshes the access
    assert p.protect([t[1]], 2)               # evict-preferred: no change
    assert not p.protect([t[2], 99], 0)       # unknown block: error (t[2] refreshed first)
    assert p.hint_protect(s)                  # t[0], t[1] refreshed in table order
    assert p.evict(2) == 2
    assert [p.location(b) for b in t] == [0, 0, 1, 1]


def test_set_policy(make):
    p = make(**geo())
    t = p.alloc(3)
    assert p.set_policy("LFU") and p.policy_name() == "lfu"
    assert p.evict(3) == 0                    # a fresh policy has no history
    assert p.protect([t[1]], 1)
    assert p.evict(3) == 1 and p.location(t[1]) == 1
    assert not p.set_policy("mru") and p.policy_name() == "lfu"
    assert p.set_policy("arc") and p.evict(1) == 1 and p.location(t[0]) == 1


def test_disabled(make):
    p = make(**geo(), tiering=False)
    [b] = p.alloc(1)
    assert p.evict(4) == 0 and p.location(b) == 0
    assert p.restore_one(b) is None and not p.restore([b])
    assert not p.set_policy("lru")


def test_restore_errors(make):
    p = make(**geo())
    t = p.alloc(2)
    p.evict(1)
    assert p.restore_one(999) is None
    assert not p.restore([t[0], 999])          # nothing restored
    assert p.location(t[0]) == 1
    p.free([t[1]])
    assert not p.restore([t[1]])


def test_free_swapped_block(make):
    p = make(**geo())
    t = p.alloc(2)
    free0 = p.stats()["free_physical_blocks"]
    p.evict(1)
    p.free([t[0]])
    st = p.stats()
    assert st["free_physical_blocks"] == free0 + 1 and st["blocks_in_use"] == 1
    assert p.location(t[0]) is None


def test_restore_grows_and_batches(make):
    p = make(**geo(max_batch=64, max_seq_len=1024))
    bps = p.stats()["blocks_per_superblock"]
    t = p.alloc(bps)
    assert p.evict(10) == 10
    p.alloc(10)                                # the freed pages are reused
    assert p.restore(t[:10])                   # a batch of 10: superblock 1 is mapped
    assert p.stats()["superblock_count"] == 2
    assert all(p.block_offset(b) // SB == 1 for b in t[:10])


def test_restore_capacity_exhausted(make):
    """Without a free page: fewer than 8 blocks stop at the first failure,
    8 or more restore what fits (here none) and report an error."""
    p = make(**geo(max_batch=1, max_seq_len=16 * 4))   # room for one superblock only
    bps = p.stats()["blocks_per_superblock"]
    t = p.alloc(bps)
    assert p.evict(9) == 9
    p.alloc(9)
    assert not p.restore(t[:2]) and p.location(t[0]) == 1
    assert not p.restore(t[:9]) and all(p.location(b) == 1 for b in t[:9])
    p.free(t[20:22])                            # two pages come free
    assert not p.restore(t[:9])                 # batch: two restored, error for the rest
    assert [p.location(b) for b in t[:9]].count(0) == 2


def snapshot(a, nblocks):
    return ([a.location(b) for b in range(nblocks)],
            [a.block_offset(b) for b in range(nblocks)],
            a.offsets_f16(), a.stats())


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("policy", [0, 1, 2])
def test_randomized_against_oracle(hostcheck_lib, oracle_lib, seed, policy):
    rng = random.Random(seed * 7 + policy)
    g = geo(max_batch=8, max_seq_len=512, num_layers=3, max_blocks=rng.choice([12, 64, 256]),
            max_batch_blocks=rng.choice([4, 64]))
    o = OracleAdapter(**g, tiering=True, policy=policy)
    q = ProductAdapter(hostcheck_lib, **g, tiering=True, policy=policy)
    try:
        live, seqs = [], []
        for step in range(300):
            op = rng.random()
            if op < 0.25:
                n = rng.randint(1, 6)
                a, b = o.alloc(n), q.alloc(n)
                assert a == b
                if a:
                    live += a
                    if rng.random() < 0.3:
                        s1, s2 = o.register(a), q.register(a)
                        assert s1 == s2
                        seqs.append(s1)
            elif op < 0.35 and live:
                k = rng.sample(live, min(len(live), rng.randint(1, 4)))
                o.free(k)
                q.free(k)
                live = [b for b in live if b not in k]
            elif op < 0.55:
                c = rng.randint(0, 8)
                assert o.evict(c) == q.evict(c)
            elif op < 0.7 and live:
                k = rng.sample(live, min(len(live), rng.randint(1, 10)))
                if rng.random() < 0.5:
                    assert o.restore(k) == q.restore(k)
                else:
                    assert o.restore_one(k[0]) == q.restore_one(k[0])
            elif op < 0.8 and live:
                k = rng.sample(live, min(len(live), 3)) + ([10**6] if rng.random() < 0.2 else [])
                lvl = rng.choice([0, 1, 2])
                assert o.protect(k, lvl) == q.protect(k, lvl)
            elif op < 0.88 and seqs:
                s = rng.choice(seqs)
                assert o.hint_protect(s) == q.hint_protect(s)
            elif op < 0.9:
                name = rng.choice(["lru", "lfu", "fifo", "arc", "sink_window", "bogus"])
                assert o.set_policy(name) == q.set_policy(name)
            n = o.stats()["total_blocks"]
            assert snapshot(o, n) == snapshot(q, n), f"step {step}"
    finally:
        q.close()


def test_abi_flags(hostcheck_lib):
    pool = hostcheck_lib.create_pool(make_config(num_layers=2, kv_heads=4, head_dim=64,
                                                 max_batch=4, max_seq_len=64, tiering=True))
    try:
        assert pool.tiering_enabled() and pool.stats()["tiering_enabled"] == 1
        assert pool.eviction_policy() == "lru"
        [b] = pool.alloc_blocks(1)
        assert pool.is_gpu_resident(b) and pool.evict_blocks(1) == 1
        assert not pool.is_gpu_resident(b) and pool.block_location(b) == "cpu"
        # writes into a swapped-out block are refused until it is restored
        # (argument checks precede any device work, so fake source addresses do)
        with pytest.raises(KcmmError, match="not resident in HBM"):
            pool.append_kv_slots(0, [b * 16], 64, 64, 0)
        s = pool.register_sequence([b])
        with pytest.raises(KcmmError, match="not resident in HBM"):
            pool.append_kv_step(0, [s], [0], 64, 64)
        assert pool.restore_block(b) > 0 and pool.block_location(b) == "gpu"
    finally:
        pool.destroy()
