"""Page allocator / block table: the reference's own unit-test constants
(ref superblock.rs:183-477, pool.rs:1886-2400, paged_kv.rs:826-895), run
against the oracle (which they pin) and against the product's pool code
through the host-check build of the C ABI; then a randomized differential
run of oracle vs product over every observable (ids, offsets, tables, counts,
stats, metrics)."""
import math
import random

import numpy as np
import pytest

import oracle as O
from tests.poolapi import OracleAdapter, ProductAdapter

SB = 2 * 1024 * 1024


@pytest.fixture(params=["oracle", "product"])
def make(request, hostcheck_lib, oracle_lib):
    made = []

    def factory(**kw):
        if request.param == "oracle":
            a = OracleAdapter(**kw)
        else:
            a = ProductAdapter(hostcheck_lib, **kw)
            made.append(a)
        return a

    yield factory
    for a in made:
        a.close()


def geo(kv_heads=4, head_dim=64, block_size=16, num_layers=22, max_batch=8, max_seq_len=128):
    return dict(block_size=block_size, num_layers=num_layers, kv_heads=kv_heads,
                head_dim=head_dim, max_batch=max_batch, max_seq_len=max_seq_len)


@pytest.mark.parametrize("kv,d,block_bytes,bps", [
    (4, 128, 16384, 128),   # ref superblock.rs:190-198
    (4, 64, 8192, 256),     # ref superblock.rs:201-207
    (32, 64, 65536, 32),    # ref superblock.rs:247-252
])
def test_block_sizing(make, kv, d, block_bytes, bps):
    p = make(**geo(kv_heads=kv, head_dim=d))
    st = p.stats()
    assert st["block_bytes"] == block_bytes and st["blocks_per_superblock"] == bps
    assert st["total_physical_blocks"] == 0 and st["free_physical_blocks"] == 0


def test_pool_construction(make):
    # ref pool.rs:1949-1962
    p = make(**geo())
    st = p.stats()
    assert st["block_size"] == 16 and st["num_layers"] == 22 and st["max_blocks_per_seq"] == 8
    assert st["blocks_in_use"] == 0 and st["total_blocks"] == 0 and st["active_sequences"] == 0


def test_tail_padding_5120(make):
    # ref superblock.rs:286-302: 5120-byte blocks -> 409 per superblock, 3072 B tail
    p = make(**geo(kv_heads=5, head_dim=32, max_batch=1, max_seq_len=409 * 16))
    st = p.stats()
    assert st["block_bytes"] == 5120 and st["blocks_per_superblock"] == 409
    assert SB - 409 * 5120 == 3072
    ids = p.alloc(409)
    offs = [p.block_offset(i) for i in ids]
    assert max(o // 5120 for o in offs) == 408 and all(o < SB for o in offs)
    assert p.stats()["superblock_count"] == 1


def test_first_block_is_top_of_superblock(make):
    # LIFO pop of a fresh superblock yields index bps-1 (ref superblock.rs:95-116);
    # consistent with ref paged_kv.rs:936 asserting va > 0.
    p = make(**geo())
    ids = p.alloc(3)
    assert ids == [0, 1, 2]
    assert [p.block_offset(i) for i in ids] == [255 * 8192, 254 * 8192, 253 * 8192]


def test_lifo_reuse(make):
    # ref superblock.rs:445-463 and pool.rs:412-454: last freed is reused first
    p = make(**geo(kv_heads=32, head_dim=64, max_batch=4, max_seq_len=1024))
    a, b = p.alloc(2)
    off_a, off_b = p.block_offset(a), p.block_offset(b)
    p.free([a])
    p.free([b])
    r1, r2 = p.alloc(1)[0], p.alloc(1)[0]
    assert (r1, r2) == (b, a)
    assert (p.block_offset(r1), p.block_offset(r2)) == (off_b, off_a)


def test_sequential_superblocks(make):
    # ref superblock.rs:416-442 with 64 KiB blocks (32 per superblock)
    p = make(**geo(kv_heads=32, head_dim=64, max_batch=4, max_seq_len=1024))
    first = p.alloc(32)
    assert all(p.block_offset(i) < SB for i in first)
    assert p.stats()["free_physical_blocks"] == 0
    second = p.alloc(32)
    assert all(SB <= p.block_offset(i) < 2 * SB for i in second)
    p.free(first[:10])
    again = p.alloc(10)
    assert all(p.block_offset(i) < SB for i in again)


def test_capacity_rounds_up_to_superblock(make):
    # ref pool.rs:2245-2295: max_blocks_total = 1, 32 blocks per superblock
    p = make(**geo(kv_heads=32, head_dim=64, num_layers=2, max_batch=1, max_seq_len=16))
    got = [p.alloc(1) for _ in range(32)]
    assert all(g is not None for g in got)
    assert p.alloc(1) is None
    assert p.stats()["total_physical_blocks"] == 32


def test_blocks_in_use_and_total(make):
    # ref pool.rs:2107-2130
    p = make(**geo())
    t1 = p.alloc(3)
    assert (p.stats()["blocks_in_use"], p.stats()["total_blocks"]) == (3, 3)
    t2 = p.alloc(5)
    assert (p.stats()["blocks_in_use"], p.stats()["total_blocks"]) == (8, 8)
    p.free(t1)
    assert (p.stats()["blocks_in_use"], p.stats()["total_blocks"]) == (5, 8)
    p.free(t2)
    assert p.stats()["blocks_in_use"] == 0


def test_sequence_lifecycle(make):
    # ref pool.rs:1997-2024 and examples/kcmm_c_integration.c sequence test
    p = make(**geo())
    t = p.alloc(3)
    s = p.register(t)
    assert s == 0 and p.stats()["active_sequences"] == 1
    p.update_seq_len(s, 45)
    extra = p.alloc(1)[0]
    assert p.append_block(s, extra)
    assert p.block_table(s) == t + [extra]
    offs = p.table_offsets(s)
    assert len(set(offs)) == 4 and all(o > 0 for o in offs)
    p.unregister(s)
    assert p.stats()["blocks_in_use"] == 0
    assert p.block_table(s) == []
    assert p.register([]) == 1  # indices are never reused (ref pool.rs:551-557)
    assert not p.append_block(99, 0)
    assert p.block_table(99) is None and p.table_offsets(99) is None


def test_many_blocks_across_superblocks(make):
    # ref pool.rs:2230-2243
    p = make(**geo(max_batch=4, max_seq_len=16384))
    n = 256 + 10
    t = p.alloc(n)
    st = p.stats()
    assert st["superblock_count"] >= 2 and st["blocks_in_use"] == n
    p.free(t)
    assert p.stats()["blocks_in_use"] == 0


def test_offset_table_holes_are_zero(make):
    # ref pool.rs:724-748: freed ids report offset 0 and valid 0
    p = make(**geo())
    ids = p.alloc(4)
    p.free([ids[1]])
    offs, valid = p.offsets_f16(), p.valid()
    assert offs[1] == 0 and valid == [1, 0, 1, 1]
    assert offs[0] == p.block_offset(ids[0]) // 2


def test_metrics(make):
    # ref pool.rs:2211-2228 plus the closed forms of ref pool.rs:1179-1240
    p = make(**geo())
    s = p.register(p.alloc(4))
    p.update_seq_len(s, 50)
    m = p.metrics()
    ideal = 50 * 4 * 64 * 22 * 2
    actual = SB * 22 * 2
    assert m["ifr"] == pytest.approx((64 - 50) / 64, rel=1e-6)
    assert m["bu"] == pytest.approx(4 / 256, rel=1e-6)
    assert m["pme"] == pytest.approx(ideal / actual, rel=1e-6)
    assert m["rfi"] == pytest.approx(1 - ideal / actual, rel=1e-6)
    st = p.stats()
    assert st["physical_idle_ratio"] == pytest.approx(1 - 4 * 8192 / SB, rel=1e-6)


def test_low_watermark(make):
    # ref pool.rs:2230: empty pool is never below the watermark
    p = make(**geo())
    assert not p.below(0.2)
    p.alloc(10)
    assert p.below(1.0) == ((256 - 10) / 256 < 1.0)
    assert not p.below(0.01)


def test_fork_and_cow(make):
    p = make(**geo())
    t = p.alloc(3)
    s = p.register(t)
    p.update_seq_len(s, 40)
    f = p.fork(s)
    assert p.block_table(f) == t and all(p.refcount(b) == 2 for b in t)
    rc, pair = p.cow(f, 2)
    assert rc == 1 and pair[0] == t[2] and pair[1] not in t
    assert p.refcount(t[2]) == 1 and p.block_table(f) == t[:2] + [pair[1]]
    assert p.cow(f, 2) == (0, None)          # now private
    assert p.cow(f, 9)[0] == -1              # past the table
    p.unregister(s)                          # drops one reference of each shared block
    assert p.refcount(t[0]) == 1 and p.refcount(t[2]) == 0
    p.unregister(f)
    assert p.stats()["blocks_in_use"] == 0


def test_share_prefix(make):
    p = make(**geo())
    src = p.register(p.alloc(4))
    dst = p.register(p.alloc(1))
    shared = p.share_prefix(src, dst, 3)
    assert shared == p.block_table(src)[:3]
    assert p.block_table(dst)[1:] == shared and all(p.refcount(b) == 2 for b in shared)
    assert p.share_prefix(src, dst, 5) is None
    assert p.share_prefix(src, 77, 1) is None


def test_failed_multi_block_alloc_leaves_no_blocks_behind(make):
    # The reference leaks the blocks installed before a capacity failure
    # (ref pool.rs:462-476); this build undoes them (documented deviation).
    p = make(**geo(kv_heads=32, head_dim=64, num_layers=2, max_batch=1, max_seq_len=16))
    keep = p.alloc(30)
    before = (p.stats(), p.offsets_f16(), p.valid())
    assert p.alloc(5) is None
    assert (p.stats(), p.offsets_f16(), p.valid()) == before
    assert p.alloc(2) is not None and keep


def _random_ops(seed, n_ops=400):
    rng = random.Random(seed)
    ops = []
    for _ in range(n_ops):
        r = rng.random()
        if r < 0.30:
            ops.append(("alloc", rng.randint(1, 40)))
        elif r < 0.45:
            ops.append(("free_some", rng.random()))
        elif r < 0.60:
            ops.append(("register", rng.randint(0, 6)))
        elif r < 0.68:
            ops.append(("unregister", rng.randint(0, 30)))
        elif r < 0.74:
            ops.append(("append", rng.randint(0, 30)))
        elif r < 0.80:
            ops.append(("seq_len", rng.randint(0, 30), rng.randint(0, 500)))
        elif r < 0.86:
            ops.append(("fork", rng.randint(0, 30)))
        elif r < 0.93:
            ops.append(("cow", rng.randint(0, 30), rng.randint(0, 8)))
        else:
            ops.append(("share", rng.randint(0, 30), rng.randint(0, 30), rng.randint(1, 4)))
    return ops


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("shape", [dict(kv_heads=32, head_dim=64, num_layers=2, max_batch=4,
                                        max_seq_len=512),
                                   dict(kv_heads=5, head_dim=32, num_layers=3, max_batch=2,
                                        max_seq_len=409 * 16 * 2 // 2)])
def test_differential_oracle_vs_product(hostcheck_lib, oracle_lib, seed, shape):
    """Random operation sequences: every observable must match exactly."""
    kw = dict(block_size=16, **shape)
    a, b = OracleAdapter(**kw), ProductAdapter(hostcheck_lib, **kw)
    owned = []   # blocks allocated and not yet handed to a sequence
    rng = random.Random(seed + 1000)
    try:
        for op in _random_ops(seed):
            kind = op[0]
            if kind == "alloc":
                ra, rb = a.alloc(op[1]), b.alloc(op[1])
                assert ra == rb, op
                if ra:
                    owned.extend(ra)
            elif kind == "free_some" and owned:
                k = int(len(owned) * op[1])
                ids, owned[:] = owned[:k], owned[k:]
                a.free(ids)
                b.free(ids)
            elif kind == "register":
                t, owned[:] = owned[: op[1]], owned[op[1]:]
                assert a.register(t) == b.register(t)
            elif kind == "unregister":
                a.unregister(op[1])
                b.unregister(op[1])
            elif kind == "append" and owned:
                blk = owned.pop()
                assert a.append_block(op[1], blk) == b.append_block(op[1], blk)
            elif kind == "seq_len":
                a.update_seq_len(op[1], op[2])
                b.update_seq_len(op[1], op[2])
            elif kind == "fork":
                assert a.fork(op[1]) == b.fork(op[1])
            elif kind == "cow":
                assert a.cow(op[1], op[2]) == b.cow(op[1], op[2])
            elif kind == "share":
                assert a.share_prefix(op[1], op[2], op[3]) == b.share_prefix(op[1], op[2], op[3])
            # every observable after every step
            assert a.stats() == b.stats(), op
            assert a.offsets_f16() == b.offsets_f16()
            assert a.valid() == b.valid()
            for s in range(a.stats()["active_sequences"] + 1):
                assert a.block_table(s) == b.block_table(s)
                assert a.table_offsets(s) == b.table_offsets(s)
            for blk in range(a.stats()["total_blocks"]):
                assert a.refcount(blk) == b.refcount(blk)
            am, bm = a.metrics(), b.metrics()
            assert all(math.isclose(am[k], bm[k], rel_tol=0, abs_tol=0) for k in am), (am, bm)
            t = rng.random()
            assert a.below(t) == b.below(t)
    finally:
        b.close()


def test_fp32_pool_geometry_matches_oracle(hostcheck_lib):
    """fp32 pages: 4-byte elements, so a page at
    Hkv = 8, D = 64, bs = 16 is 32 KiB (64 per 2 MiB superblock); ids and
    offsets of the product pool equal the oracle pool's."""
    from lattice_amd.bindings import KV_F32, make_config
    cfg = make_config(num_layers=1, kv_heads=8, head_dim=64, max_batch=4, max_seq_len=1024)
    pool = hostcheck_lib.create_pool(cfg, KV_F32)
    opool = O.OraclePool(16, 1, 8, 64, 4, 1024, O.F32)
    try:
        assert pool.kv_dtype() == KV_F32
        ids = pool.alloc_blocks(256)
        assert ids == opool.alloc(256) == list(range(256))
        st = pool.stats()
        assert st["block_bytes"] == 32768 and st["blocks_per_superblock"] == 64
        assert st["superblock_count"] == 4
        assert np.array_equal(pool.all_block_offsets_f16(), opool.offsets_f16()[:256])
        with pytest.raises(Exception):
            pool.alloc_blocks(1)                 # capacity: 4 x 1024 / 16 = 256 pages
    finally:
        pool.destroy()
