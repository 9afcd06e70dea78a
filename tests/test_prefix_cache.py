"""Prefix cache (the reference's SharingManager contract, ref
src/kcmm/sharing.rs:9-65: content hash -> prefix blocks, reference counted;
a placeholder there) on the CPU: the chained block hash against the published
FNV-1a-64 test vectors and its prefix properties, then the product (host-check
build of the C ABI) against the oracle's restatement over random operation
sequences, comparing every returned value, refcount, table and the ids the
allocator hands out afterwards (free order)."""
import random

import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KcmmError
from tests.poolapi import OracleAdapter, ProductAdapter

GEO = dict(block_size=16, num_layers=2, kv_heads=4, head_dim=64, max_batch=8, max_seq_len=256)


def test_fnv1a64_published_vectors():
    """The FNV-1a 64-bit test vectors published with the algorithm."""
    assert O.fnv1a64(b"") == 0xCBF29CE484222325
    assert O.fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert O.fnv1a64(b"foobar") == 0x85944171F73967E8


@pytest.mark.parametrize("bs,n,seed", [(16, 100, 0), (1, 7, 5), (7, 64, 2**63 + 11), (16, 15, 3)])
def test_block_hashes_match_oracle(hostcheck_lib, bs, n, seed):
    rng = np.random.default_rng(n + bs)
    tokens = rng.integers(-2**31, 2**31, size=n, dtype=np.int64).astype(np.int32)
    got = hostcheck_lib.prefix_hash_blocks(tokens, bs, seed).tolist()
    want = O.prefix_hash_blocks(tokens, bs, seed)
    assert got == want and len(got) == n // bs          # partial last block: no hash


def test_block_hash_chain_properties(hostcheck_lib):
    """Prefix-closed (the hashes of a prefix are a prefix of the hashes);
    changing one token of block j changes hashes j.. and none before; block 0
    depends on the seed."""
    rng = np.random.default_rng(9)
    t = rng.integers(0, 128000, size=160).astype(np.int32)
    full = hostcheck_lib.prefix_hash_blocks(t, 16).tolist()
    assert hostcheck_lib.prefix_hash_blocks(t[:70], 16).tolist() == full[:4]
    u = t.copy()
    u[16 * 5 + 3] += 1
    changed = hostcheck_lib.prefix_hash_blocks(u, 16).tolist()
    assert changed[:5] == full[:5] and all(a != b for a, b in zip(changed[5:], full[5:]))
    assert hostcheck_lib.prefix_hash_blocks(t, 16, seed=1).tolist()[0] != full[0]
    # block 0 is FNV-1a over (seed as 8 LE bytes) + 16 int32 LE tokens
    assert full[0] == O.fnv1a64(bytes(8) + t[:16].astype("<i4").tobytes())


class _Both:
    """The same calls on the oracle (pool + cache) and the product."""

    def __init__(self, lib):
        self.a = OracleAdapter(**GEO)
        self.b = ProductAdapter(lib, **GEO)
        self.cache = O.OraclePrefixCache(self.a.p)

    def close(self):
        self.b.close()

    def alloc(self, n):
        ra, rb = self.a.alloc(n), self.b.alloc(n)
        assert ra == rb
        return ra

    def register(self, table, seq_len):
        sa, sb = self.a.register(table), self.b.register(table)
        assert sa == sb
        self.a.update_seq_len(sa, seq_len)
        self.b.update_seq_len(sb, seq_len)
        return sa

    def prefix_register(self, seq, hashes):
        ra = self.cache.register(seq, hashes)
        try:
            rb = self.b.pool.prefix_register(seq, hashes)
        except KcmmError:
            rb = None
        assert ra == rb, (seq, len(hashes))
        return ra

    def check(self, nblocks, nseqs):
        for blk in range(nblocks):
            assert self.a.refcount(blk) == self.b.refcount(blk), blk
        for s in range(nseqs):
            assert self.a.block_table(s) == self.b.block_table(s), s
        assert len(self.cache.entries) == self.b.pool.prefix_entries()
        assert self.a.offsets_f16() == self.b.offsets_f16()


def test_cached_prefix_outlives_its_sequence(hostcheck_lib):
    both = _Both(hostcheck_lib)
    try:
        t = both.alloc(5)
        s0 = both.register(t, 5 * 16)
        h = [101, 102, 103, 104, 105]
        assert both.prefix_register(s0, h[:4]) == 4
        assert both.prefix_register(s0, h[:4]) == 0              # first registration wins
        assert both.b.pool.refcount(t[0]) == 2
        both.a.unregister(s0)
        both.b.unregister(s0)
        assert [both.b.pool.refcount(x) for x in t] == [1, 1, 1, 1, 0]   # block 4 freed
        s1 = both.register([], 0)
        assert both.cache.attach(s1, h) == both.b.pool.prefix_attach(s1, h) == t[:4]
        assert both.b.pool.prefix_match([101, 999, 103]) == [t[0]]
        assert both.cache.evict(10) == both.b.pool.prefix_evict(10) == 4
        assert [both.b.pool.refcount(x) for x in t[:4]] == [1, 1, 1, 1]  # held by s1 only
        both.check(8, 2)
        both.a.unregister(s1)
        both.b.unregister(s1)
        assert both.alloc(4) is not None                          # same ids, same order
        both.check(8, 2)
    finally:
        both.close()


def test_register_rejects_partial_and_unknown(hostcheck_lib):
    both = _Both(hostcheck_lib)
    try:
        t = both.alloc(3)
        s = both.register(t, 2 * 16 + 5)                        # blocks 0, 1 full; 2 partial
        assert both.prefix_register(s, [1, 2, 3]) is None       # partial block refused
        assert both.prefix_register(s, [1, 2]) == 2
        assert both.prefix_register(s, [1, 2, 3, 4]) is None    # more than the table
        assert both.prefix_register(7, [1]) is None             # unknown sequence
        with pytest.raises(KcmmError):
            both.b.pool.prefix_attach(9, [1])
        both.check(4, 1)
    finally:
        both.close()


@pytest.mark.parametrize("seed", range(6))
def test_differential_random_ops(hostcheck_lib, seed):
    """Random register / match / attach / evict / unregister / alloc against
    the oracle; token contents come from a few shared prompts so prefixes
    really repeat."""
    rng = random.Random(seed)
    both = _Both(hostcheck_lib)
    prompts = [[rng.randrange(1000) for _ in range(16 * 6)] for _ in range(3)]
    live = []          # (seq, hashes)
    nseqs = 0
    try:
        for step in range(120):
            op = rng.random()
            if op < 0.35:
                # a request: a prompt prefix, attach what is cached, allocate the rest
                p = prompts[rng.randrange(3)]
                ntok = rng.randrange(16, len(p) + 1)
                hashes = O.prefix_hash_blocks(p[:ntok], 16)
                assert hashes == hostcheck_lib.prefix_hash_blocks(np.array(p[:ntok]), 16).tolist()
                s = both.register([], 0)
                nseqs += 1
                ga = both.cache.attach(s, hashes)
                gb = both.b.pool.prefix_attach(s, hashes)
                assert ga == gb
                need = -(-ntok // 16) - len(ga)
                ids = both.alloc(need) if need else []
                if ids is None:
                    continue
                for blk in ids:
                    both.a.append_block(s, blk)
                    both.b.append_block(s, blk)
                both.a.update_seq_len(s, ntok)
                both.b.update_seq_len(s, ntok)
                live.append((s, hashes))
            elif op < 0.55 and live:
                s, hashes = live[rng.randrange(len(live))]
                k = rng.randrange(0, len(hashes) + 1)
                both.prefix_register(s, hashes[:k])
            elif op < 0.7 and live:
                s, hashes = live.pop(rng.randrange(len(live)))
                both.a.unregister(s)
                both.b.unregister(s)
            elif op < 0.8:
                n = rng.choice([1, 2, 5, 0xFFFFFFFF])
                assert both.cache.evict(n) == both.b.pool.prefix_evict(n)
            elif op < 0.9 and live:
                _, hashes = live[rng.randrange(len(live))]
                assert both.cache.match(hashes) == both.b.pool.prefix_match(hashes)
            else:
                ids = both.alloc(rng.randrange(1, 4))
                if ids:
                    both.a.free(ids)
                    both.b.free(ids)
            both.check(96, nseqs)
    finally:
        both.close()
