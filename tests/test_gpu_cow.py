"""Copy-on-write fork on the GPU: fork + private-copy of the last partial
page, page copies across every layer's K and V region bit-exact with the
oracle, and attention of the other beams unchanged by the copy."""
import math

import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, KV_FP8, make_config, memcpy_dtoh, memcpy_htod

pytestmark = pytest.mark.gpu

SB = 2 * 1024 * 1024


def fill_random(pool, rng):
    n = pool.stats()["superblock_count"] * SB
    regs = []
    for l in range(pool.stats()["num_layers"]):
        pair = []
        for base in (pool.va_k(l), pool.va_v(l)):
            # random finite bf16 / fp8-free bytes: low-magnitude bf16 pattern
            x = O.encode(O.BF16, rng.standard_normal(n // 2).astype(np.float32)).view(np.uint8)
            memcpy_htod(base, x)
            pair.append(x.copy())
        regs.append(pair)
    return regs


def read_all(pool):
    n = pool.stats()["superblock_count"] * SB
    return [[memcpy_dtoh(pool.va_k(l), n), memcpy_dtoh(pool.va_v(l), n)]
            for l in range(pool.stats()["num_layers"])]


@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_beam_fork_cow_copy_bit_exact(gpu_lib, dtype):
    import torch
    rng = np.random.default_rng(31 + dtype)
    L, hk, d, bs, B, beams = 3, 8, 128, 16, 4, 4
    pool = gpu_lib.create_pool(make_config(num_layers=L, kv_heads=hk, head_dim=d,
                                           max_batch=B * beams, max_seq_len=256), dtype)
    opool = O.OraclePool(bs, L, hk, d, B * beams, 256, dtype)
    try:
        seqs = []
        for b in range(B):
            n = int(rng.integers(1, 6))
            ids = pool.alloc_blocks(n)
            assert ids == opool.alloc(n)
            s = pool.register_sequence(ids)
            assert s == opool.register(ids)
            pool.update_seq_len(s, n * bs - int(rng.integers(1, bs)))
            seqs.append(s)
        regs = fill_random(pool, rng)
        pairs = []
        for s in seqs:
            for _ in range(beams - 1):
                f = pool.fork_sequence(s)
                assert f == opool.fork(s)
                last = len(pool.block_table(f)) - 1
                pair = pool.cow_block_for_append(f, last)
                rc, opair = opool.cow(f, last)
                assert rc == 1 and tuple(opair) == pair
                pairs.append(pair)
            # the original is still shared by nobody once all forks copied
            assert pool.refcount(pool.block_table(s)[-1]) == 1
        stream = torch.cuda.current_stream()
        pool.copy_blocks(pairs, stream_ptr=stream.cuda_stream)
        stream.synchronize()
        flat = [r for pair in regs for r in pair]
        offs = [(opool.block_offset(s_), opool.block_offset(d_)) for s_, d_ in pairs]
        O.copy_pages(flat, offs, pool.stats()["block_bytes"])
        got = read_all(pool)
        for l in range(L):
            assert np.array_equal(got[l][0], regs[l][0]) and np.array_equal(got[l][1], regs[l][1])

        # device-side variant (vLLM copy_blocks contract) on fresh pairs
        more = []
        for s in seqs[:2]:
            f = pool.fork_sequence(s)
            opool.fork(s)
            pair = pool.cow_block_for_append(f, 0)
            opool.cow(f, 0)
            if pair:
                more.append(pair)
        offs_host = pool.all_block_offsets_f16()
        offs_t = torch.tensor(offs_host, dtype=torch.int64, device="cuda")
        # pairs naming ids the pool never issued are skipped by the kernel
        bad = [(10**9, more[0][1]), (-1, more[0][1]), (more[0][0], len(offs_host))]
        pairs_t = torch.tensor(bad[:2] + more + bad[2:], dtype=torch.int64, device="cuda")
        pool.copy_blocks_device(pairs_t.data_ptr(), offs_t.data_ptr(), len(more) + len(bad),
                                stream_ptr=stream.cuda_stream)
        stream.synchronize()
        O.copy_pages(flat, [(opool.block_offset(a), opool.block_offset(b)) for a, b in more],
                     pool.stats()["block_bytes"])
        got = read_all(pool)
        for l in range(L):
            assert np.array_equal(got[l][0], regs[l][0]) and np.array_equal(got[l][1], regs[l][1])
    finally:
        pool.destroy()


def test_shared_block_write_is_refused(gpu_lib):
    import torch
    pool = gpu_lib.create_pool(make_config(num_layers=1, kv_heads=2, head_dim=64, max_batch=2,
                                           max_seq_len=64), KV_BF16)
    try:
        s = pool.register_sequence(pool.alloc_blocks(1))
        f = pool.fork_sequence(s)
        k = torch.zeros((1, 128), dtype=torch.bfloat16, device="cuda")
        with pytest.raises(Exception):
            pool.append_kv_step(0, [f], [3], k.data_ptr(), k.data_ptr())
        assert pool.cow_block_for_append(f, 0) is not None
        pool.append_kv_step(0, [f], [3], k.data_ptr(), k.data_ptr())
        pool.synchronize()
    finally:
        pool.destroy()


@pytest.mark.parametrize("dtype,width", [(KV_BF16, 4), (KV_FP8, 4), (KV_BF16, 1), (KV_BF16, 2)])
def test_fork_beams_matches_separate_calls(gpu_lib, dtype, width):
    """kcmm_fork_beams_on_stream against the oracle pool doing fork + CoW per
    child in the same order: child ids, every table and refcount, the number
    of copies, and every byte of all 2*L regions after the one copy kernel.
    Sequences whose next token opens a new page need no copy."""
    import torch
    rng = np.random.default_rng(7 + dtype + width)
    L, hk, d, bs, B = 2, 8, 128, 16, 6
    pool = gpu_lib.create_pool(make_config(num_layers=L, kv_heads=hk, head_dim=d,
                                           max_batch=B * width, max_seq_len=256), dtype)
    opool = O.OraclePool(bs, L, hk, d, B * width, 256, dtype)
    try:
        seqs, lens = [], {}
        for b in range(B):
            n = int(rng.integers(1, 6))
            ids = pool.alloc_blocks(n)
            assert ids == opool.alloc(n)
            s = pool.register_sequence(ids)
            assert s == opool.register(ids)
            # every other sequence ends exactly on a page boundary
            ln = n * bs if b % 2 else n * bs - int(rng.integers(1, bs))
            pool.update_seq_len(s, ln)
            opool.update_seq_len(s, ln)
            seqs.append(s)
            lens[s] = ln
        regs = fill_random(pool, rng)
        stream = torch.cuda.current_stream()
        children, ncopy = pool.fork_beams(seqs, width, stream_ptr=stream.cuda_stream)
        stream.synchronize()
        ochildren, opairs = [], []
        for s in seqs:
            for _ in range(width - 1):
                c = opool.fork(s)
                ochildren.append(c)
                logical = lens[s] // bs          # the child's next token
                if logical < len(opool.block_table(c)):
                    rc, pair = opool.cow(c, logical)
                    if rc == 1:
                        opairs.append(tuple(pair))
        assert children == ochildren
        assert ncopy == len(opairs) == (width - 1) * (B // 2 + B % 2)
        for s in seqs + children:
            assert pool.block_table(s) == opool.block_table(s)
            for blk in pool.block_table(s):
                assert pool.refcount(blk) == opool.refcount(blk)
        flat = [r for pair in regs for r in pair]
        O.copy_pages(flat, [(opool.block_offset(a), opool.block_offset(b)) for a, b in opairs],
                     pool.stats()["block_bytes"])
        got = read_all(pool)
        for l in range(L):
            assert np.array_equal(got[l][0], regs[l][0]) and np.array_equal(got[l][1], regs[l][1])
    finally:
        pool.destroy()


def test_fork_beams_repeated_steps(gpu_lib):
    """Four beam steps in a row, each forking every parent into 3 children
    whose last partial page is made private, then releasing the children (so
    later forks take recycled table buffers): after every step the child ids,
    tables, refcounts and the allocator's next ids equal the oracle pool's
    fork + CoW + unregister; the regions hold every copy at the end."""
    import torch
    rng = np.random.default_rng(19)
    L, hk, d, bs, B, width = 2, 8, 128, 16, 5, 4
    pool = gpu_lib.create_pool(make_config(num_layers=L, kv_heads=hk, head_dim=d,
                                           max_batch=B * width, max_seq_len=512), KV_BF16)
    opool = O.OraclePool(bs, L, hk, d, B * width, 512, KV_BF16)
    try:
        seqs, lens = [], {}
        for b in range(B):
            n = int(rng.integers(2, 9))
            ids = pool.alloc_blocks(n)
            assert ids == opool.alloc(n)
            s = pool.register_sequence(ids)
            assert s == opool.register(ids)
            ln = n * bs - int(rng.integers(1, bs))       # a partial last page
            pool.update_seq_len(s, ln)
            opool.update_seq_len(s, ln)
            seqs.append(s)
            lens[s] = ln
        regs = fill_random(pool, rng)
        stream = torch.cuda.current_stream()
        all_pairs = []
        for step in range(4):
            children, ncopy = pool.fork_beams(seqs, width, stream_ptr=stream.cuda_stream)
            stream.synchronize()
            ochildren = []
            for s in seqs:
                for _ in range(width - 1):
                    c = opool.fork(s)
                    ochildren.append(c)
                    rc, pair = opool.cow(c, lens[s] // bs)
                    assert rc == 1
                    all_pairs.append(tuple(pair))
            assert children == ochildren and ncopy == B * (width - 1), step
            for s in seqs + children:
                assert pool.block_table(s) == opool.block_table(s), (step, s)
                for blk in pool.block_table(s):
                    assert pool.refcount(blk) == opool.refcount(blk), (step, blk)
            # the copies of this step land before its children are released
            flat = [r for pair in regs for r in pair]
            O.copy_pages(flat, [(opool.block_offset(a), opool.block_offset(b))
                                for a, b in all_pairs[-ncopy:]], pool.stats()["block_bytes"])
            got = read_all(pool)
            for l in range(L):
                assert np.array_equal(got[l][0], regs[l][0]), (step, l)
                assert np.array_equal(got[l][1], regs[l][1]), (step, l)
            for c in children:
                pool.unregister_sequence(c)
                opool.unregister(c)
            for s in seqs:
                for blk in pool.block_table(s):
                    assert pool.refcount(blk) == opool.refcount(blk) == 1, (step, blk)
        # the freed private pages come back in the oracle's order
        ids = pool.alloc_blocks(3)
        assert ids == opool.alloc(3)
    finally:
        pool.destroy()
