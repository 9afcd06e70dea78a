"""Tiering on the GPU through the C ABI: blocks evicted to the host swap
buffer and restored come back byte-identical in every layer's K and V page
(oracle of a byte copy: the bytes read before eviction), also after their
old pages were reused and overwritten, through both the batched (>= 8
blocks, several gather / scatter launches) and the one-by-one restore; and
paged attention over restored pages gives the same bits as before the
round trip."""
import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, KV_FP8, make_config, memcpy_dtoh, memcpy_htod
from lattice_amd.workload import build_decode_case

pytestmark = pytest.mark.gpu

SB = 2 * 1024 * 1024


def regions(pool):
    n = pool.stats()["num_layers"]
    return [b for l in range(n) for b in (pool.va_k(l), pool.va_v(l))]


def fill(pool, rng):
    n = pool.stats()["superblock_count"] * SB
    for base in regions(pool):
        memcpy_htod(base, rng.integers(0, 256, n, dtype=np.uint8))


def page_bytes(pool, blk):
    bb = pool.stats()["block_bytes"]
    off = pool.block_va_offset(blk)
    return [memcpy_dtoh(base + off, bb) for base in regions(pool)]


@pytest.mark.parametrize("dtype,layers,n_evict", [(KV_BF16, 2, 70), (KV_FP8, 3, 9),
                                                  (KV_BF16, 4, 3)])
def test_evict_restore_bytes(gpu_lib, dtype, layers, n_evict):
    rng = np.random.default_rng(40 + layers)
    cfg = make_config(num_layers=layers, kv_heads=8, head_dim=128, max_batch=8, max_seq_len=4096,
                      tiering=True, max_blocks=512)
    pool = gpu_lib.create_pool(cfg, dtype)
    try:
        blocks = pool.alloc_blocks(120)
        fill(pool, rng)
        before = {b: page_bytes(pool, b) for b in blocks}
        print(f"evict {n_evict} of {len(blocks)} blocks, {layers} layers, dtype {dtype}", flush=True)
        assert pool.evict_blocks(n_evict) == n_evict
        gone = [b for b in blocks if pool.block_location(b) == "cpu"]
        assert gone == blocks[:n_evict]           # LRU: the oldest allocations
        # the freed pages are reused and overwritten before the restore
        reuse = pool.alloc_blocks(n_evict)
        fill(pool, rng)
        if n_evict >= 8:
            pool.restore_blocks(gone)
        else:
            for b in gone:
                assert pool.restore_block(b) == pool.block_va_offset(b)
        assert all(pool.block_location(b) == "gpu" for b in gone)
        for b in gone:
            after = page_bytes(pool, b)
            assert all(np.array_equal(x, y) for x, y in zip(before[b], after)), b
        # pages stay distinct among live blocks
        offs = [pool.block_va_offset(b) for b in blocks + reuse]
        assert len(set(offs)) == len(offs)
    finally:
        pool.destroy()


@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_attention_after_round_trip(gpu_lib, dtype):
    """Every page of a decode batch evicted, its pages handed to new blocks
    and overwritten, then restored (new pages): attention over the refreshed
    offset table gives the same output bits as before."""
    import torch
    ctx = [1, 17, 300, 64, 1000, 33]
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=dtype, num_layers=2, seed=41,
                             tiering=True)
    try:
        pool = case.pool
        case.run_attention(layer=1)
        torch.cuda.synchronize()
        out0 = case.out_bits().copy()
        ids = [b for b in range(pool.total_blocks()) if pool.block_location(b) is not None]
        n = pool.evict_blocks(len(ids))
        assert n == len(ids) and all(pool.block_location(b) == "cpu" for b in ids)
        spare = pool.alloc_blocks(len(ids))      # take the freed pages
        rng = np.random.default_rng(5)
        nbytes = pool.stats()["superblock_count"] * SB
        for base in regions(pool):
            memcpy_htod(base, rng.integers(0, 256, nbytes, dtype=np.uint8))
        pool.restore_blocks(ids)
        offs = np.asarray(pool.all_block_offsets_f16(), dtype=np.uint64)
        moved = sum(int(offs[b]) != int(case.offsets_f16[b]) for b in ids)
        print(f"restored {len(ids)} blocks, {moved} on new pages", flush=True)
        assert moved == len(ids)
        case.dev["offs"] = torch.from_numpy(offs.view(np.int64)).cuda()
        case.dev["out"].fill_(float("nan"))
        case.run_attention(layer=1)
        torch.cuda.synchronize()
        assert np.array_equal(case.out_bits(), out0)
        pool.free_blocks(spare)
    finally:
        case.pool.destroy()
