"""Prefix cache on the GPU: pages cached under their content hashes outlive
their sequences, and a new sequence rebuilt from the cache attends to exactly
the same K/V (bit-identical attention output), for bf16 and fp8 pages."""
import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, KV_FP8
from lattice_amd.workload import build_decode_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_attention_over_attached_prefix_is_unchanged(gpu_lib, dtype):
    import torch
    ctx = [16 * 20, 16 * 7 + 5, 16 * 33, 16 * 2 + 9]
    case = build_decode_case(gpu_lib, batch=4, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=dtype, seed=40 + dtype)
    pool = case.pool
    try:
        full = [c // 16 for c in ctx]
        sl = torch.tensor([n * 16 for n in full], dtype=torch.int32, device="cuda")
        case.dev["sl"] = sl
        stream = torch.cuda.current_stream().cuda_stream
        case.run_attention(stream_ptr=stream)
        torch.cuda.synchronize()
        before = case.out_bits().copy()

        rng = np.random.default_rng(7)
        hashes = [O.prefix_hash_blocks(rng.integers(0, 128000, size=c), 16, seed=b)
                  for b, c in enumerate(ctx)]
        for b in range(4):
            assert pool.prefix_register(b, hashes[b][:full[b]]) == full[b]
        cached = {int(x) for b in range(4) for x in case.block_tables[b, :full[b]]}
        assert pool.prefix_entries() == len(cached)
        offs0 = pool.all_block_offsets_f16()
        for b in range(4):
            pool.unregister_sequence(b)
        fresh = pool.alloc_blocks(8)                 # reuses the freed partial pages first
        assert not cached & set(fresh)

        bt = np.zeros_like(case.block_tables)
        for b in range(4):
            s = pool.register_sequence([])
            got = pool.prefix_attach(s, hashes[b])
            assert got == case.block_tables[b, :full[b]].tolist()
            bt[b, :len(got)] = got
            pool.update_seq_len(s, full[b] * 16)
        offs1 = pool.all_block_offsets_f16()
        assert all(offs1[i] == offs0[i] for i in cached)
        case.dev["bt"] = torch.from_numpy(bt).cuda()
        case.dev["out"].fill_(float("nan"))
        case.run_attention(stream_ptr=stream)
        torch.cuda.synchronize()
        assert np.array_equal(case.out_bits(), before)
        assert all(pool.refcount(i) == 2 for i in cached)       # the cache + one sequence
        assert pool.prefix_evict() == len(cached)
        assert all(pool.refcount(i) == 1 for i in cached)
    finally:
        pool.destroy()
