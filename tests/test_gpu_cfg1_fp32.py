"""BASELINE configs[0] at its exact workload on the GPU: fp32 pages, batch 4,
8 q heads = 8 kv heads, head_dim 64, block_size 16, contexts U[1, 512], q/k/v
N(0,1); the 256-page pool is allocated through kcmm_alloc_blocks, its ids
given to the sequences in a seeded random permutation, one new token is
appended per sequence (kcmm_append_kv_step) and attention reads it
(seq_lens include it, ref kcmm_vllm_paged_attn.cu:10-102).  Pages must match
the oracle's bit for bit; attention within 1e-5 relative of the fp64 oracle
(the fp32 tolerance north_star states)."""
import math

import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_F32, make_config, memcpy_dtoh, memcpy_htod

pytestmark = pytest.mark.gpu

SB = 2 * 1024 * 1024
B, HQ, HKV, D, BS = 4, 8, 8, 64, 16


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("sync_variant", [True, False])
def test_cfg1_fp32_append_then_attention(gpu_lib, seed, sync_variant):
    import torch
    rng = np.random.default_rng(1000 + seed)
    # capacity: 4 sequences x 1024 tokens / 16 = 256 pages = 4 superblocks of 64
    cfg = make_config(num_layers=1, kv_heads=HKV, head_dim=D, max_batch=B, max_seq_len=1024,
                      block_size=BS)
    pool = gpu_lib.create_pool(cfg, KV_F32)
    opool = O.OraclePool(BS, 1, HKV, D, B, 1024, O.F32)
    try:
        ids = pool.alloc_blocks(256)
        assert ids == opool.alloc(256) == list(range(256))
        st = pool.stats()
        assert st["block_bytes"] == BS * HKV * D * 4 and st["superblock_count"] == 4
        perm = rng.permutation(np.asarray(ids))
        ctx = rng.integers(1, 513, size=B)
        L = ctx + 1                                   # one appended token each
        pages = [-(-int(n) // BS) for n in L]
        mbps = max(pages)
        bt = np.zeros((B, mbps), np.int32)
        pos, seqs = 0, []
        for b in range(B):
            bt[b, :pages[b]] = perm[pos:pos + pages[b]]
            pos += pages[b]
            s = pool.register_sequence(bt[b, :pages[b]].tolist())
            assert s == opool.register(bt[b, :pages[b]].tolist())
            pool.update_seq_len(s, int(ctx[b]))
            seqs.append(s)
        offs = np.asarray(pool.all_block_offsets_f16(), np.uint64)
        assert np.array_equal(offs, opool.offsets_f16()[:len(offs)])
        nb = st["superblock_count"] * SB
        row = HKV * D * 4
        # cached tokens 0 .. ctx-1: N(0,1) fp32 rows at their page slots
        kreg, vreg = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
        for b in range(B):
            for t in range(int(ctx[b])):
                page = int(offs[bt[b, t // BS]]) * 2 + (t % BS) * row
                kreg[page:page + row] = rng.standard_normal(HKV * D).astype(np.float32).view(np.uint8)
                vreg[page:page + row] = rng.standard_normal(HKV * D).astype(np.float32).view(np.uint8)
        memcpy_htod(pool.va_k(0), kreg)
        memcpy_htod(pool.va_v(0), vreg)
        # the appended token, through the reference's (seq, pos) entry point
        knew = rng.standard_normal((B, HKV * D)).astype(np.float32)
        vnew = rng.standard_normal((B, HKV * D)).astype(np.float32)
        kt, vt = torch.from_numpy(knew).cuda(), torch.from_numpy(vnew).cuda()
        pool.append_kv_step(0, seqs, [int(c) for c in ctx], kt.data_ptr(), vt.data_ptr())
        page_off = [int(offs[bt[b, int(ctx[b]) // BS]]) * 2 for b in range(B)]
        O.kv_write_rows(O.F32, kreg, vreg, knew, vnew, page_off, [int(c) % BS for c in ctx],
                        list(range(B)), HKV, D, row, row * BS)
        for s, n in zip(seqs, L):
            pool.update_seq_len(s, int(n))
        q = rng.standard_normal((B, HQ, D)).astype(np.float32)
        dev = dict(q=torch.from_numpy(q).cuda(), out=torch.full((B, HQ, D), float("nan"), device="cuda"),
                   bt=torch.from_numpy(bt).cuda(), sl=torch.from_numpy(L.astype(np.int32)).cuda(),
                   offs=torch.from_numpy(offs.view(np.int64)).cuda())
        stream = None if sync_variant else torch.cuda.current_stream().cuda_stream
        pool.paged_attn_decode(layer_idx=0, query_ptr=dev["q"].data_ptr(),
                               out_ptr=dev["out"].data_ptr(), block_tables_ptr=dev["bt"].data_ptr(),
                               seq_lens_ptr=dev["sl"].data_ptr(),
                               block_offsets_f16_ptr=dev["offs"].data_ptr(), batch=B,
                               num_q_heads=HQ, kv_heads=HKV, head_dim=D, block_size=BS,
                               max_blocks_per_seq=mbps, scale=1.0 / math.sqrt(D),
                               stream_ptr=stream)
        torch.cuda.synchronize()
        # pages bit-exact with the oracle's (the append included)
        assert np.array_equal(memcpy_dtoh(pool.va_k(0), nb), kreg)
        assert np.array_equal(memcpy_dtoh(pool.va_v(0), nb), vreg)
        ref = O.attn_decode_f64(O.F32, q, kreg, vreg, bt, L.astype(np.int32), offs, HQ, HKV, D,
                                BS, row, row * BS, 1.0 / math.sqrt(D))
        got = dev["out"].cpu().numpy().astype(np.float64)
        err = np.abs(got - ref).max() / np.abs(ref).max()
        assert err <= 1e-5, err
    finally:
        pool.destroy()


def test_fp32_edge_lengths_and_prefill(gpu_lib):
    """fp32 pages: zero and negative lengths write zeros, a one-token
    sequence returns its V row exactly (ref non_default_stream_ffi_smoke.py
    KAT), and chunked prefill over fp32 pages matches the fp64 oracle at 1e-5."""
    import torch
    from lattice_amd.workload import build_decode_case
    case = build_decode_case(gpu_lib, batch=5, num_q_heads=8, kv_heads=2, head_dim=128,
                             block_size=16, ctx_lens=[0, 1, 17, 300, 5], dtype=KV_F32, seed=9)
    try:
        case.dev["sl"].copy_(torch.tensor([0, 1, 17, 300, -3], dtype=torch.int32))
        case.seq_lens = np.array([0, 1, 17, 300, -3], np.int32)
        case.run_attention()
        g = case.geometry
        got = case.out_bits().astype(np.float64)
        ref = O.attn_decode_f64(O.F32, case.q_bits, case.k_mirror[0], case.v_mirror[0],
                                case.block_tables, case.seq_lens, case.offsets_f16, 8, 2, 128, 16,
                                g["row_bytes"], g["data_bytes"], 1 / math.sqrt(128))
        assert not got[0].any() and not got[4].any()
        page = int(case.offsets_f16[case.block_tables[1, 0]]) * 2
        for h in range(8):
            kvh = h * 2 // 8
            vrow = case.v_mirror[0][page + kvh * 512:page + (kvh + 1) * 512].view(np.float32)
            assert np.array_equal(got[1, h].astype(np.float32), vrow)
        assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-5
    finally:
        case.pool.destroy()
    from tests.test_gpu_prefill import rel_err, run_prefill
    ctx, lens = [40, 17, 70, 1, 300], [13, 17, 32, 1, 100]
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=16, kv_heads=4, head_dim=64,
                             block_size=16, ctx_lens=ctx, dtype=KV_F32, seed=11)
    try:
        got, ref = run_prefill(case, lens, 16, seed=12)
        assert np.isfinite(got).all() and rel_err(got, ref) <= 1e-5
    finally:
        case.pool.destroy()
