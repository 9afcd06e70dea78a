"""Causal chunked-prefill attention on the GPU through the C ABI vs the
oracle (fp64).  Tolerance (max|got-ref| / max|ref|): bf16 / f16 1e-2, fp8
pages 3e-2 (the decode tolerances).  The reference has no chunked prefill
(ref src/model/transformer.rs:50-65), so the oracle's textbook definition is
the target, pinned in tests/test_oracle_prefill.py."""
import math

import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, KV_F16, KV_FP8, memcpy_dtoh, memcpy_htod
from lattice_amd.workload import (build_decode_case, build_prefix_shared_case, encode16,
                                  io_dtype, torch_io_dtype)

pytestmark = pytest.mark.gpu

TOL = {KV_BF16: 1e-2, KV_F16: 1e-2, KV_FP8: 3e-2}


def rel_err(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def run_prefill(case, lens, hq, seed, scale=None):
    """Queries for the last lens[b] tokens of every sequence of a decode case."""
    import torch
    g = case.geometry
    d = case.head_dim
    qsl = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    qdt = io_dtype(case.dtype)
    rng = np.random.default_rng(seed)
    q = encode16(qdt, rng.standard_normal((int(qsl[-1]), hq, d)).astype(np.float32))
    tdt = torch_io_dtype(case.dtype)
    qt = (torch.from_numpy(q.copy()) if qdt == O.F32 else
          torch.from_numpy(q.view(np.int16)).view(tdt)).cuda()
    out = torch.full((int(qsl[-1]), hq, d), float("nan"), dtype=tdt, device="cuda")
    qslt = torch.from_numpy(qsl).cuda()
    scale = 1 / math.sqrt(d) if scale is None else scale
    dv = case.dev
    case.pool.paged_attn_prefill(
        layer_idx=0, query_ptr=qt.data_ptr(), out_ptr=out.data_ptr(),
        block_tables_ptr=dv["bt"].data_ptr(), seq_lens_ptr=dv["sl"].data_ptr(),
        query_start_loc_ptr=qslt.data_ptr(), block_offsets_f16_ptr=dv["offs"].data_ptr(),
        batch=case.batch, total_query_tokens=int(qsl[-1]), num_q_heads=hq,
        kv_heads=case.kv_heads, head_dim=d, block_size=case.block_size,
        max_blocks_per_seq=case.mbps, scale=scale,
        stream_ptr=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    if qdt == O.F32:
        got = out.cpu().numpy().astype(np.float64)
    else:
        got = O.decode(O.F16 if qdt == KV_F16 else O.BF16,
                       out.cpu().view(torch.int16).numpy().view(np.uint16)).astype(np.float64)
    ref = O.attn_prefill_f64(case.dtype, q, case.k_mirror[0], case.v_mirror[0],
                             case.block_tables, case.seq_lens, qsl, case.offsets_f16, hq,
                             case.kv_heads, d, case.block_size, g["row_bytes"],
                             g["data_bytes"], scale)
    return got, ref


CTX = [40, 17, 70, 1, 300, 129]
LENS = [13, 17, 32, 1, 100, 64]      # a chunk may be the whole sequence


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (32, 4), (32, 2)])
@pytest.mark.parametrize("d", [128, 64])
def test_mfma_groups_and_head_dims(gpu_lib, hq, hkv, d):
    case = build_decode_case(gpu_lib, batch=len(CTX), num_q_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=16, ctx_lens=CTX, dtype=KV_BF16, seed=hq + d)
    try:
        got, ref = run_prefill(case, LENS, hq, seed=hq * d)
        err = rel_err(got, ref)
        print(f"prefill G={hq // hkv} D={d} err={err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= TOL[KV_BF16]
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("dtype,bs", [(KV_F16, 16), (KV_BF16, 8), (KV_BF16, 32)])
def test_dtypes_and_block_sizes(gpu_lib, dtype, bs):
    case = build_decode_case(gpu_lib, batch=len(CTX), num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=bs, ctx_lens=CTX, dtype=dtype, seed=bs + dtype)
    try:
        got, ref = run_prefill(case, LENS, 32, seed=bs)
        err = rel_err(got, ref)
        print(f"prefill dtype={dtype} bs={bs} err={err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= TOL[dtype]
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8), (32, 4), (32, 2)])
@pytest.mark.parametrize("bs", [16, 8, 32])
def test_fp8_pages_on_mfma(gpu_lib, hq, hkv, bs):
    """fp8-e4m3 pages at head_dim 128 take the MFMA kernel: codes gathered,
    dequantized with their page's per-kv-head scale to bf16 in LDS; against
    the oracle on the same pages (3e-2), every GQA group, three block sizes
    (a 32-key tile spans 1, 2 or 4 pages, each with its own scale)."""
    case = build_decode_case(gpu_lib, batch=len(CTX), num_q_heads=hq, kv_heads=hkv, head_dim=128,
                             block_size=bs, ctx_lens=CTX, dtype=KV_FP8, seed=hq + bs)
    try:
        got, ref = run_prefill(case, LENS, hq, seed=hq * bs)
        err = rel_err(got, ref)
        print(f"prefill fp8 mfma G={hq // hkv} bs={bs} err={err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= TOL[KV_FP8]
    finally:
        case.pool.destroy()


def test_fp8_mfma_matches_generic(gpu_lib, tunables):
    """The fp8 MFMA path and the generic kernel (KCMM_ATTN_GENERIC) agree
    within the fp8 tolerance on the same pages and queries."""
    case = build_decode_case(gpu_lib, batch=len(CTX), num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=CTX, dtype=KV_FP8, seed=31)
    try:
        got, ref = run_prefill(case, LENS, 32, seed=32)
        tunables.setenv("KCMM_ATTN_GENERIC", "1")
        gen, _ = run_prefill(case, LENS, 32, seed=32)
        assert rel_err(got, gen) <= TOL[KV_FP8] and rel_err(gen, ref) <= TOL[KV_FP8]
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("dtype,hq,hkv,d", [(KV_FP8, 32, 8, 64), (KV_BF16, 12, 4, 80),
                                            (KV_F16, 24, 8, 64)])
def test_generic_path(gpu_lib, dtype, hq, hkv, d):
    """fp8 pages at head_dim 64, head_dim 80 and a group of 3 run on the
    generic kernel."""
    ctx, lens = [40, 9, 77], [13, 9, 30]
    case = build_decode_case(gpu_lib, batch=3, num_q_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=16, ctx_lens=ctx, dtype=dtype, seed=d)
    try:
        got, ref = run_prefill(case, lens, hq, seed=d)
        err = rel_err(got, ref)
        print(f"prefill generic dtype={dtype} D={d} err={err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= TOL[dtype]
    finally:
        case.pool.destroy()


def test_chunk_of_one_matches_decode(gpu_lib):
    """A one-token chunk is decode at the same length: prefill output equals
    the decode entry point's within bf16 tolerance."""
    import torch
    ctx = [40, 17, 300, 129]
    case = build_decode_case(gpu_lib, batch=4, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=KV_BF16, seed=21)
    try:
        got, ref = run_prefill(case, [1, 1, 1, 1], 32, seed=22)
        assert rel_err(got, ref) <= TOL[KV_BF16]
        # the same queries through decode
        qsl = np.arange(5, dtype=np.int32)
        rng = np.random.default_rng(22)
        q = encode16(KV_BF16, rng.standard_normal((4, 32, 128)).astype(np.float32))
        case.dev["q"] = torch.from_numpy(q.view(np.int16)).view(torch.bfloat16).cuda()
        case.run_attention(stream_ptr=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        dec = O.decode(O.BF16, case.out_bits()).astype(np.float64)
        assert rel_err(got, dec) <= TOL[KV_BF16]
        del qsl
    finally:
        case.pool.destroy()


def test_more_queries_than_tokens_gives_zero_rows(gpu_lib):
    """Seq 0 holds 5 tokens but has 8 queries: queries 0..2 would sit before
    position 0 and are written as zeros; 3..7 are positions 0..4.  Seq 1
    holds no token at all (no page is read)."""
    case = build_decode_case(gpu_lib, batch=3, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=[5, 0, 40], dtype=KV_BF16, seed=23)
    try:
        got, ref = run_prefill(case, [8, 4, 10], 32, seed=23)
        assert not got[:3].any() and not ref[:3].any()
        assert not got[8:12].any() and not ref[8:12].any()
        assert rel_err(got, ref) <= TOL[KV_BF16]
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_shared_prefix_chunked_prefill(gpu_lib, dtype):
    """BASELINE configs[2] layout at reduced batch: sequences share refcounted
    prefix pages (kcmm_share_prefix) and own their suffix; the chunk is the
    suffix.  Regions are read back for the oracle.  bf16 and fp8 pages."""
    import torch
    case = build_prefix_shared_case(gpu_lib, batch=4, prefix_tokens=1024, suffix_tokens=256,
                                    chunk=256, num_q_heads=32, kv_heads=8, head_dim=128,
                                    block_size=16, dtype=dtype, seed=24)
    try:
        pre = case.block_tables[:, :64]
        assert (pre == pre[0]).all()                       # same physical prefix pages
        assert case.pool.refcount(int(pre[0, 0])) == 4
        case.dev["out"].fill_(float("nan"))
        case.run(stream_ptr=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        st = case.pool.stats()
        mapped = st["superblock_count"] * 2 * 1024 * 1024
        kreg = memcpy_dtoh(case.pool.va_k(0), mapped)
        vreg = memcpy_dtoh(case.pool.va_v(0), mapped)
        got = O.decode(O.BF16, case.dev["out"].cpu().view(torch.int16).numpy().view(np.uint16))
        eb = 1 if dtype == KV_FP8 else 2
        ref = O.attn_prefill_f64(dtype, case.q_bits, kreg, vreg, case.block_tables,
                                 case.seq_lens, case.qsl, case.offsets_f16, 32, 8, 128, 16,
                                 8 * 128 * eb, 8 * 128 * eb * 16, 1 / math.sqrt(128))
        err = rel_err(got.astype(np.float64), ref)
        print(f"shared-prefix prefill dtype={dtype} err={err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= TOL[dtype]
    finally:
        case.pool.destroy()


def test_many_sequences_ragged_chunks(gpu_lib):
    """70 sequences (two 64-lane chunks in the workgroup -> (sequence,
    token block) lookup, which deals blocks longest first across
    sequences), chunk lengths 0..200 so sequences own 0..4 token blocks."""
    rng = np.random.default_rng(71)
    lens = rng.integers(0, 201, size=70)
    lens[[0, 63, 64, 69]] = [200, 0, 130, 1]
    ctx = lens + rng.integers(0, 120, size=70)
    ctx = np.maximum(ctx, 1)
    case = build_decode_case(gpu_lib, batch=70, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=KV_BF16, seed=72)
    try:
        got, ref = run_prefill(case, lens, 32, 73)
        err = rel_err(got, ref)
        print(f"70 sequences, {int(lens.sum())} queries, err={err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= TOL[KV_BF16]
    finally:
        case.pool.destroy()


def test_running_max_grows_on_most_tiles(gpu_lib):
    """Keys whose size grows along the sequence (row t scaled by 1 + t/8) make
    each column maximum grow by more than 8 (log2 units) on about a third of
    the tiles (6-9 of 22 at 700 keys), so a wave of 32 columns takes the
    rescale path on most tiles, where N(0,1) data stays on the fast path after
    the first; a spike (rows 300..363 four times larger) then holds the maxima
    for the tiles after it.  Against the oracle,
    ragged chunks, one sequence whose chunk is all of it."""
    ctx = [700, 257, 96, 33]
    lens = [200, 64, 96, 33]
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=KV_BF16, seed=91)
    try:
        g = case.geometry
        mk = case.k_mirror[0]
        rb = g["row_bytes"]
        for b, L in enumerate(ctx):
            for t in range(L):
                at = int(case.offsets_f16[case.block_tables[b, t // 16]]) * 2 + (t % 16) * rb
                vals = O.decode(O.BF16, mk[at:at + rb].view(np.uint16)).astype(np.float32)
                vals *= (1.0 + t / 8.0) * (4.0 if 300 <= t < 364 else 1.0)
                mk[at:at + rb] = encode16(KV_BF16, vals).view(np.uint8).reshape(-1)
        memcpy_htod(case.pool.va_k(0), mk)
        got, ref = run_prefill(case, lens, 32, seed=92)
        err = rel_err(got, ref)
        print(f"growing maxima: err={err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= TOL[KV_BF16]
    finally:
        case.pool.destroy()
