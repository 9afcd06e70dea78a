"""kcmm_paged_attn_decode_bf16_noalloc_on_stream: decode attention whose
scratch (partials, segment table) is a static device array, so the call
allocates nothing.  Checked through the C ABI against
kcmm_paged_attn_decode_bf16_on_stream on the same inputs (same kernels, so
the same bits), on two calls in a row, the second with a smaller input; a
batch whose scratch would not fit is refused with an error before any
device work."""
import ctypes as C
import math

import numpy as np
import pytest

from lattice_amd.bindings import KV_BF16, make_config
from lattice_amd.workload import build_decode_case

pytestmark = pytest.mark.gpu


def _call(case, fn, out, stream, batch=None):
    d = case.dev
    b = case.batch if batch is None else batch
    return fn(case.pool.handle, 0, d["q"].data_ptr(), out.data_ptr(), d["bt"].data_ptr(),
              d["sl"].data_ptr(), d["offs"].data_ptr(), b, case.num_q_heads, case.kv_heads,
              case.head_dim, case.block_size, case.mbps, C.c_float(1 / math.sqrt(case.head_dim)),
              stream)


def test_noalloc_matches_allocating_entry_point(gpu_lib):
    import torch
    lib = gpu_lib.lib
    rng = np.random.default_rng(3)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    # first call: the Llama-3-8B decode shape (Cfg2), second: a smaller batch
    for batch, lo, hi, seed in ((64, 512, 4096, 1), (9, 1, 700, 2)):
        ctx = rng.integers(lo, hi + 1, size=batch) + 1
        case = build_decode_case(gpu_lib, batch=batch, num_q_heads=32, kv_heads=8, head_dim=128,
                                 block_size=16, ctx_lens=ctx, dtype=KV_BF16, seed=seed,
                                 host_mirror=False)
        try:
            ref = torch.full_like(case.dev["out"], float("nan"))
            got = torch.full_like(case.dev["out"], float("nan"))
            assert _call(case, lib.kcmm_paged_attn_decode_bf16_on_stream, ref, sp) == 0
            assert _call(case, lib.kcmm_paged_attn_decode_bf16_noalloc_on_stream, got, sp) == 0, \
                case.pool.last_error()
            stream.synchronize()
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), batch
            assert torch.isfinite(got.float()).all()
        finally:
            case.pool.destroy()


def test_noalloc_calls_on_two_streams_take_turns(gpu_lib):
    """Back-to-back calls on two streams with no host synchronization in
    between share the one scratch array: each call on the other stream waits
    for the previous call's kernels, so every output equals the allocating
    entry point's (same kernels, same bits)."""
    import torch
    lib = gpu_lib.lib
    rng = np.random.default_rng(8)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    cases = []
    try:
        for batch, lo, hi, seed in ((64, 512, 4096, 11), (48, 256, 3000, 12)):
            ctx = rng.integers(lo, hi + 1, size=batch) + 1
            cases.append(build_decode_case(gpu_lib, batch=batch, num_q_heads=32, kv_heads=8,
                                           head_dim=128, block_size=16, ctx_lens=ctx,
                                           dtype=KV_BF16, seed=seed, host_mirror=False))
        refs = []
        for case in cases:
            ref = torch.full_like(case.dev["out"], float("nan"))
            assert _call(case, lib.kcmm_paged_attn_decode_bf16_on_stream, ref, 0) == 0
            refs.append(ref)
        torch.cuda.synchronize()
        outs = [[torch.full_like(c.dev["out"], float("nan")) for _ in range(3)] for c in cases]
        for rep in range(3):
            for case, out, st in zip(cases, outs, (s1, s2)):
                assert _call(case, lib.kcmm_paged_attn_decode_bf16_noalloc_on_stream, out[rep],
                             st.cuda_stream) == 0, case.pool.last_error()
        torch.cuda.synchronize()
        for ref, out in zip(refs, outs):
            for rep, o in enumerate(out):
                assert torch.equal(o.view(torch.int16), ref.view(torch.int16)), rep
    finally:
        for case in cases:
            case.pool.destroy()


def test_noalloc_refuses_batches_past_its_scratch(gpu_lib):
    """400 sequences of long tables need more than the static scratch: the
    call fails with an error naming the sizes; the inputs are real
    (one-token sequences over one page) so nothing would read past them."""
    import torch
    lib = gpu_lib.lib
    B, mbps = 400, 512
    pool = gpu_lib.create_pool(make_config(num_layers=1, kv_heads=8, head_dim=128, max_batch=B,
                                           max_seq_len=mbps * 16), KV_BF16)
    try:
        blk = pool.alloc_blocks(1)[0]
        q = torch.zeros((B, 32, 128), dtype=torch.bfloat16, device="cuda")
        out = torch.zeros_like(q)
        bt = torch.full((B, mbps), blk, dtype=torch.int32, device="cuda")
        sl = torch.full((B,), mbps * 16, dtype=torch.int32, device="cuda")
        offs = torch.tensor(pool.all_block_offsets_f16(), dtype=torch.int64, device="cuda")
        rc = lib.kcmm_paged_attn_decode_bf16_noalloc_on_stream(
            pool.handle, 0, q.data_ptr(), out.data_ptr(), bt.data_ptr(), sl.data_ptr(),
            offs.data_ptr(), B, 32, 8, 128, 16, mbps, C.c_float(0.088), 0)
        assert rc == -1
        assert "static scratch" in pool.last_error()
    finally:
        pool.destroy()
