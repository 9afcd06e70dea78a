"""Paged decode attention on the GPU through the C ABI vs the oracle.

Tolerance (relative to the output's scale, max|got-ref| / max|ref|): bf16
1e-2, fp8 KV 3e-2 (against the oracle on the same dequantized pages), f16
1e-2 (BASELINE tolerances; f16 shares bf16's since outputs and P are 16-bit).
"""
import math

import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, KV_F16, KV_FP8, memcpy_dtoh, memcpy_htod
from lattice_amd.workload import build_decode_case

pytestmark = pytest.mark.gpu

TOL = {KV_BF16: 1e-2, KV_F16: 1e-2, KV_FP8: 3e-2}


def oracle_out(case, layer=0, scale=None, regions=None):
    g = case.geometry
    scale = 1 / math.sqrt(case.head_dim) if scale is None else scale
    kreg, vreg = regions if regions else (case.k_mirror[layer], case.v_mirror[layer])
    return O.attn_decode_f64(case.dtype, case.q_bits, kreg, vreg, case.block_tables,
                             case.seq_lens, case.offsets_f16, case.num_q_heads, case.kv_heads,
                             case.head_dim, case.block_size, g["row_bytes"], g["data_bytes"],
                             scale)


def gpu_out(case):
    bits = case.out_bits()
    return O.decode(O.F16 if case.dtype == KV_F16 else O.BF16, bits).astype(np.float64)


def rel_err(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def check(case, **kw):
    import torch
    case.dev["out"].fill_(float("nan"))
    case.run_attention(**kw)
    torch.cuda.synchronize()
    got, ref = gpu_out(case), oracle_out(case, scale=kw.get("scale"))
    err = rel_err(got, ref)
    print(f"shape B={case.batch} Hq={case.num_q_heads} Hkv={case.kv_heads} D={case.head_dim} "
          f"bs={case.block_size} dtype={case.dtype} max_len={case.seq_lens.max()} err={err:.3e}",
          flush=True)
    assert np.isfinite(got).all()
    assert err <= TOL[case.dtype], err
    zero = case.seq_lens <= 0
    assert not got[zero].any()
    return err


@pytest.mark.parametrize("dtype", [KV_BF16, KV_F16])
def test_llama3_8b_shape_reduced_batch(gpu_lib, dtype):
    rng = np.random.default_rng(100 + dtype)
    ctx = rng.integers(512, 4097, size=8) + 1          # BASELINE configs[1], 8 of 64 seqs
    case = build_decode_case(gpu_lib, batch=8, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=dtype, seed=1)
    try:
        check(case)
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("dtype", [KV_BF16, KV_F16])
def test_ragged_lengths_and_chunk_edges(gpu_lib, dtype):
    ctx = [0, 1, 2, 15, 16, 17, 31, 32, 33, 63, 255, 256, 257, 511, 512, 513, 1024, 1025, -3]
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=dtype, seed=2)
    try:
        check(case)
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("hq,hkv,d,bs", [
    (8, 8, 64, 16),      # BASELINE configs[0] geometry (MHA)
    (16, 8, 128, 16),
    (32, 2, 128, 16),    # group 16 (largest MFMA path)
    (8, 1, 256, 16),
    (32, 8, 128, 32),    # block size not 16: runtime divide path
    (12, 4, 64, 8),
    (24, 6, 128, 16),    # 6 kv heads
])
def test_mfma_path_shapes(gpu_lib, hq, hkv, d, bs):
    rng = np.random.default_rng(hq * d + bs)
    ctx = rng.integers(1, 700, size=5)
    case = build_decode_case(gpu_lib, batch=5, num_q_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=bs, ctx_lens=ctx, dtype=KV_BF16, seed=3)
    try:
        check(case)
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("hw,hq,hkv", [("4", 24, 6), ("8", 24, 12), ("8", 10, 5)])
@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_head_block_not_dividing(gpu_lib, tunables, hw, hq, hkv, dtype):
    """Workgroups take the largest divisor of Hkv not above KCMM_ATTN_HW
    (6 kv heads at 4 -> 3, 12 at 8 -> 6, 5 at 8 -> 5)."""
    tunables.setenv("KCMM_ATTN_HW", hw)
    rng = np.random.default_rng(hq + hkv)
    ctx = rng.integers(1, 900, size=7)
    case = build_decode_case(gpu_lib, batch=7, num_q_heads=hq, kv_heads=hkv, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=dtype, seed=12)
    try:
        check(case)
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("hq,hkv,d,bs", [(6, 4, 80, 8), (32, 1, 96, 16), (40, 8, 128, 16),
                                        (4, 2, 66, 3), (8, 8, 256, 5), (3, 3, 8, 16)])
def test_generic_path_shapes(gpu_lib, hq, hkv, d, bs):
    # head_dim not in {64,128,256} (66: not a multiple of 4, element loads),
    # Hq not a multiple of Hkv, group > 16, block sizes not a multiple of 8
    ctx = [1, 40, 129, 0]
    case = build_decode_case(gpu_lib, batch=4, num_q_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=bs, ctx_lens=ctx, dtype=KV_F16, seed=4)
    try:
        check(case)
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("dtype", [KV_BF16, KV_F16, KV_FP8])
@pytest.mark.parametrize("bs,ctx", [(16, [2500, 1, 1024, 1025, 0, 700]), (1, [1100, 3, 2049])])
def test_generic_kernel_forced(gpu_lib, tunables, dtype, bs, ctx):
    """KCMM_ATTN_GENERIC forces the any-shape kernel at the Llama-3-8B head
    shape: contexts across its 1024-position staging chunks (and exactly at
    their edges), one-token pages, an empty sequence."""
    tunables.setenv("KCMM_ATTN_GENERIC", "1")
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=bs, ctx_lens=ctx, dtype=dtype, seed=21 + bs)
    try:
        check(case)
    finally:
        case.pool.destroy()


def test_generic_kernel_many_pairs(gpu_lib, tunables):
    """1280 (sequence, head) pairs: the any-shape kernel's 256-lane
    workgroups."""
    tunables.setenv("KCMM_ATTN_GENERIC", "1")
    rng = np.random.default_rng(77)
    ctx = rng.integers(0, 700, size=40)
    case = build_decode_case(gpu_lib, batch=40, num_q_heads=32, kv_heads=8, head_dim=64,
                             block_size=16, ctx_lens=ctx, dtype=KV_BF16, seed=77)
    try:
        check(case)
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("bs", [16, 32, 8])
def test_fp8_pages(gpu_lib, bs):
    """fp8-e4m3 pages (per (page, kv head) scales in the page footer) against
    the oracle over the same dequantized pages; block sizes 16, 32 and 8
    move the 8-token groups across page boundaries differently."""
    rng = np.random.default_rng(5 + bs)
    ctx = rng.integers(1, 900, size=6)
    case = build_decode_case(gpu_lib, batch=6, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=bs, ctx_lens=ctx, dtype=KV_FP8, seed=5)
    try:
        import torch
        case.dev["out"].fill_(float("nan"))
        case.run_attention(stream_ptr=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        err = rel_err(gpu_out(case), oracle_out(case))
        print(f"fp8 err={err:.3e}", flush=True)
        assert err <= TOL[KV_FP8]
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("dtype", [KV_F16, KV_BF16])
def test_seq_len_one_returns_v_row_exactly(gpu_lib, dtype):
    """ref non_default_stream_ffi_smoke.py:172-179,334-343 (q = 0, exact)."""
    import torch
    case = build_decode_case(gpu_lib, batch=3, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=[1, 1, 1], dtype=dtype, seed=6)
    try:
        case.dev["q"].zero_()
        case.run_attention(scale=1.0, stream_ptr=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        out = case.out_bits()
        g = case.geometry
        for b in range(3):
            page = int(case.offsets_f16[case.block_tables[b, 0]]) * 2
            v = case.v_mirror[0][page:page + g["row_bytes"]].view(np.uint16).reshape(8, 128)
            for h in range(32):
                assert np.array_equal(out[b, h], v[h * 8 // 32]), (b, h)
    finally:
        case.pool.destroy()


def test_entry_point_variants_agree(gpu_lib):
    import torch
    ctx = [300, 5, 2000]
    case = build_decode_case(gpu_lib, batch=3, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=KV_F16, seed=7)
    try:
        outs = []
        s = torch.cuda.Stream()
        for kw in [dict(), dict(stream_ptr=s.cuda_stream),
                   dict(stream_ptr=s.cuda_stream, variant="current_context")]:
            case.dev["out"].zero_()
            torch.cuda.synchronize()
            d = case.dev
            case.pool.paged_attn_decode(
                layer_idx=0, query_ptr=d["q"].data_ptr(), out_ptr=d["out"].data_ptr(),
                block_tables_ptr=d["bt"].data_ptr(), seq_lens_ptr=d["sl"].data_ptr(),
                block_offsets_f16_ptr=d["offs"].data_ptr(), batch=3, num_q_heads=32, kv_heads=8,
                head_dim=128, block_size=16, max_blocks_per_seq=case.mbps, scale=0.088, **kw)
            torch.cuda.synchronize()
            outs.append(case.out_bits().copy())
        assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    finally:
        case.pool.destroy()


@pytest.fixture(params=["default", "depth3", "many_waves", "four_heads_per_wg", "all_heads_per_wg"])
def stream_tuning(request, tunables):
    """Streaming-kernel settings: the default, three tiles in flight, a tiny
    slice per workgroup (every (b, kv head) split over many slices, so the
    log-sum-exp merge runs everywhere), and workgroups of four waves (four
    kv heads) or of eight waves (all kv heads of a token row); the default
    is one wave per workgroup for 16-bit pages, eight for fp8."""
    if request.param == "depth3":
        tunables.setenv("KCMM_ATTN_DEPTH", "3")
    elif request.param == "many_waves":
        tunables.setenv("KCMM_ATTN_WAVES", "4096")
        tunables.setenv("KCMM_ATTN_MIN_TILES", "1")
    elif request.param == "four_heads_per_wg":
        tunables.setenv("KCMM_ATTN_HW", "4")
    elif request.param == "all_heads_per_wg":
        tunables.setenv("KCMM_ATTN_HW", "8")
        tunables.setenv("KCMM_ATTN_WAVES", "2048")
        tunables.setenv("KCMM_ATTN_MIN_TILES", "2")
    return request.param


@pytest.mark.parametrize("dtype", [KV_BF16, KV_F16, KV_FP8])
def test_stream_settings_ragged(gpu_lib, stream_tuning, dtype):
    ctx = [0, 1, 33, 4100, 31, 32, 64, 2049, -1, 700, 17, 1500]
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=dtype, seed=9)
    try:
        check(case)
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_many_short_sequences(gpu_lib, stream_tuning, dtype):
    """130 sequences (three 64-lane chunks of the slice lookup) of 0..40
    tokens: most (b, kv head) pairs are a single tile, so the query rows
    switch at nearly every tile."""
    rng = np.random.default_rng(10)
    ctx = rng.integers(-2, 41, size=130)
    ctx[[0, 64, 65, 129]] = 0
    case = build_decode_case(gpu_lib, batch=130, num_q_heads=16, kv_heads=4, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=dtype, seed=10)
    try:
        check(case)
    finally:
        case.pool.destroy()


def test_head_dim_64_stream(gpu_lib, stream_tuning):
    rng = np.random.default_rng(11)
    ctx = rng.integers(1, 900, size=9)
    case = build_decode_case(gpu_lib, batch=9, num_q_heads=8, kv_heads=8, head_dim=64,
                             block_size=16, ctx_lens=ctx, dtype=KV_F16, seed=11)
    try:
        check(case)
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_nan_in_unused_page_rows(gpu_lib, dtype):
    """Rows of a sequence's last page past seq_len may hold any bits; they
    must not reach the output (the kernel reads whole 8-token groups)."""
    ctx = [5, 17, 40, 100, 1]
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=dtype, seed=12)
    try:
        g = case.geometry
        if dtype == KV_FP8:
            nan_row = np.full(g["row_bytes"], 0x7F, dtype=np.uint8)      # e4m3 NaN
        else:
            nan_row = np.full(g["row_bytes"] // 2, 0x7FC1, dtype=np.uint16)
        for b, L in enumerate(ctx):
            last = (L - 1) // 16
            page = int(case.offsets_f16[case.block_tables[b, last]]) * 2
            for slot in range(L - last * 16, 16):
                off = page + slot * g["row_bytes"]
                memcpy_htod(case.pool.va_k(0) + off, nan_row)
                memcpy_htod(case.pool.va_v(0) + off, nan_row)
        check(case)
    finally:
        case.pool.destroy()


def test_full_llama3_8b_decode_shape(gpu_lib):
    """BASELINE configs[1] at full size (64 seqs, ctx U[512,4096] + 1): the
    GPU result against the oracle run on the device regions read back."""
    import torch
    rng = np.random.default_rng(2024)
    ctx = rng.integers(512, 4097, size=64) + 1
    case = build_decode_case(gpu_lib, batch=64, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=KV_BF16, seed=8,
                             host_mirror=False)
    try:
        case.run_attention(stream_ptr=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        g = case.geometry
        kreg = memcpy_dtoh(case.pool.va_k(0), g["mapped_bytes"])
        vreg = memcpy_dtoh(case.pool.va_v(0), g["mapped_bytes"])
        err = rel_err(gpu_out(case), oracle_out(case, regions=(kreg, vreg)))
        print(f"full Cfg2 err={err:.3e}", flush=True)
        assert err <= TOL[KV_BF16]
    finally:
        case.pool.destroy()


def test_fp8_device_filled_long_contexts(gpu_lib):
    """fp8 pages quantized on the device (the Cfg5 fill) at a larger shape:
    32 sequences of up to 6000 tokens, regions read back for the oracle."""
    import torch
    rng = np.random.default_rng(2025)
    ctx = rng.integers(512, 6001, size=32)
    ctx[3] = 16 * 7 + 1            # one page plus one token
    case = build_decode_case(gpu_lib, batch=32, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=KV_FP8, seed=13,
                             host_mirror=False)
    try:
        case.run_attention(stream_ptr=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        g = case.geometry
        kreg = memcpy_dtoh(case.pool.va_k(0), g["mapped_bytes"])
        vreg = memcpy_dtoh(case.pool.va_v(0), g["mapped_bytes"])
        err = rel_err(gpu_out(case), oracle_out(case, regions=(kreg, vreg)))
        print(f"fp8 device-filled err={err:.3e}", flush=True)
        assert err <= TOL[KV_FP8]
    finally:
        case.pool.destroy()


def test_stream_kernel_timing(gpu_lib):
    """kcmm_attn_stream_timing_start / stop: one event pair per streaming-kernel
    launch, an average below the whole call's (which adds the merge), the
    output unchanged by the timing, and errors for a stop without a start and
    a second start."""
    import torch
    from lattice_amd.bindings import KcmmError
    ctx = [900, 1, 33, 2500, 64, 700, 17, 1500]
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=KV_BF16, seed=77)
    try:
        sp = torch.cuda.current_stream().cuda_stream
        case.run_attention(stream_ptr=sp)
        torch.cuda.synchronize()
        ref = case.out_bits().copy()
        with pytest.raises(KcmmError):
            gpu_lib.attn_stream_timing_stop()
        gpu_lib.attn_stream_timing_start(8)
        with pytest.raises(KcmmError):
            gpu_lib.attn_stream_timing_start(8)
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record()
        for _ in range(3):
            case.run_attention(stream_ptr=sp)
        eb.record()
        torch.cuda.synchronize()
        avg_us, n = gpu_lib.attn_stream_timing_stop()
        call_us = ea.elapsed_time(eb) * 1e3 / 3
        print(f"stream kernel {avg_us:.2f} us, call {call_us:.2f} us, {n} launches", flush=True)
        assert n == 3 and 0 < avg_us < call_us
        assert np.array_equal(case.out_bits(), ref)
        # off again: launches take no event pair
        case.run_attention(stream_ptr=sp)
        gpu_lib.attn_stream_timing_start(2)
        _, n0 = gpu_lib.attn_stream_timing_stop()
        assert n0 == 0
    finally:
        case.pool.destroy()
