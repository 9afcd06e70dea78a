"""Seeded random sweeps of the decode and prefill attention entry points and
the projection GEMMs against the oracle (fp64), over combinations the
hand-picked cases do not list together.  Attention: page type, GQA group,
head_dim, block size, batch, ragged lengths (empty, one token, tile and page
edges), softmax scale, and the decode kernel's work split (total waves, waves
per workgroup, minimum slice, tiles in flight).  GEMM: shapes around the
kernel dispatch boundaries, bf16 or fp8 weights, the residual form, forced K
splits and workgroup widths.  Decoder layer: head shapes, hidden and
intermediate sizes, bf16 or fp8 pools, ragged batches, checked stage by stage
and end to end.  Every case prints its parameters before it runs.
Tolerances as the other tests: bf16 / f16 1e-2, fp8 pages 3e-2, GEMM 1e-2;
the layer's stages 1e-2 (3e-2 on fp8 pools) and its end-to-end bounds as
test_gpu_glue.test_decode_layer_step."""
import math

import numpy as np
import pytest

from lattice_amd.bindings import KV_BF16, KV_F16, KV_FP8
from lattice_amd.workload import build_decode_case
from tests.test_gpu_attention import check as check_decode
from tests.test_gpu_prefill import TOL, rel_err, run_prefill

pytestmark = pytest.mark.gpu

GROUPS = [(8, 8), (16, 8), (32, 8), (32, 4), (16, 2), (32, 2), (16, 1), (12, 4), (10, 5)]


def ragged_lengths(rng, batch, block_size, max_len):
    """Lengths drawn from a mix of edge cases and uniform values."""
    edges = [0, 1, 2, block_size - 1, block_size, block_size + 1, 31, 32, 33, 63, 64, 65]
    out = []
    for _ in range(batch):
        r = rng.random()
        if r < 0.35:
            out.append(int(rng.choice(edges)))
        elif r < 0.5:
            k = int(rng.integers(1, max(2, max_len // 32)))
            out.append(int(32 * k + rng.integers(-1, 2)))
        else:
            out.append(int(rng.integers(1, max_len + 1)))
    if max(out) <= 0:
        out[0] = 1
    return [max(0, min(x, max_len)) for x in out]


def decode_params(seed):
    rng = np.random.default_rng(1000 + seed)
    dtype = [KV_BF16, KV_F16, KV_FP8][seed % 3]
    hq, hkv = GROUPS[int(rng.integers(len(GROUPS)))]
    d = 128 if dtype == KV_FP8 or rng.random() < 0.6 else 64
    bs = int(rng.choice([8, 16, 32]))
    batch = int(rng.integers(1, 25))
    ctx = ragged_lengths(rng, batch, bs, int(rng.choice([200, 700, 1500])))
    scale = float(rng.choice([1.0 / math.sqrt(d), 0.05, 0.2]))
    tun = {}
    if rng.random() < 0.6:
        tun["KCMM_ATTN_WAVES"] = str(int(rng.choice([64, 256, 1024, 3000])))
    if rng.random() < 0.4:
        tun["KCMM_ATTN_HW"] = str(int(rng.choice([1, 2, 4, 8])))
    if rng.random() < 0.4:
        tun["KCMM_ATTN_MIN_TILES"] = str(int(rng.choice([1, 2, 8, 40])))
    if rng.random() < 0.3:
        tun["KCMM_ATTN_DEPTH"] = "3"
    return dtype, hq, hkv, d, bs, ctx, scale, tun


@pytest.mark.parametrize("seed", range(30))
def test_decode_attention_random(gpu_lib, tunables, seed):
    dtype, hq, hkv, d, bs, ctx, scale, tun = decode_params(seed)
    print(f"decode seed={seed} dtype={dtype} Hq={hq} Hkv={hkv} D={d} bs={bs} B={len(ctx)} "
          f"ctx={ctx} scale={scale:.4f} tunables={tun}", flush=True)
    for k, v in tun.items():
        tunables.setenv(k, v)
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=bs, ctx_lens=ctx, dtype=dtype, seed=seed)
    try:
        check_decode(case, scale=scale)
    finally:
        case.pool.destroy()


def prefill_params(seed):
    rng = np.random.default_rng(2000 + seed)
    dtype = [KV_BF16, KV_F16, KV_FP8][seed % 3]
    hq, hkv = GROUPS[int(rng.integers(len(GROUPS)))]
    d = 128 if dtype == KV_FP8 or rng.random() < 0.6 else 64
    bs = int(rng.choice([8, 16, 32]))
    batch = int(rng.integers(1, 9))
    ctx = [max(1, x) for x in ragged_lengths(rng, batch, bs, int(rng.choice([120, 400])))]
    lens = [int(rng.integers(1, L + 1)) if rng.random() < 0.8 else L for L in ctx]
    scale = float(rng.choice([1.0 / math.sqrt(d), 0.05]))
    return dtype, hq, hkv, d, bs, ctx, lens, scale


@pytest.mark.parametrize("seed", range(18))
def test_prefill_attention_random(gpu_lib, seed):
    dtype, hq, hkv, d, bs, ctx, lens, scale = prefill_params(seed)
    print(f"prefill seed={seed} dtype={dtype} Hq={hq} Hkv={hkv} D={d} bs={bs} ctx={ctx} "
          f"lens={lens} scale={scale:.4f}", flush=True)
    case = build_decode_case(gpu_lib, batch=len(ctx), num_q_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=bs, ctx_lens=ctx, dtype=dtype, seed=seed + 50)
    try:
        got, ref = run_prefill(case, lens, hq, seed=seed + 60, scale=scale)
        err = rel_err(got, ref)
        print(f"  err={err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= TOL[dtype], err
    finally:
        case.pool.destroy()


def gemm_params(seed):
    rng = np.random.default_rng(3000 + seed)
    edges = [1, 2, 16, 17, 32, 33, 64, 65, 127, 128, 129, 200, 255, 256, 257, 300]
    m = int(rng.choice(edges)) if rng.random() < 0.7 else int(rng.integers(1, 301))
    n = 64 * int(rng.integers(1, 41))
    k = 256 * int(rng.integers(1, 13))
    fp8 = seed % 3 == 2
    residual = not fp8 and rng.random() < 0.4
    tun = {}
    if rng.random() < 0.4:
        tun["KCMM_GEMM_SPLITS"] = str(int(rng.choice([1, 2, 4, 8])))
    if rng.random() < 0.3:
        tun["KCMM_GEMM_TILED"] = "0"
    if rng.random() < 0.3:
        tun["KCMM_GEMM_WAVES"] = "4"
    if rng.random() < 0.3:
        tun["KCMM_GEMM_HELPERS"] = "0"
    return m, n, k, fp8, residual, tun


@pytest.mark.parametrize("seed", range(24))
def test_gemm_random(gpu_lib, tunables, seed):
    """kcmm_gemm_bf16 / kcmm_gemm_bf16_add / kcmm_gemm_fp8w_bf16 on random
    shapes around the dispatch boundaries (M = 128 / 129 between the
    weight-stream and tiled kernels, N not a multiple of 128, forced K
    splits) against the fp64 oracle (1e-2); a repeated call gives the same
    bits."""
    import torch
    import oracle as O
    m, n, k, fp8, residual, tun = gemm_params(seed)
    print(f"gemm seed={seed} m={m} n={n} k={k} fp8={fp8} residual={residual} tunables={tun}",
          flush=True)
    for name, v in tun.items():
        tunables.setenv(name, v)
    rng = np.random.default_rng(seed + 70)
    xb = O.encode(O.BF16, rng.standard_normal((m, k)))
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    rb = O.encode(O.BF16, rng.standard_normal((m, n)))
    s = torch.cuda.current_stream().cuda_stream
    if fp8:
        w8, sc = O.quantize_fp8_rows(rng.standard_normal((n, k)).astype(np.float32) * 0.02)
        w8d, scd = torch.from_numpy(w8).cuda(), torch.from_numpy(sc).cuda()
        ref = O.gemm_fp8w_f64(xb, w8, sc)
    else:
        wb = O.encode(O.BF16, rng.standard_normal((n, k)) * 0.02)
        w = torch.from_numpy(wb.view(np.int16)).view(torch.bfloat16).cuda()
        ref = O.gemm_bf16_f64(xb, wb)
        if residual:
            ref = O.decode(O.BF16, O.encode(O.BF16, ref)).astype(np.float64) + \
                O.decode(O.BF16, rb).astype(np.float64)
    outs = []
    for _ in range(2):
        if residual:
            y = torch.from_numpy(rb.view(np.int16)).view(torch.bfloat16).cuda()
            gpu_lib.gemm_bf16_add(x.data_ptr(), w.data_ptr(), y.data_ptr(), y.data_ptr(), m, n, k, s)
        else:
            y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
            if fp8:
                gpu_lib.gemm_fp8w_bf16(x.data_ptr(), w8d.data_ptr(), scd.data_ptr(), y.data_ptr(),
                                       m, n, k, s)
            else:
                gpu_lib.gemm_bf16(x.data_ptr(), w.data_ptr(), y.data_ptr(), m, n, k, s)
        torch.cuda.synchronize()
        outs.append(y.cpu().view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(outs[0], outs[1])
    got = O.decode(O.BF16, outs[0]).astype(np.float64)
    err = float(np.abs(got - ref).max() / np.abs(ref).max())
    print(f"  err={err:.3e}", flush=True)
    assert np.isfinite(got).all() and err <= 1e-2, err


LAYER_HEADS = [(8, 2, 64), (16, 4, 64), (16, 8, 128), (8, 8, 128), (32, 4, 128), (32, 8, 128)]


def layer_params(seed):
    rng = np.random.default_rng(4000 + seed)
    hq, hkv, d = LAYER_HEADS[int(rng.integers(len(LAYER_HEADS)))]
    h = int(rng.choice([512, 1024, 2048]))
    inter = int(rng.choice([512, 768, 1024, 1536]))
    dtype = KV_FP8 if seed % 3 == 2 and d == 128 else KV_BF16
    batch = int(rng.integers(1, 41))
    lens = [max(1, x) for x in ragged_lengths(rng, batch, 16, int(rng.choice([100, 300])))]
    return hq, hkv, d, h, inter, dtype, lens


@pytest.mark.parametrize("seed", range(12))
def test_decode_layer_random(gpu_lib, seed):
    """kcmm_decode_layer_step_on_stream on random layer shapes, pool types,
    batches and ragged lengths: every stage against the oracle's stage
    (tests/layer_stages.py), the fused step against its components bit for
    bit, and the whole layer against the oracle's layer (as
    test_gpu_glue.test_decode_layer_step)."""
    import torch
    import oracle as O
    from lattice_amd.bindings import memcpy_htod
    from tests import layer_stages as LS
    from tests.test_gpu_glue import _layer_weights, _region, bf16_dev, bits_of
    from tests.test_gpu_glue import rel_err as rel_err_glue
    hq, hkv, d, h, inter, dtype, lens = layer_params(seed)
    print(f"layer seed={seed} Hq={hq} Hkv={hkv} D={d} h={h} inter={inter} dtype={dtype} "
          f"lens={lens}", flush=True)
    fp8 = dtype == KV_FP8
    case = build_decode_case(gpu_lib, batch=len(lens), num_q_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=16, ctx_lens=lens, dtype=dtype, seed=seed + 80)
    try:
        g = case.geometry
        rng = np.random.default_rng(seed + 90)
        w, wdev, lw = _layer_weights(torch, rng, h, inter, hq, hkv, d)
        hid = O.encode(O.BF16, rng.standard_normal((len(lens), h)))
        inv = O.default_inv_freq(500000.0, d)
        invd = torch.from_numpy(inv.astype(np.float32)).cuda()
        dv = case.dev
        stream = torch.cuda.current_stream().cuda_stream
        st = LS.run_stages(gpu_lib, case, wdev, hid, invd, hq, h, inter, 1e-5, stream)
        errs = LS.check_stages(st, case, w, inv, hq, inter, 1e-5, dtype)
        print("  stages " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
        kreg, vreg = st["kv0"]
        memcpy_htod(case.pool.va_k(0), kreg)
        memcpy_htod(case.pool.va_v(0), vreg)
        hd = bf16_dev(torch, hid)
        case.pool.decode_layer_step(layer_idx=0, weights=lw, hidden_ptr=hd.data_ptr(),
                                    block_tables_ptr=dv["bt"].data_ptr(),
                                    seq_lens_ptr=dv["sl"].data_ptr(),
                                    block_offsets_f16_ptr=dv["offs"].data_ptr(),
                                    inv_freq_ptr=invd.data_ptr(), batch=len(lens),
                                    hidden_size=h, num_q_heads=hq, intermediate_size=inter,
                                    max_blocks_per_seq=case.mbps, rms_eps=1e-5,
                                    stream_ptr=stream)
        torch.cuda.synchronize()
        assert np.array_equal(bits_of(hd), st["out"]), "layer step != its components"
        assert np.array_equal(_region(case, "k"), st["kv1"][0])
        assert np.array_equal(_region(case, "v"), st["kv1"][1])
        got = O.decode(O.BF16, bits_of(hd)).astype(np.float64)
        ref = O.decode_layer_step_f64(hid, w, kreg.copy(), vreg.copy(), case.block_tables,
                                      case.seq_lens, case.offsets_f16, inv, hq, hkv, d, inter, 16,
                                      g["row_bytes"], 1e-5, dtype=dtype,
                                      data_bytes=g["data_bytes"])
        x = O.decode(O.BF16, hid).astype(np.float64)
        err = rel_err_glue(got, ref)
        upd = rel_err_glue(got - x, ref - x)
        print(f"  layer err {err:.2e}, update err {upd:.2e}", flush=True)
        assert np.isfinite(got).all() and err <= (3e-2 if fp8 else 1e-2)
        assert upd <= (1.75e-2 if fp8 else 1.25e-2)
    finally:
        case.pool.destroy()
