"""Fused projection epilogues on the GPU, through the C ABI.

The fused entry points must give the same bits as the unfused pair they
replace (same GEMM arithmetic, then the same element arithmetic):
  kcmm_gemm_bf16_swiglu        == kcmm_gemm_bf16 -> kcmm_silu_mul_bf16
  kcmm_qkv_rope_append_bf16    == kcmm_gemm_bf16 -> kcmm_rope_append_bf16
  kcmm_gemm_bf16_add_rmsnorm   == kcmm_gemm_bf16_add -> kcmm_rmsnorm_bf16
(the unfused GEMM on the weight-stream kernel: KCMM_GEMM_TILED=0).  The
unfused kernels are themselves checked against the oracle
(tests/test_gpu_glue.py, tests/test_gpu_gemm.py).  Shapes cover both the
single-pass GEMM (epilogue in its store) and the split-K path whose fp32
partials are summed, in split order, by the finishing kernel."""
import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, memcpy_dtoh
from lattice_amd.workload import build_decode_case, rope_inv_freq

pytestmark = pytest.mark.gpu


def _bits(t):
    import torch
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _randn_bf16(torch, shape, std, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * std).to(torch.bfloat16)


@pytest.mark.parametrize("m,inter,k", [(5, 256, 512), (64, 1024, 4096), (64, 14336, 4096),
                                       (100, 512, 1024), (256, 768, 2048)])
def test_swiglu_gemm_matches_unfused(gpu_lib, tunables, m, inter, k):
    import torch
    tunables.setenv("KCMM_GEMM_TILED", "0")   # the unfused GEMM on the same kernel
    x = _randn_bf16(torch, (m, k), 1.0, 1)
    w = _randn_bf16(torch, (2 * inter, k), 0.05, 2)
    gu = torch.empty((m, 2 * inter), dtype=torch.bfloat16, device="cuda")
    act_ref = torch.full((m, inter), float("nan"), dtype=torch.bfloat16, device="cuda")
    act = torch.full((m, inter), float("nan"), dtype=torch.bfloat16, device="cuda")
    sp = torch.cuda.current_stream().cuda_stream
    gpu_lib.gemm_bf16(x.data_ptr(), w.data_ptr(), gu.data_ptr(), m, 2 * inter, k, sp)
    gpu_lib.silu_mul_bf16(gu.data_ptr(), act_ref.data_ptr(), m, inter, sp)
    gpu_lib.gemm_bf16_swiglu(x.data_ptr(), w.data_ptr(), act.data_ptr(), m, inter, k, sp)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(act), _bits(act_ref))
    # and the unfused pair against the oracle at one row (bf16 tolerance)
    g = O.gemm_bf16_f64(_bits(x)[:1], _bits(w))
    gb = O.bf16_round(g)
    gate = gb[:, :inter]
    ref = O.bf16_round(O.bf16_round(gate / (1.0 + np.exp(-gate))) * gb[:, inter:])
    got = O.decode(O.BF16, _bits(act)[:1]).astype(np.float64)
    assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()


@pytest.mark.parametrize("hq,hkv,d,h,nseq", [(32, 8, 128, 4096, 6), (8, 2, 64, 256, 6),
                                              (12, 4, 80, 512, 6), (32, 8, 128, 256, 6),
                                              (8, 2, 128, 1024, 160)])
def test_qkv_rope_append_matches_unfused(gpu_lib, tunables, hq, hkv, d, h, nseq):
    """q_out and every byte of both regions identical between the fused QKV
    projection and projection -> RoPE/append; ragged lengths, a sequence
    with no token and one whose position lies past its table (both
    skipped: their q_out rows keep the NaN fill)."""
    import torch
    tunables.setenv("KCMM_GEMM_TILED", "0")   # the unfused GEMM on the same kernel
    lens = ([1, 16, 17, 300, 0, 48] * (nseq // 6 + 1))[:nseq]
    B = len(lens)
    n = (hq + 2 * hkv) * d
    if n % 64:
        pytest.skip("fused QKV needs (Hq + 2 Hkv) * head_dim % 64 == 0")
    outs = []
    for fused in (False, True):
        case = build_decode_case(gpu_lib, batch=B, num_q_heads=hq, kv_heads=hkv, head_dim=d,
                                 block_size=16, ctx_lens=lens, dtype=KV_BF16, seed=3)
        try:
            x = _randn_bf16(torch, (B, h), 1.0, 4)
            w = _randn_bf16(torch, (n, h), 0.05, 5)
            inv = torch.from_numpy(rope_inv_freq(500000.0, d)).cuda()
            qo = torch.full((B, hq, d), float("nan"), dtype=torch.bfloat16, device="cuda")
            dv = case.dev
            dv["sl"][1] = case.mbps * 16 + 3           # position past the table
            sp = torch.cuda.current_stream().cuda_stream
            common = dict(layer_idx=0, q_out_ptr=qo.data_ptr(), block_tables_ptr=dv["bt"].data_ptr(),
                          seq_lens_ptr=dv["sl"].data_ptr(),
                          block_offsets_f16_ptr=dv["offs"].data_ptr(), inv_freq_ptr=inv.data_ptr(),
                          batch=B, num_q_heads=hq, max_blocks_per_seq=case.mbps, stream_ptr=sp)
            if fused:
                case.pool.qkv_rope_append(x_ptr=x.data_ptr(), w_qkv_ptr=w.data_ptr(),
                                          hidden_size=h, **common)
            else:
                qkv = torch.empty((B, n), dtype=torch.bfloat16, device="cuda")
                gpu_lib.gemm_bf16(x.data_ptr(), w.data_ptr(), qkv.data_ptr(), B, n, h, sp)
                case.pool.rope_append(qkv_ptr=qkv.data_ptr(), **common)
            torch.cuda.synchronize()
            mb = case.geometry["mapped_bytes"]
            outs.append((_bits(qo), memcpy_dtoh(case.pool.va_k(0), mb), memcpy_dtoh(case.pool.va_v(0), mb)))
        finally:
            case.pool.destroy()
    (q0, k0, v0), (q1, k1, v1) = outs
    assert np.array_equal(q0, q1)
    skipped = [b for b, L in enumerate(lens) if b == 1 or L == 0]
    live = [b for b in range(B) if b not in skipped]
    assert np.isnan(O.decode(O.BF16, q1[skipped])).all()
    assert not np.isnan(O.decode(O.BF16, q1[live])).any()
    assert np.array_equal(k0, k1)
    assert np.array_equal(v0, v1)


@pytest.mark.parametrize("splits", ["2", "4", "8", "16"])
def test_split_k_in_kernel_reduction(gpu_lib, tunables, splits):
    """Forced split counts: every split count gives the oracle's product,
    and repeated calls give identical bits (partials are summed in split
    order)."""
    import torch
    tunables.setenv("KCMM_GEMM_SPLITS", splits)
    m, n, k = 64, 4096, 4096
    x = _randn_bf16(torch, (m, k), 1.0, 6)
    w = _randn_bf16(torch, (n, k), 0.02, 7)
    r = _randn_bf16(torch, (m, n), 1.0, 8)
    sp = torch.cuda.current_stream().cuda_stream
    ys = []
    for _ in range(3):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        gpu_lib.gemm_bf16_add(x.data_ptr(), w.data_ptr(), r.data_ptr(), y.data_ptr(), m, n, k, sp)
        ys.append(y)
    torch.cuda.synchronize()
    b0 = _bits(ys[0])
    for y in ys[1:]:
        assert np.array_equal(_bits(y), b0)
    ref = O.bf16_round(O.decode(O.BF16, _bits(r)).astype(np.float64) +
                       O.bf16_round(O.gemm_bf16_f64(_bits(x), _bits(w))))
    got = O.decode(O.BF16, b0).astype(np.float64)
    assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()


@pytest.mark.parametrize("m,n,k", [(64, 4096, 4096), (7, 512, 256), (64, 512, 14336), (200, 1024, 1024)])
def test_add_rmsnorm_matches_unfused(gpu_lib, tunables, m, n, k):
    import torch
    tunables.setenv("KCMM_GEMM_TILED", "0")   # the unfused GEMM on the same kernel
    x = _randn_bf16(torch, (m, k), 1.0, 11)
    w = _randn_bf16(torch, (n, k), 0.02, 12)
    h0 = _randn_bf16(torch, (m, n), 1.0, 13)
    nw = (1.0 + 0.1 * _randn_bf16(torch, (n,), 1.0, 14).float()).to(torch.bfloat16)
    sp = torch.cuda.current_stream().cuda_stream
    h_ref, h = h0.clone(), h0.clone()
    y_ref = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    gpu_lib.gemm_bf16_add(x.data_ptr(), w.data_ptr(), h_ref.data_ptr(), h_ref.data_ptr(), m, n, k, sp)
    gpu_lib.rmsnorm_bf16(h_ref.data_ptr(), nw.data_ptr(), y_ref.data_ptr(), m, n, 1e-5, sp)
    gpu_lib.gemm_bf16_add_rmsnorm(x.data_ptr(), w.data_ptr(), h.data_ptr(), nw.data_ptr(),
                                  y.data_ptr(), m, n, k, 1e-5, sp)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(h), _bits(h_ref))
    assert np.array_equal(_bits(y), _bits(y_ref))
