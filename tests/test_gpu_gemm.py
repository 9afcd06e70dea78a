"""Projection GEMM Y = X W^T (bf16, fp32 accumulate) on the GPU vs the
oracle (fp64) on small shapes and vs a torch fp32 matmul at the Llama-3-8B
decode shapes.  Tolerance: max|Y-ref| / max|ref| <= 1e-2 (bf16)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def rel_err(got, ref):
    return float(np.abs(got - ref).max() / np.abs(ref).max())


@pytest.fixture(params=["tiled", "stream"])
def backend(request, tunables):
    """kcmm_gemm_bf16 runs products with M > 128 on the LDS-tiled MFMA
    kernel; KCMM_GEMM_TILED=0 keeps them on the weight-stream kernel.  Both
    are checked."""
    tunables.setenv("KCMM_GEMM_TILED", "1" if request.param == "tiled" else "0")
    return request.param


def run(gpu_lib, x, w):
    import torch
    m, k = x.shape
    n = w.shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    gpu_lib.gemm_bf16(x.data_ptr(), w.data_ptr(), y.data_ptr(), m, n, k,
                      torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("m,n,k", [(1, 64, 256), (17, 192, 512), (64, 256, 1024),
                                   (100, 128, 768), (256, 320, 2048), (129, 192, 512),
                                   (300, 1024, 256), (513, 640, 1024)])
def test_vs_oracle(gpu_lib, backend, m, n, k):
    import torch
    if backend == "tiled" and m <= 128:
        pytest.skip("M <= 128 always runs the weight-stream kernel")
    rng = np.random.default_rng(m + n + k)
    xb = O.encode(O.BF16, rng.standard_normal((m, k)))
    wb = O.encode(O.BF16, rng.standard_normal((n, k)) * 0.02)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    w = torch.from_numpy(wb.view(np.int16)).view(torch.bfloat16).cuda()
    y = run(gpu_lib, x, w)
    got = O.decode(O.BF16, y.cpu().view(torch.int16).numpy().view(np.uint16))
    err = rel_err(got, O.gemm_bf16_f64(xb, wb))
    print(f"gemm {backend} {m}x{n}x{k} err={err:.3e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("m", [64, 256])
@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)])
def test_llama3_8b_projections(gpu_lib, backend, m, n, k):
    import torch
    if backend == "tiled" and m <= 128:
        pytest.skip("M <= 128 always runs the weight-stream kernel")
    g = torch.Generator(device="cuda")
    g.manual_seed(m * 7 + n + k)
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    y = run(gpu_lib, x, w).float()
    ref = x.float() @ w.float().t()
    err = float((y - ref).abs().max() / ref.abs().max())
    print(f"gemm {backend} {m}x{n}x{k} err={err:.3e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("target", ["1", "64", "256", "100000"])
@pytest.mark.parametrize("m,n,k", [(1, 128, 256), (17, 384, 512), (33, 1280, 2304),
                                   (64, 256, 14336), (64, 6144, 4096), (48, 64, 1024)])
def test_split_k_choices(gpu_lib, tunables, target, m, n, k):
    """The K split chosen for a target workgroup count (1 = never split,
    100000 = as many splits as chunks allow) gives the same product: split
    partials and their reduction are exact up to fp32 rounding."""
    import torch
    tunables.setenv("KCMM_GEMM_WGS", target)
    g = torch.Generator(device="cuda")
    g.manual_seed(m * 31 + n + k + len(target))
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    y = run(gpu_lib, x, w).float()
    ref = x.float() @ w.float().t()
    err = float((y - ref).abs().max() / ref.abs().max())
    print(f"gemm target={target} {m}x{n}x{k} err={err:.3e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("m,n,k", [(64, 16384, 1024), (1, 16384, 512), (100, 16384, 768),
                                   (64, 128256, 4096)])
@pytest.mark.parametrize("residual", [False, True])
def test_eight_wave_workgroups(gpu_lib, tunables, m, n, k, residual):
    """Unsplit plain products in 8-wave workgroups (KCMM_GEMM_WAVES=8: 128
    weight rows share one staged activation chunk; the last shape is the
    Llama-3-8B lm_head at the decode batch) give the same bits as 4-wave
    workgroups, each output being summed by one wave in the same k order;
    both against a torch fp32 product."""
    import torch
    assert gpu_lib.gemm_plan(m, n, k)["splits"] == 1
    g = torch.Generator(device="cuda")
    g.manual_seed(m + n + k + residual)
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    r = torch.randn((m, n), generator=g, device="cuda").to(torch.bfloat16)
    s = torch.cuda.current_stream().cuda_stream
    outs = {}
    for waves in ("4", "8"):
        tunables.setenv("KCMM_GEMM_WAVES", waves)
        if residual:
            y = r.clone()
            gpu_lib.gemm_bf16_add(x.data_ptr(), w.data_ptr(), y.data_ptr(), y.data_ptr(), m, n, k, s)
        else:
            y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
            gpu_lib.gemm_bf16(x.data_ptr(), w.data_ptr(), y.data_ptr(), m, n, k, s)
        torch.cuda.synchronize()
        outs[waves] = y
    assert torch.equal(outs["4"], outs["8"])
    prod = x.float() @ w.float().t()
    ref = prod.to(torch.bfloat16).float() + r.float() if residual else prod
    err = float((outs["8"].float() - ref).abs().max() / ref.abs().max())
    print(f"8-wave gemm {m}x{n}x{k} residual={residual} err={err:.3e}", flush=True)
    assert err <= 1e-2


def test_eight_wave_swiglu(gpu_lib, tunables):
    """The fused gate/up + SwiGLU product at the Llama-3-8B decode shape
    (unsplit, 224 workgroups of 8 waves) gives the same bits as 4-wave
    workgroups; against silu(g)*u of a torch fp32 product.  (fp8 weights
    reach this kernel through the layer driver: tests/test_gpu_glue.py.)"""
    import torch
    m, inter, k = 64, 14336, 4096
    assert gpu_lib.gemm_plan(m, 2 * inter, k)["splits"] == 1
    g = torch.Generator(device="cuda")
    g.manual_seed(17)
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((2 * inter, k), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    s = torch.cuda.current_stream().cuda_stream
    outs = {}
    for waves in ("4", "8"):
        tunables.setenv("KCMM_GEMM_WAVES", waves)
        act = torch.full((m, inter), float("nan"), dtype=torch.bfloat16, device="cuda")
        gpu_lib.gemm_bf16_swiglu(x.data_ptr(), w.data_ptr(), act.data_ptr(), m, inter, k, s)
        torch.cuda.synchronize()
        outs[waves] = act
    assert torch.equal(outs["4"], outs["8"])
    gu = (x.float() @ w.float().t()).to(torch.bfloat16).float()
    gate, up = gu[:, :inter], gu[:, inter:]
    ref = (gate * torch.sigmoid(gate)).to(torch.bfloat16).float() * up
    err = float((outs["8"].float() - ref).abs().max() / ref.abs().max())
    print(f"8-wave swiglu err={err:.3e}", flush=True)
    assert err <= 1e-2


def test_eight_wave_workgroups_fp8_weights(gpu_lib, tunables):
    """The same for fp8-e4m3 weights (row scales applied in the store)."""
    import torch
    m, n, k = 64, 16384, 2048
    assert gpu_lib.gemm_plan(m, n, k, fp8_weights=True)["splits"] == 1
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    wf = torch.randn((n, k), generator=g, device="cuda") * 0.02
    sc = (wf.abs().amax(dim=1) / 448.0).clamp_min(1e-12)
    w8 = (wf / sc[:, None]).to(torch.float8_e4m3fn)
    s = torch.cuda.current_stream().cuda_stream
    outs = {}
    for waves in ("4", "8"):
        tunables.setenv("KCMM_GEMM_WAVES", waves)
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        gpu_lib.gemm_fp8w_bf16(x.data_ptr(), w8.view(torch.uint8).data_ptr(), sc.data_ptr(),
                               y.data_ptr(), m, n, k, s)
        torch.cuda.synchronize()
        outs[waves] = y
    assert torch.equal(outs["4"], outs["8"])
    ref = x.float() @ (w8.float() * sc[:, None]).t()
    err = float((outs["8"].float() - ref).abs().max() / ref.abs().max())
    print(f"8-wave fp8w gemm {m}x{n}x{k} err={err:.3e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("tile", [str(i) for i in range(11)])
@pytest.mark.parametrize("splits", ["1", "2", "4"])
@pytest.mark.parametrize("residual", [False, True])
def test_tiled_tiles_splits_residual(gpu_lib, tunables, tile, splits, residual):
    """Every configuration of the tiled kernel (tiles 128x256, 128x128,
    128x64, 64x128, 64x64, 128x256 on 4 waves, 256x128, 128x256 with 2
    stages) with 1, 2 or 4 K splits, M not a multiple of the tile, with and
    without a residual (in place: R == Y), against the fp64 oracle; two
    calls in a row give the same bits."""
    import torch
    tunables.setenv("KCMM_GEMM_TILE", tile)
    tunables.setenv("KCMM_GEMM_SPLITS", splits)
    m, n, k = 300, 768, 1024
    rng = np.random.default_rng(int(tile) * 10 + int(splits) + residual)
    xb = O.encode(O.BF16, rng.standard_normal((m, k)))
    wb = O.encode(O.BF16, rng.standard_normal((n, k)) * 0.02)
    rb = O.encode(O.BF16, rng.standard_normal((m, n)))
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    w = torch.from_numpy(wb.view(np.int16)).view(torch.bfloat16).cuda()
    outs = []
    for _ in range(2):
        y = torch.from_numpy(rb.view(np.int16)).view(torch.bfloat16).cuda().clone()
        if residual:
            gpu_lib.gemm_bf16_add(x.data_ptr(), w.data_ptr(), y.data_ptr(), y.data_ptr(), m, n, k,
                                  torch.cuda.current_stream().cuda_stream)
        else:
            gpu_lib.gemm_bf16(x.data_ptr(), w.data_ptr(), y.data_ptr(), m, n, k,
                              torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        outs.append(y.cpu().view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(outs[0], outs[1])
    got = O.decode(O.BF16, outs[0]).astype(np.float64)
    prod = O.gemm_bf16_f64(xb, wb)
    ref = (O.decode(O.BF16, O.encode(O.BF16, prod)).astype(np.float64) +
           O.decode(O.BF16, rb)) if residual else prod
    err = rel_err(got, ref)
    print(f"tiled tile={tile} splits={splits} residual={residual} err={err:.3e}", flush=True)
    assert err <= 1e-2


def _fp8_weights(torch, rng, n, k, std):
    w8, s = O.quantize_fp8_rows(rng.standard_normal((n, k)).astype(np.float32) * std)
    return w8, s, torch.from_numpy(w8).cuda(), torch.from_numpy(s).cuda()


@pytest.mark.parametrize("m,n,k", [(1, 64, 256), (17, 192, 512), (64, 256, 1024),
                                   (100, 128, 768), (129, 192, 512), (256, 640, 2048)])
def test_fp8_weights_vs_oracle(gpu_lib, m, n, k):
    """kcmm_gemm_fp8w_bf16: e4m3 weights with per-row scales against the fp64
    oracle (relative 1e-2, the bf16 output's tolerance); a second call gives
    the same bits."""
    import torch
    rng = np.random.default_rng(m * 3 + n + k)
    xb = O.encode(O.BF16, rng.standard_normal((m, k)))
    w8, s, w8d, sd = _fp8_weights(torch, rng, n, k, 0.02)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    outs = []
    for _ in range(2):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        gpu_lib.gemm_fp8w_bf16(x.data_ptr(), w8d.data_ptr(), sd.data_ptr(), y.data_ptr(), m, n, k,
                               torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        outs.append(y.cpu().view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(outs[0], outs[1])
    got = O.decode(O.BF16, outs[0]).astype(np.float64)
    err = rel_err(got, O.gemm_fp8w_f64(xb, w8, s))
    print(f"fp8w gemm {m}x{n}x{k} err={err:.3e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("m", [64, 128, 256])
@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)])
def test_fp8_weights_llama3_8b_projections(gpu_lib, m, n, k):
    """The four Llama-3-8B projections with fp8 weights vs a torch fp32 product
    of the dequantized weights."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(m + n + k)
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    w = torch.randn((n, k), generator=g, device="cuda") * 0.02
    s = (w.abs().amax(dim=1) / 448.0).clamp_min(1e-30)
    w8 = (w / s[:, None]).to(torch.float8_e4m3fn)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    gpu_lib.gemm_fp8w_bf16(x.data_ptr(), w8.view(torch.uint8).data_ptr(), s.data_ptr(),
                           y.data_ptr(), m, n, k, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref = x.float() @ (w8.float() * s[:, None]).t()
    err = float((y.float() - ref).abs().max() / ref.abs().max())
    print(f"fp8w gemm {m}x{n}x{k} err={err:.3e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("tile", [str(i) for i in range(11)])
@pytest.mark.parametrize("splits", ["1", "2", "4"])
def test_fp8_weights_tiled(gpu_lib, tunables, tile, splits):
    """fp8 weights with more than 128 tokens take the LDS-tiled kernel (codes
    staged in 64-byte LDS rows, converted to bf16 as they are read): every
    tiling with 1, 2 or 4 K splits, M not a multiple of the tile, against the
    fp64 oracle; two calls give the same bits; the weight-stream kernel
    (KCMM_GEMM_TILED=0) agrees within the same tolerance."""
    import torch
    tunables.setenv("KCMM_GEMM_TILE", tile)
    tunables.setenv("KCMM_GEMM_SPLITS", splits)
    m, n, k = 300, 768, 1024
    rng = np.random.default_rng(int(tile) * 10 + int(splits) + 5)
    xb = O.encode(O.BF16, rng.standard_normal((m, k)))
    w8, s, w8d, sd = _fp8_weights(torch, rng, n, k, 0.02)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    assert gpu_lib.gemm_plan(m, n, k, fp8_weights=True)["kernel"] == "tiled"
    outs = []
    for _ in range(2):
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        gpu_lib.gemm_fp8w_bf16(x.data_ptr(), w8d.data_ptr(), sd.data_ptr(), y.data_ptr(), m, n, k,
                               torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        outs.append(y.cpu().view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(outs[0], outs[1])
    got = O.decode(O.BF16, outs[0]).astype(np.float64)
    ref = O.gemm_fp8w_f64(xb, w8, s)
    err = rel_err(got, ref)
    print(f"fp8w tiled tile={tile} splits={splits} err={err:.3e}", flush=True)
    assert err <= 1e-2
    tunables.setenv("KCMM_GEMM_TILED", "0")
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    gpu_lib.gemm_fp8w_bf16(x.data_ptr(), w8d.data_ptr(), sd.data_ptr(), y.data_ptr(), m, n, k,
                           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    stream = O.decode(O.BF16, y.cpu().view(torch.int16).numpy().view(np.uint16)).astype(np.float64)
    assert rel_err(stream, ref) <= 1e-2


@pytest.mark.parametrize("splits", ["1", "2", "4", "8"])
def test_fp8_weights_split_k(gpu_lib, tunables, splits):
    import torch
    tunables.setenv("KCMM_GEMM_SPLITS", splits)
    rng = np.random.default_rng(int(splits))
    m, n, k = 64, 512, 4096
    xb = O.encode(O.BF16, rng.standard_normal((m, k)))
    w8, s, w8d, sd = _fp8_weights(torch, rng, n, k, 0.02)
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).cuda()
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    gpu_lib.gemm_fp8w_bf16(x.data_ptr(), w8d.data_ptr(), sd.data_ptr(), y.data_ptr(), m, n, k,
                           torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = O.decode(O.BF16, y.cpu().view(torch.int16).numpy().view(np.uint16)).astype(np.float64)
    assert rel_err(got, O.gemm_fp8w_f64(xb, w8, s)) <= 1e-2


def test_workspace_two_host_threads(gpu_lib):
    """Two host threads launch split-K GEMMs on the same (null) stream with
    growing shapes: each thread has its own split-partial workspace, so one
    thread growing (and freeing) its buffer never frees the buffer the other
    is about to launch with.  Every product is checked."""
    import threading
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    shapes = [(64, n, 4096) for n in (256, 512, 1024, 2048, 3072)]
    data = {}
    for m, n, k in shapes:
        x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
        w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        data[n] = (x, w, (x.float() @ w.float().t()))
    torch.cuda.synchronize()
    errors = []

    def worker(order):
        try:
            torch.cuda.set_device(0)
            for rep in range(3):
                for n in order:
                    x, w, ref = data[n]
                    y = torch.empty((64, n), dtype=torch.bfloat16, device="cuda")
                    gpu_lib.gemm_bf16(x.data_ptr(), w.data_ptr(), y.data_ptr(), 64, n, 4096, 0)
                    torch.cuda.synchronize()
                    err = float((y.float() - ref).abs().max() / ref.abs().max())
                    if not err <= 1e-2:
                        errors.append((n, rep, err))
        except Exception as e:          # reported below
            errors.append(repr(e))

    ns = [n for _, n, _ in shapes]
    threads = [threading.Thread(target=worker, args=(ns,)),
               threading.Thread(target=worker, args=(ns[::-1],))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert errors == []


def test_gemm_plan(gpu_lib, tunables):
    """kcmm_gemm_plan reports what the product entry points run."""
    p = gpu_lib.gemm_plan(64, 6144, 4096)
    assert p["kernel"] == "stream" and p["tile"] == -1
    assert p["partial_bytes"] == (p["splits"] * 64 * 6144 * 4 if p["splits"] > 1 else 0)
    assert gpu_lib.gemm_plan(256, 6144, 4096)["kernel"] == "tiled"
    assert gpu_lib.gemm_plan(256, 6144, 4096, fp8_weights=True)["kernel"] == "tiled"
    assert gpu_lib.gemm_plan(128, 6144, 4096, fp8_weights=True)["kernel"] == "stream"
    tunables.setenv("KCMM_GEMM_SPLITS", "2")
    assert gpu_lib.gemm_plan(64, 512, 4096)["splits"] == 2
    tunables.setenv("KCMM_GEMM_TILED", "0")
    assert gpu_lib.gemm_plan(256, 6144, 4096)["kernel"] == "stream"
    with pytest.raises(Exception):
        gpu_lib.gemm_plan(64, 100, 4096)          # n not a multiple of 64
