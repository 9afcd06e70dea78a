"""HIP graph capture of the decode path, through the C ABI.

The entry points launch kernels only once their per-stream workspaces exist
(no allocation, copy, memset or synchronization on a warm stream), so a
caller can capture them.  Each case runs the work eagerly twice on a side
stream (growing that stream's workspaces), captures it once on that stream
(torch.cuda.CUDAGraph), then replays the graph three times with eager work on
another stream and synchronizations between the replays.  The outputs are
filled with NaN before every replay, and every replay and every eager run
must reproduce the first eager result bit for bit.

Cases: embedding + a three-layer kcmm_decode_layers_on_stream call + logits
(bf16 and fp8-e4m3 pools; the fp8 page writer's zero-restored counters are
replayed too), standalone paged decode attention (bf16, fp8), and a
split-K projection with its reduction kernel."""
import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, KV_FP8, memcpy_dtoh
from lattice_amd.workload import build_decode_case
from tests.test_gpu_glue import _layer_weights, bf16_dev

pytestmark = pytest.mark.gpu


def _check_replays(torch, run, outputs, replays=3):
    """run(stream_ptr) launches the work; outputs() lists the result tensors."""
    gs = torch.cuda.Stream()
    torch.cuda.synchronize()
    run(gs.cuda_stream)
    run(gs.cuda_stream)
    torch.cuda.synchronize()
    ref = [t.clone() for t in outputs()]
    assert all(bool(torch.isfinite(t.float()).all()) for t in ref)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=gs):
        run(gs.cuda_stream)
    torch.cuda.synchronize()
    main = torch.cuda.current_stream().cuda_stream
    for r in range(replays):
        for t in outputs():
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (t, e) in enumerate(zip(outputs(), ref)):
            assert torch.equal(t, e), f"replay {r}: output {i} differs from the eager run"
        run(main)                       # eager work between the replays
        torch.cuda.synchronize()
        for i, (t, e) in enumerate(zip(outputs(), ref)):
            assert torch.equal(t, e), f"eager run after replay {r}: output {i} differs"
    del graph


@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_decode_step_graph_replays(gpu_lib, dtype):
    import torch
    hq, hkv, d, h, inter, vocab, nl = 32, 8, 128, 4096, 1024, 1024, 3
    lens = [1, 16, 17, 130, 700]
    case = build_decode_case(gpu_lib, batch=len(lens), num_q_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=16, ctx_lens=lens, dtype=dtype, seed=3, num_layers=nl)
    try:
        rng = np.random.default_rng(21)
        ws = [_layer_weights(torch, rng, h, inter, hq, hkv, d) for _ in range(nl)]
        embed = bf16_dev(torch, O.encode(O.BF16, rng.standard_normal((vocab, h))))
        head = bf16_dev(torch, O.encode(O.BF16, rng.standard_normal((vocab, h)) * 0.02))
        fnorm = bf16_dev(torch, O.encode(O.BF16, 1.0 + 0.1 * rng.standard_normal(h)))
        ids = torch.tensor(rng.integers(0, vocab, size=len(lens)), dtype=torch.int32, device="cuda")
        hidden = torch.empty((len(lens), h), dtype=torch.bfloat16, device="cuda")
        logits = torch.empty((len(lens), vocab), dtype=torch.bfloat16, device="cuda")
        invd = torch.from_numpy(O.default_inv_freq(500000.0, d).astype(np.float32)).cuda()
        dv = case.dev
        B = len(lens)

        def run(s):
            gpu_lib.embed_tokens_bf16(embed.data_ptr(), ids.data_ptr(), hidden.data_ptr(), B, h,
                                      vocab, s)
            case.pool.decode_layers(first_layer=0, weights=[w[2] for w in ws],
                                    hidden_ptr=hidden.data_ptr(),
                                    block_tables_ptr=dv["bt"].data_ptr(),
                                    seq_lens_ptr=dv["sl"].data_ptr(),
                                    block_offsets_f16_ptr=dv["offs"].data_ptr(),
                                    inv_freq_ptr=invd.data_ptr(), batch=B, hidden_size=h,
                                    num_q_heads=hq, intermediate_size=inter,
                                    max_blocks_per_seq=case.mbps, rms_eps=1e-5, stream_ptr=s)
            gpu_lib.decode_logits_bf16(hidden.data_ptr(), fnorm.data_ptr(), head.data_ptr(),
                                       logits.data_ptr(), B, h, vocab, 1e-5, s)

        _check_replays(torch, run, lambda: [hidden, logits])
        # the appended K/V rows are the same bytes in every run
        mb = case.geometry["mapped_bytes"]
        regions = [memcpy_dtoh(case.pool.va_k(l), mb) for l in range(nl)]
        run(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert all(np.array_equal(r, memcpy_dtoh(case.pool.va_k(l), mb))
                   for l, r in enumerate(regions))
    finally:
        case.pool.destroy()


@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_attention_graph_replays(gpu_lib, dtype):
    import torch
    hq, hkv, d = 32, 8, 128
    lens = [2500, 1, 0, 1025, 4096, 37, 300, 2049]
    case = build_decode_case(gpu_lib, batch=len(lens), num_q_heads=hq, kv_heads=hkv, head_dim=d,
                             block_size=16, ctx_lens=lens, dtype=dtype, seed=4)
    try:
        dv = case.dev
        out = torch.empty((len(lens), hq, d), dtype=torch.bfloat16, device="cuda")

        def run(s):
            case.pool.paged_attn_decode(layer_idx=0, query_ptr=dv["q"].data_ptr(),
                                        out_ptr=out.data_ptr(), block_tables_ptr=dv["bt"].data_ptr(),
                                        seq_lens_ptr=dv["sl"].data_ptr(),
                                        block_offsets_f16_ptr=dv["offs"].data_ptr(),
                                        batch=len(lens), num_q_heads=hq, kv_heads=hkv, head_dim=d,
                                        block_size=16, max_blocks_per_seq=case.mbps,
                                        scale=1.0 / np.sqrt(d), stream_ptr=s)

        _check_replays(torch, run, lambda: [out])
    finally:
        case.pool.destroy()


def test_split_gemm_graph_replays(gpu_lib):
    import torch
    m, n, k = 64, 4096, 4096
    assert gpu_lib.gemm_plan(m, n, k)["splits"] > 1     # partials + the reduction kernel
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    x = torch.randn((m, k), generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    r = torch.randn((m, n), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")

    def run(s):
        gpu_lib.gemm_bf16_add(x.data_ptr(), w.data_ptr(), r.data_ptr(), y.data_ptr(), m, n, k, s)

    _check_replays(torch, run, lambda: [y])
