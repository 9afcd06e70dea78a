#!/usr/bin/env python3
"""Decode-step benchmark on one MI355X (Llama-3-8B shape).

Workload (synthetic, seeded): 64 sequences, 32 query / 8 KV heads, head_dim
128, block_size 16, context ~ U[512, 4096] plus one token appended per
sequence before attention, bf16 K/V scattered over a shuffled page pool.  The
pool holds several layers and consecutive steps cycle through them, so each
step reads KV that is not resident in the 256 MB Infinity Cache -- as the 32
layers of a real decode step do.

A timed step = one decoder layer of a decode step through libkcmm.so, one
C-ABI call per kernel: RMSNorm -> QKV GEMM -> RoPE + KV append into the page
row -> paged attention -> O GEMM + residual -> RMSNorm -> gate+up GEMM ->
SiLU*up -> down GEMM + residual.  HIP events on the launch stream time every
call.  After the timed steps the same layer is timed through the single
entry point kcmm_decode_layer_step_on_stream, the standalone slot append
(kcmm_append_kv_device_slots) on its own, and a whole decode step -- all 32
layers, each over its own KV -- through the token embedding
(kcmm_embed_tokens_bf16), one kcmm_decode_layers_on_stream call, the final
RMSNorm and the lm_head GEMM (vocab 128256) to bf16 logits.

Printed JSON: `value` is decode-attention KV GB/s (algorithmic K+V bytes of
one layer-step / attention call time, the call's average launch duration over
consecutive calls on the cycled KV sets); decode tokens/s = 64 / t_step with
t_step the embedding, the 32-layer call, the final norm and lm_head (sampling
is outside this path and excluded).

`roofline` prices the dominant kernel, the attention's streaming kernel
(attn_decode_stream), against MI355X's 8 TB/s: algorithmic K+V bytes / its
average launch duration, from HIP events that the library records around
each launch on the launch stream (kcmm_attn_stream_timing_*) over the same
back-to-back calls; `roofline.call` repeats the figures for the whole call
(the kernel, the log-sum-exp merge and the gap between them).  `traffic`
(HBM bytes per launch) is read from the rocprofv3 FETCH_SIZE / WRITE_SIZE
summary committed in profiles/, which records the commands and the
copy-kernel calibration it was scaled with.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, vendor figure

B, HQ, HKV, D, BS = 64, 32, 8, 128, 16
CTX_LO, CTX_HI = 512, 4096
MODEL_LAYERS = 32
HIDDEN, INTER, VOCAB = 4096, 14336, 128256
KV_BF16_CODE = 1
KV_FP8_CODE = 2
ROPE_THETA, RMS_EPS = 500000.0, 1e-5      # Llama-3-8B config.json
BEAM_WIDTH = 4                             # configs[4]
GEMMS = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)]


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--layers", type=int, default=4, help="KV/weight sets cycled through")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--attn-only", action="store_true", help="time attention (+append) only")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-shuffle", action="store_true",
                    help="give each sequence contiguous pages (locality experiment)")
    ap.add_argument("--config", choices=["cfg2", "cfg3", "cfg5"], default="cfg2",
                    help="cfg2: the headline bf16 decode layer-step; cfg3: chunked prefill, "
                         "16 seqs x 256-token chunk over a shared 1024-token prefix; cfg5: "
                         "fp8-e4m3 pages, B=128, ctx 80%% U[1024,8192] + 20%% U[16384,32768] "
                         "(attention only)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="time the four M=64 projection GEMMs alone, as the layer's component "
                         "pass calls them (for HBM counter runs under rocprofv3)")
    ap.add_argument("--m", type=int, default=64,
                    help="--gemm-only: tokens per product (64: the decode batch, O and down add "
                         "their residual; other values: plain products, e.g. 256 for the "
                         "LDS-tiled kernel)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="also run one 256 MiB device copy (HBM counter calibration under rocprofv3)")
    ap.add_argument("--decode-graph", action="store_true",
                    help="also time the decode step replayed from a HIP graph")
    ap.add_argument("--no-sub-configs", action="store_true",
                    help="cfg2: skip the cfg3 prefill and cfg5 fp8 runs that the default run "
                         "adds as sub-objects of its JSON line")
    return ap.parse_args()


def sub_config(cfg, args) -> dict | None:
    """Runs `bench.py --config cfg` in a child process (its own pool and
    workload) and returns its JSON line, or an error record."""
    import subprocess
    cmd = [sys.executable, str(Path(__file__).resolve()), "--config", cfg,
           "--steps", str(max(4, min(args.steps, 20))), "--warmup", str(max(2, min(args.warmup, 5))),
           "--no-cpu-baseline", "--seed", str(args.seed)]
    log(f"sub-config {cfg}: {' '.join(cmd[1:])}")
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, text=True)
    lines = [l for l in proc.stdout.splitlines() if l.startswith("{")]
    if proc.returncode != 0 or not lines:
        return {"error": f"bench.py --config {cfg} exited {proc.returncode}"}
    out = json.loads(lines[-1])
    out["cmd"] = "python3 bench.py " + " ".join(cmd[2:])
    return out


TRAFFIC_FILES = {"cfg2": ROOT / "profiles" / "attn_decode_cfg2_hbm_traffic.txt",
                 "cfg3": ROOT / "profiles" / "attn_prefill_cfg3_hbm_traffic.txt",
                 "cfg5": ROOT / "profiles" / "attn_decode_fp8_cfg5_hbm_traffic.txt"}


def measured_traffic(config="cfg2", key="traffic_bytes_per_call"):
    """HBM bytes per attention call (or, with key="traffic_bytes_stream_kernel",
    per launch of the streaming kernel alone) from the committed rocprofv3
    counter summary of that config (None if the file or the line is absent)."""
    try:
        for line in TRAFFIC_FILES[config].read_text().splitlines():
            if line.startswith(key + ":"):
                return int(line.split(":")[1].split()[0])
    except OSError:
        pass
    return None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def quantize_layer_fp8(w):
    """fp8-e4m3 copies of a layer's four projections (per-row amax/448 scales,
    quantized on the device) and the ABI struct of the fp8-weight layer."""
    import torch
    from lattice_amd.bindings import KcmmLayerWeightsFp8
    w8 = {"attn_norm": w["attn_norm"], "mlp_norm": w["mlp_norm"]}
    for name, _, _ in GEMMS:
        wf = w[name].float()
        sc = (wf.abs().amax(dim=1) / 448.0).clamp_min(1e-30)
        w8[name] = (wf / sc[:, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
        w8[name + "_scale"] = sc.contiguous()
        del wf
    return w8, KcmmLayerWeightsFp8(**{k: t.data_ptr() for k, t in w8.items()})


def cpu_baseline(case, seconds, threads):
    """The reference kernel's loop (oracle restatement) on host cores, on a
    bounded sample: layer 0 of the same workload, the first sequences that
    fit the time budget."""
    import oracle as O
    from lattice_amd.bindings import memcpy_dtoh
    g = case.geometry
    kreg = memcpy_dtoh(case.pool.va_k(0), g["mapped_bytes"])
    vreg = memcpy_dtoh(case.pool.va_v(0), g["mapped_bytes"])
    scale = 1 / math.sqrt(D)
    # estimate with 4 sequences, then size the sample to ~`seconds`
    def run(nseq, reps=1):
        bt = case.block_tables[:nseq]
        sl = case.seq_lens[:nseq]
        q = case.q_bits[:nseq]
        out = np.zeros((nseq, HQ, D), np.float32)
        t0 = time.perf_counter()
        for _ in range(reps):
            O.attn_decode_ref_f32(1, q, kreg, vreg, bt, sl, case.offsets_f16, HQ, HKV, D, BS,
                                  g["row_bytes"], scale, threads=threads, out=out)
        return (time.perf_counter() - t0) / reps
    t4 = run(4)
    per_seq = t4 / 4
    nseq = B
    reps = max(1, int(seconds / max(per_seq * B, 1e-6)))
    if per_seq * B > seconds:
        nseq = max(4, int(seconds / per_seq))
        reps = 1
    t = run(nseq, reps)
    kv = int(case.seq_lens[:nseq].astype(np.int64).sum()) * 2 * HKV * D * 2
    return dict(value=round(kv / t / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                sample=(f"oracle restatement of ref kcmm_vllm_paged_attn.cu loop (fp32, bf16 KV), "
                        f"layer 0, {nseq} of {B} seqs ({kv / 1e6:.1f} MB KV) x {reps} reps, "
                        f"{t * 1e3:.1f} ms per pass"))


def cpu_baseline_detail(lib, case, args, threads) -> dict:
    """BASELINE's CPU plan beside the headline baseline: the Cfg2 sample on one
    thread, and configs[0] (fp32 pages, B=4, 8/8 heads, head_dim 64, ctx
    U[1,512] + 1, pages shuffled over the pool) on one thread and on all
    threads, with the GPU's time for the same configs[0] call beside it."""
    import torch
    import oracle as O
    from lattice_amd.bindings import KV_F32, memcpy_dtoh
    from lattice_amd.workload import build_decode_case
    out = {"cfg2_1_thread": cpu_baseline(case, max(2.0, args.cpu_seconds / 3), 1)}
    rng = np.random.default_rng(args.seed + 7)
    ctx = rng.integers(1, 513, size=4) + 1
    c1 = build_decode_case(lib, batch=4, num_q_heads=8, kv_heads=8, head_dim=64, block_size=16,
                           ctx_lens=ctx, dtype=KV_F32, seed=args.seed + 8)
    try:
        g = c1.geometry
        kreg = memcpy_dtoh(c1.pool.va_k(0), g["mapped_bytes"])
        vreg = memcpy_dtoh(c1.pool.va_v(0), g["mapped_bytes"])
        kv = int(c1.seq_lens.astype(np.int64).sum()) * 2 * 8 * 64 * 4
        stream = torch.cuda.current_stream()
        for _ in range(5):
            c1.run_attention(stream_ptr=stream.cuda_stream)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record(stream)
        for _ in range(50):
            c1.run_attention(stream_ptr=stream.cuda_stream)
        ev[1].record(stream)
        torch.cuda.synchronize()
        gpu_s = ev[0].elapsed_time(ev[1]) / 50 / 1e3
        res = O.attn_decode_ref_f32(O.F32, c1.q_bits, kreg, vreg, c1.block_tables, c1.seq_lens,
                                    c1.offsets_f16, 8, 8, 64, 16, g["row_bytes"], 1 / math.sqrt(64),
                                    threads=1)
        for label, th in (("cfg1_fp32_1_thread", 1), ("cfg1_fp32_all_threads", threads)):
            reps, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < 2.0:
                O.attn_decode_ref_f32(O.F32, c1.q_bits, kreg, vreg, c1.block_tables, c1.seq_lens,
                                      c1.offsets_f16, 8, 8, 64, 16, g["row_bytes"],
                                      1 / math.sqrt(64), threads=th, out=res)
                reps += 1
            t = (time.perf_counter() - t0) / reps
            out[label] = dict(value=round(kv / t / 1e9, 3), unit="GB/s", cores=th, kind="port",
                              us_per_call=round(t * 1e6, 2),
                              sample=f"configs[0], {kv / 1e6:.2f} MB KV, {reps} reps")
        out["cfg1_fp32_gpu"] = dict(value=round(kv / gpu_s / 1e9, 3), unit="GB/s",
                                    us_per_call=round(gpu_s * 1e6, 2),
                                    note="kcmm_paged_attn_decode_f32_on_stream, any-shape kernel")
    finally:
        c1.pool.destroy()
    return out


def gemm_bytes(lib, name, n, k, m):
    """Algorithmic HBM bytes of one projection call (W, X, Y; O and down also
    read their residual) and the fp32 split-K partials its plan writes and
    the reduction reads back (not algorithmic: the cost of the split)."""
    res = 2 if name in ("o", "down") else 1
    plan = lib.gemm_plan(m, n, k)
    return 2.0 * (n * k + m * k + m * n * res), plan


def time_decode_graph(decode_step, logits, sp, steps, warmup):
    """The decode step captured once in a HIP graph (torch.cuda.CUDAGraph) on a
    stream of its own and replayed: ms per replay.  The stream's workspaces
    grow in two eager steps before the capture; the eager step's logits are
    the reference, and three replays -- each followed by an eager step on the
    bench's stream -- must reproduce them bit for bit before any timing."""
    import torch
    gs = torch.cuda.Stream()
    gsp = gs.cuda_stream
    torch.cuda.synchronize()
    decode_step(0, gsp)
    decode_step(0, gsp)
    torch.cuda.synchronize()
    ref = logits.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=gs):
        decode_step(0, gsp)
    torch.cuda.synchronize()
    for r in range(3):
        logits.fill_(0)
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(logits, ref):
            raise RuntimeError(f"decode-step graph replay {r} differs from the eager step")
        decode_step(0)
        torch.cuda.synchronize()
        if not torch.equal(logits, ref):
            raise RuntimeError(f"eager step after graph replay {r} differs")
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        graph.replay()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    for i in range(steps):
        evs[i].record(stream)
        graph.replay()
    evs[-1].record(stream)
    torch.cuda.synchronize()
    ms = float(np.mean([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]))
    del graph
    return ms


def bench_gemm(args):
    """--gemm-only: the four Llama-3-8B projections at M = --m tokens (64 by
    default: each called as in the layer's component pass, QKV and gate/up
    plain, O and down with the residual added in place; other M: plain
    products), two weight sets alternating so that the weights come from
    HBM; HIP events per call."""
    import torch
    from lattice_amd.bindings import KcmmLibrary
    lib = KcmmLibrary()
    dev = "cuda"
    M = args.m
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed + 2)
    sets = [{name: (torch.randn((n, k), generator=g, device=dev) * 0.02).to(torch.bfloat16)
             for name, n, k in GEMMS} for _ in range(2)]
    x = {k: torch.randn((M, k), generator=g, device=dev).to(torch.bfloat16) for k in (HIDDEN, INTER)}
    y = torch.empty((M, 2 * INTER), dtype=torch.bfloat16, device=dev)
    hidden = torch.randn((M, HIDDEN), generator=g, device=dev).to(torch.bfloat16)
    sp = torch.cuda.current_stream().cuda_stream
    if args.calib_copy:
        src = torch.empty(128 << 20, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        dst.copy_(src)                               # 256 MiB read + 256 MiB written
        torch.cuda.synchronize()
        del src, dst

    def call(name, n, k, i):
        w = sets[i % 2][name].data_ptr()
        if name in ("o", "down") and M == B:
            lib.gemm_bf16_add(x[k].data_ptr(), w, hidden.data_ptr(), hidden.data_ptr(), M, n, k, sp)
        else:
            lib.gemm_bf16(x[k].data_ptr(), w, y.data_ptr(), M, n, k, sp)

    out = {}
    for name, n, k in GEMMS:
        for i in range(args.warmup):
            call(name, n, k, i)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        torch.cuda.synchronize()
        for i in range(args.steps):
            ev[i].record()
            call(name, n, k, i)
        ev[-1].record()
        torch.cuda.synchronize()
        us = float(np.mean([ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps)])) * 1e3
        alg, plan = gemm_bytes(lib, name, n, k, M)
        if M != B and name in ("o", "down"):
            alg -= 2.0 * M * n          # plain product: no residual read
        out[name] = {"us": round(us, 2), "algorithmic_bytes": int(alg), "plan": plan,
                     "gbs": round(alg / us / 1e3, 1),
                     "frac_of_hbm_peak": round(alg / us / 1e3 / HBM_PEAK_GBS, 4),
                     "tflops": round(2.0 * M * n * k / us / 1e6, 1)}
        log(f"{name}: {us:.2f} us, plan {plan}")
    print(json.dumps({"metric": f"M={M} projection GEMM time", "unit": "us", "steps": args.steps,
                      "warmup": args.warmup, "m": M, "gemms": out}), flush=True)


def bench_prefill(args):
    """Cfg3: causal chunked prefill over shared-prefix pages; MFMA-bound."""
    import torch
    from lattice_amd.bindings import KcmmLibrary
    from lattice_amd.workload import build_prefix_shared_case
    lib = KcmmLibrary()
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    if args.calib_copy:
        # a 256 MiB device copy (256 MiB read + 256 MiB written) that the
        # counter runs scale their FETCH_SIZE / WRITE_SIZE readings by
        src = torch.empty(128 << 20, dtype=torch.int16, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def timed(dtype):
        case = build_prefix_shared_case(lib, batch=16, prefix_tokens=1024, suffix_tokens=256,
                                        chunk=256, num_q_heads=HQ, kv_heads=HKV, head_dim=D,
                                        block_size=BS, dtype=dtype, num_layers=args.layers,
                                        seed=args.seed)
        for i in range(args.warmup):
            case.run(layer=i % args.layers, stream_ptr=sp)
        torch.cuda.synchronize()
        # back-to-back calls between two events (as the decode attention's
        # value), then the same calls with an event after each one
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record(stream)
        for i in range(args.steps):
            case.run(layer=i % args.layers, stream_ptr=sp)
        eb.record(stream)
        torch.cuda.synchronize()
        ms = ea.elapsed_time(eb) / args.steps
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        ev[0].record(stream)
        for i in range(args.steps):
            case.run(layer=i % args.layers, stream_ptr=sp)
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
        ms_evented = float(np.mean([ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps)]))
        flops = case.flops()
        case.pool.destroy()
        return ms, flops, ms_evented

    ms, flops, ms_ev = timed(KV_BF16_CODE)
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"prefill per-call ms: {ms:.4f} back to back ({ms_ev:.4f} with an event after each "
        f"call), {flops / 1e9:.1f} GFLOP")
    ms8, _, _ = timed(KV_FP8_CODE)
    log(f"prefill per-call ms with fp8-e4m3 pages: {ms8:.4f}")
    result = {
        "metric": "chunked prefill attention TFLOP/s (% bf16 MFMA peak), 1 GPU",
        "value": round(tflops, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "cfg3: 16 seqs share a refcounted 1024-token prefix + own 256 "
                               "tokens; causal 256-token chunk each",
                   "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "block_size": BS},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": measured_traffic("cfg3"),
                     "kernel": "attn_prefill_mfma (bf16 pages)"},
        "gflop_per_call": round(flops / 1e9, 2),
        "ms_per_call_evented": round(ms_ev, 4),
        # the same chunk over fp8-e4m3 pages (dequantized to bf16 in LDS by
        # the same MFMA kernel): half the K/V bytes, the same flops
        "fp8_pages": {"ms": round(ms8, 4), "tflops": round(flops / (ms8 * 1e-3) / 1e12, 1)},
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                          "(the path would shard by sequence or kv head; no multi-GPU run is made)"}))
        sys.exit(2)
    if args.config == "cfg3":
        return bench_prefill(args)
    if args.gemm_only:
        return bench_gemm(args)
    import torch
    from lattice_amd.bindings import KV_BF16, KcmmLayerWeights, KcmmLibrary
    from lattice_amd.workload import build_decode_case, rope_inv_freq

    assert torch.cuda.is_available(), "bench needs a GPU"
    lib = KcmmLibrary()
    rng = np.random.default_rng(args.seed)
    global B
    kv_dtype = KV_BF16
    if args.config == "cfg5":
        from lattice_amd.bindings import KV_FP8
        B, kv_dtype, args.attn_only = 128, KV_FP8, True
        args.layers = min(args.layers, 2)
        long = rng.random(B) < 0.2
        ctx = np.where(long, rng.integers(16384, 32769, size=B), rng.integers(1024, 8193, size=B))
    else:
        ctx = rng.integers(CTX_LO, CTX_HI + 1, size=B)      # context before the appended token
    L = ctx + 1
    t0 = time.perf_counter()
    # the headline config holds all 32 layers' KV (19.6 GB) for the full-step timing
    pool_layers = args.layers if args.attn_only else max(args.layers, MODEL_LAYERS)
    case = build_decode_case(lib, batch=B, num_q_heads=HQ, kv_heads=HKV, head_dim=D,
                             block_size=BS, ctx_lens=L, dtype=kv_dtype, num_layers=pool_layers,
                             seed=args.seed + 1, host_mirror=False,
                             shuffle=not args.no_shuffle)
    log(f"workload built in {time.perf_counter() - t0:.1f}s: {case.pool.stats()['superblock_count']} "
        f"superblocks/region, backing={'vmm' if case.pool.backing_kind() == 0 else 'flat'}")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed + 2)

    # appended token: device slot ids of position ctx_b in each sequence
    slots = np.array([case.block_tables[b, int(ctx[b]) // BS] * BS + int(ctx[b]) % BS
                      for b in range(B)], dtype=np.int64)
    slots_t = torch.from_numpy(slots).to(dev)
    offs_t = case.dev["offs"]
    k_new = torch.randn((B, HKV * D), generator=g, device=dev).to(torch.bfloat16)
    v_new = torch.randn((B, HKV * D), generator=g, device=dev).to(torch.bfloat16)

    # layer weights (two sets, alternating by layer; one set is 436 MB, above
    # the 256 MB Infinity Cache) and activations
    nw = 0 if args.attn_only else 2
    weights = []
    for _ in range(nw):
        w = {name: (torch.randn((n, k), generator=g, device=dev) * 0.02).to(torch.bfloat16)
             for name, n, k in GEMMS}
        for name in ("attn_norm", "mlp_norm"):
            w[name] = (1.0 + 0.1 * torch.randn(HIDDEN, generator=g, device=dev)).to(torch.bfloat16)
        weights.append(w)
    layer_w = [KcmmLayerWeights(**{k: w[k].data_ptr() for k in
                                   ("attn_norm", "qkv", "o", "mlp_norm", "gate_up", "down")})
               for w in weights]
    inv_freq = torch.from_numpy(rope_inv_freq(ROPE_THETA, D)).to(dev)
    # embedding table, final norm and lm_head (1.05 GB each) for the whole-step timing
    if not args.attn_only:
        final_norm = (1.0 + 0.1 * torch.randn(HIDDEN, generator=g, device=dev)).to(torch.bfloat16)
        lm_head = (torch.randn((VOCAB, HIDDEN), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        logits = torch.empty((B, VOCAB), dtype=torch.bfloat16, device=dev)
        embed = torch.randn((VOCAB, HIDDEN), generator=g, device=dev).to(torch.bfloat16)
        token_ids = torch.randint(0, VOCAB, (B,), generator=g, device=dev, dtype=torch.int32)
    hidden = torch.randn((B, HIDDEN), generator=g, device=dev).to(torch.bfloat16)
    normed = torch.empty((B, HIDDEN), dtype=torch.bfloat16, device=dev)
    qkv_out = torch.empty((B, (HQ + 2 * HKV) * D), dtype=torch.bfloat16, device=dev)
    gate_up = torch.empty((B, 2 * INTER), dtype=torch.bfloat16, device=dev)
    act = torch.empty((B, INTER), dtype=torch.bfloat16, device=dev)
    kv_bytes = case.kv_bytes()                     # identical for every layer
    scale = 1 / math.sqrt(D)
    dv = case.dev

    def append(layer):
        case.pool.append_kv_device_slots_on_stream(
            layer_idx=layer, slot_mapping_ptr=slots_t.data_ptr(),
            block_offsets_f16_ptr=offs_t.data_ptr(), valid_blocks_ptr=0,
            block_offsets_f16_len=offs_t.numel(), batch=B, k_src_ptr=k_new.data_ptr(),
            v_src_ptr=v_new.data_ptr(), status_ptr=0, stream_ptr=sp)

    def norm(name, layer):
        lib.rmsnorm_bf16(hidden.data_ptr(), weights[layer % nw][name].data_ptr(),
                         normed.data_ptr(), B, HIDDEN, RMS_EPS, sp)

    def rope_append(layer):
        case.pool.rope_append(layer_idx=layer, qkv_ptr=qkv_out.data_ptr(),
                              q_out_ptr=dv["q"].data_ptr(), block_tables_ptr=dv["bt"].data_ptr(),
                              seq_lens_ptr=dv["sl"].data_ptr(),
                              block_offsets_f16_ptr=dv["offs"].data_ptr(),
                              inv_freq_ptr=inv_freq.data_ptr(), batch=B, num_q_heads=HQ,
                              max_blocks_per_seq=case.mbps, stream_ptr=sp)

    def layer_step(layer):
        case.pool.decode_layer_step(layer_idx=layer, weights=layer_w[layer % nw],
                                    hidden_ptr=hidden.data_ptr(),
                                    block_tables_ptr=dv["bt"].data_ptr(),
                                    seq_lens_ptr=dv["sl"].data_ptr(),
                                    block_offsets_f16_ptr=dv["offs"].data_ptr(),
                                    inv_freq_ptr=inv_freq.data_ptr(), batch=B,
                                    hidden_size=HIDDEN, num_q_heads=HQ, intermediate_size=INTER,
                                    max_blocks_per_seq=case.mbps, rms_eps=RMS_EPS, stream_ptr=sp)

    def decode_step(_, s=None):
        """One decode step: token embedding, all 32 layers in one call (weight
        sets alternate), then the final norm and lm_head to bf16 logits (on
        stream s, default the bench's stream)."""
        s = sp if s is None else s
        lib.embed_tokens_bf16(embed.data_ptr(), token_ids.data_ptr(), hidden.data_ptr(), B, HIDDEN,
                              VOCAB, s)
        case.pool.decode_layers(first_layer=0, weights=[layer_w[i % nw] for i in range(MODEL_LAYERS)],
                                hidden_ptr=hidden.data_ptr(), block_tables_ptr=dv["bt"].data_ptr(),
                                seq_lens_ptr=dv["sl"].data_ptr(),
                                block_offsets_f16_ptr=dv["offs"].data_ptr(),
                                inv_freq_ptr=inv_freq.data_ptr(), batch=B, hidden_size=HIDDEN,
                                num_q_heads=HQ, intermediate_size=INTER,
                                max_blocks_per_seq=case.mbps, rms_eps=RMS_EPS, stream_ptr=s)
        lib.decode_logits_bf16(hidden.data_ptr(), final_norm.data_ptr(), lm_head.data_ptr(),
                               logits.data_ptr(), B, HIDDEN, VOCAB, RMS_EPS, s)

    # the same two weight sets with fp8-e4m3 projections (per-row amax/448
    # scales, quantized on the device), for the fp8-weight decode step
    weights8, layer_w8 = [], []
    if args.config == "cfg2" and not args.attn_only:
        for w in weights:
            w8, lw8 = quantize_layer_fp8(w)
            weights8.append(w8)
            layer_w8.append(lw8)

    def decode_step_fp8w(_):
        """decode_step with the fp8-weight layers (kcmm_decode_layers_fp8w_on_stream)."""
        lib.embed_tokens_bf16(embed.data_ptr(), token_ids.data_ptr(), hidden.data_ptr(), B, HIDDEN,
                              VOCAB, sp)
        case.pool.decode_layers_fp8w(first_layer=0,
                                     weights=[layer_w8[i % nw] for i in range(MODEL_LAYERS)],
                                     hidden_ptr=hidden.data_ptr(),
                                     block_tables_ptr=dv["bt"].data_ptr(),
                                     seq_lens_ptr=dv["sl"].data_ptr(),
                                     block_offsets_f16_ptr=dv["offs"].data_ptr(),
                                     inv_freq_ptr=inv_freq.data_ptr(), batch=B,
                                     hidden_size=HIDDEN, num_q_heads=HQ, intermediate_size=INTER,
                                     max_blocks_per_seq=case.mbps, rms_eps=RMS_EPS, stream_ptr=sp)
        lib.decode_logits_bf16(hidden.data_ptr(), final_norm.data_ptr(), lm_head.data_ptr(),
                               logits.data_ptr(), B, HIDDEN, VOCAB, RMS_EPS, sp)

    W = lambda layer, name: weights[layer % nw][name].data_ptr()
    calls = {
        "norm1": lambda l: norm("attn_norm", l),
        "qkv": lambda l: lib.gemm_bf16(normed.data_ptr(), W(l, "qkv"), qkv_out.data_ptr(),
                                       B, (HQ + 2 * HKV) * D, HIDDEN, sp),
        "rope_append": rope_append,
        "append": append,
        "attn": lambda l: case.run_attention(layer=l, stream_ptr=sp, scale=scale),
        "o": lambda l: lib.gemm_bf16_add(dv["out"].data_ptr(), W(l, "o"), hidden.data_ptr(),
                                         hidden.data_ptr(), B, HIDDEN, HQ * D, sp),
        "norm2": lambda l: norm("mlp_norm", l),
        "gate_up": lambda l: lib.gemm_bf16(normed.data_ptr(), W(l, "gate_up"),
                                           gate_up.data_ptr(), B, 2 * INTER, HIDDEN, sp),
        "silu": lambda l: lib.silu_mul_bf16(gate_up.data_ptr(), act.data_ptr(), B, INTER, sp),
        "down": lambda l: lib.gemm_bf16_add(act.data_ptr(), W(l, "down"), hidden.data_ptr(),
                                            hidden.data_ptr(), B, HIDDEN, INTER, sp),
    }
    names = ["norm1", "qkv", "rope_append", "attn", "o", "norm2", "gate_up", "silu", "down"]
    if args.attn_only:
        names = ["append", "attn"]
    beam = {"children": [], "copies": 0, "host_us": []}
    if args.config == "cfg5":
        # beam search, width 4: every step each of the B sequences is forked
        # into 3 more beams whose last partial page is made private (one
        # host call, one page-copy kernel) before the step's append/attention
        parents = list(range(B))

        def beam_fork(_):
            t0 = time.perf_counter()
            children, ncopy = case.pool.fork_beams(parents, BEAM_WIDTH, stream_ptr=sp)
            beam["host_us"].append((time.perf_counter() - t0) * 1e6)
            beam["children"].extend(children)
            beam["copies"] = ncopy

        calls["beam_fork"] = beam_fork
        names = ["beam_fork", "append", "attn"]

    def release_beams():
        for c in beam["children"]:
            case.pool.unregister_sequence(c)
        beam["children"] = []

    if args.calib_copy:
        src = torch.empty(128 << 20, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        dst.copy_(src)                               # 256 MiB read + 256 MiB written
        torch.cuda.synchronize()
        del src, dst
    for i in range(args.warmup):
        for n in names:
            calls[n](i % args.layers)
        release_beams()
    torch.cuda.synchronize()
    log(f"warmup done ({args.warmup} steps)")

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for i in range(args.steps):
        layer = i % args.layers
        ev[i][0].record(stream)
        for j, n in enumerate(names):
            calls[n](layer)
            ev[i][j + 1].record(stream)
        release_beams()                              # pruned beams (between steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    per = {n: np.mean([ev[i][j].elapsed_time(ev[i][j + 1]) for i in range(args.steps)])
           for j, n in enumerate(names)}
    step_ms = float(np.mean([ev[i][0].elapsed_time(ev[i][-1]) for i in range(args.steps)]))
    log("per-call ms: " + ", ".join(f"{k}={v:.4f}" for k, v in per.items()))

    extra = {}
    if not args.attn_only:
        # the same layer through the single entry point (what a serving loop
        # calls 32 times per decode step), then the standalone slot append
        full_steps = max(4, args.steps // 8)
        def logits_step(_):
            lib.decode_logits_bf16(hidden.data_ptr(), final_norm.data_ptr(), lm_head.data_ptr(),
                                   logits.data_ptr(), B, HIDDEN, VOCAB, RMS_EPS, sp)

        timings = [("layer_step", layer_step, args.steps), ("append", append, args.steps),
                   ("logits", logits_step, args.steps), ("decode_step", decode_step, full_steps)]
        if layer_w8:
            timings.append(("decode_step_fp8w", decode_step_fp8w, full_steps))
        for label, fn, steps in timings:
            evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
            for i in range(min(args.warmup, steps)):
                fn(i % args.layers)
            torch.cuda.synchronize()
            for i in range(steps):
                evs[i].record(stream)
                fn(i % args.layers)
            evs[-1].record(stream)
            torch.cuda.synchronize()
            extra[label] = float(np.mean([evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]))
        if args.decode_graph:
            extra["decode_step_graph"] = time_decode_graph(decode_step, logits, sp, full_steps,
                                                           args.warmup)
        log(f"layer step (one call) ms={extra['layer_step']:.4f}, append ms={extra['append']:.4f}, "
            f"32-layer decode step ms={extra['decode_step']:.4f}")
        # the projections at M = 256 tokens (configs[3]'s second size), same weights:
        # kcmm_gemm_bf16 runs M > 128 on the LDS-tiled MFMA kernel; the
        # weight-stream kernel (KCMM_GEMM_TILED=0) and torch.matmul (ROCm's
        # GEMM libraries, not part of the library) are timed beside it
        m256, m256_stream, m256_torch = {}, {}, {}
        m64_cold, m64_torch = {}, {}      # M = 64 under the same protocol
        x256 = {k: torch.randn((256, k), generator=g, device=dev).to(torch.bfloat16)
                for k in (HIDDEN, INTER)}
        y256 = torch.empty((256, 2 * INTER), dtype=torch.bfloat16, device=dev)
        # each timed call starts with the weights out of the 256 MB Infinity
        # Cache, as in a model's layer loop: a 512 MiB write between calls,
        # outside the events
        flush = torch.zeros(1 << 29, dtype=torch.uint8, device=dev)
        tiled_env = os.environ.get("KCMM_GEMM_TILED")
        for mm, backend, out in ((256, "1", m256), (256, "0", m256_stream), (256, "torch", m256_torch),
                                 (B, "1", m64_cold), (B, "torch", m64_torch)):
            os.environ["KCMM_GEMM_TILED"] = "0" if backend == "0" else "1"
            lib.reload_tunables()       # the library reads KCMM_* once
            for name, n, k in GEMMS:
                xm = x256[k][:mm]      # the first mm rows (contiguous)
                if backend == "torch":
                    fn = lambda l, n=n, k=k, name=name, xm=xm: torch.matmul(
                        xm, weights[l % len(weights)][name].t())
                else:
                    fn = lambda l, n=n, k=k, name=name, xm=xm, mm=mm: lib.gemm_bf16(
                        xm.data_ptr(), W(l, name), y256.data_ptr(), mm, n, k, sp)
                evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                       for _ in range(args.steps)]
                for i in range(min(args.warmup, args.steps)):
                    fn(i)
                torch.cuda.synchronize()
                for i in range(args.steps):
                    flush.add_(1)
                    evs[i][0].record(stream)
                    fn(i)
                    evs[i][1].record(stream)
                torch.cuda.synchronize()
                out[name] = float(np.mean([a.elapsed_time(b) for a, b in evs]))
        del flush
        if tiled_env is None:
            os.environ.pop("KCMM_GEMM_TILED", None)
        else:
            os.environ["KCMM_GEMM_TILED"] = tiled_env
        lib.reload_tunables()
        del x256, y256
        log("M=256 GEMM ms (tiled MFMA kernel): " + ", ".join(f"{k}={v:.4f}" for k, v in m256.items()))
        log("M=256 GEMM ms (weight-stream kernel): " +
            ", ".join(f"{k}={v:.4f}" for k, v in m256_stream.items()))
        log("M=256 GEMM ms (torch.matmul, reference only): " +
            ", ".join(f"{k}={v:.4f}" for k, v in m256_torch.items()))
        assert torch.isfinite(hidden.float()).all(), "layer step produced non-finite hidden state"

    # attention calls back to back over the cycled KV sets (the order a decode
    # step issues them is one per layer, with the other kernels in between;
    # events between every pair of kernels, as in the component pass above,
    # add their own gaps): average launch duration of the call
    ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for i in range(args.layers):
        calls["attn"](i)
    torch.cuda.synchronize()
    ea.record(stream)
    for i in range(args.steps):
        calls["attn"](i % args.layers)
    eb.record(stream)
    torch.cuda.synchronize()
    attn_b2b_ms = ea.elapsed_time(eb) / args.steps
    log(f"attention back to back: {attn_b2b_ms:.4f} ms per call (in the component pass "
        f"{per['attn']:.4f})")
    # the dominant kernel alone: the same back-to-back calls again, with HIP
    # events recorded by the library around each streaming-kernel launch (on
    # the stream it is launched on); the merge after it is outside the pair
    lib.attn_stream_timing_start(max(1, args.steps))
    try:
        for i in range(args.steps):
            calls["attn"](i % args.layers)
        torch.cuda.synchronize()
    finally:
        stream_us, n_timed = lib.attn_stream_timing_stop()
    assert n_timed == args.steps, (n_timed, args.steps)
    log(f"attention streaming kernel: {stream_us:.2f} us per launch (HIP events, {n_timed} launches)")
    stream_gbs = kv_bytes / (stream_us * 1e-6) / 1e9
    attn_s = attn_b2b_ms / 1e3
    kv_gbs = kv_bytes / attn_s / 1e9
    result = {
        "metric": "decode attn KV GB/s (% HBM peak) + decode tokens/s, 8B-shape bs=64, 1 GPU",
        "value": round(kv_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if args.config == "cfg2" else "fp8-e4m3 KV, bf16 MFMA",
        "data": "synthetic (seeded N(0,1) K/V, N(0,0.02) weights; no checkpoint)",
        "config": {"workload": ("llama3-8b-shape decode layer-step: RMSNorm, QKV GEMM, RoPE + KV "
                                "append, paged attention, O GEMM + residual, RMSNorm, gate_up "
                                "GEMM, SiLU*up, down GEMM + residual") if args.config == "cfg2" else
                               "cfg5: beam-width-4 CoW fork of the last partial page + KV append "
                               "+ fp8-e4m3 paged decode attention, long-tail ctx",
                   "batch": B, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "block_size": BS,
                   "ctx": f"U[{CTX_LO},{CTX_HI}]+1" if args.config == "cfg2" else
                          "80% U[1024,8192] + 20% U[16384,32768], +1",
                   "mean_len": float(L.mean()),
                   "kv_sets_cycled": args.layers,
                   "kv_dtype": "bf16" if args.config == "cfg2" else "fp8-e4m3 (page scales)"},
        "kv_frac_of_hbm_peak": round(kv_gbs / HBM_PEAK_GBS, 4),
        "attn_us_per_call": round(attn_b2b_ms * 1e3, 2),
        "attn_us_in_component_pass": round(per["attn"] * 1e3, 2),
        "kv_bytes_per_layer_step": kv_bytes,
        "attn_stream_kernel_us": round(stream_us, 2),
        # the dominant kernel (attn_decode_stream): algorithmic K+V bytes per
        # launch / its average launch duration by HIP events; `value` above
        # prices the whole call (the kernel, the log-sum-exp merge and the gap)
        "roofline": {"bound": "hbm", "achieved": round(stream_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(stream_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(args.config, "traffic_bytes_stream_kernel"),
                     "kernel": "attn_decode_stream (HIP events around each launch, back to back "
                               "over the cycled KV sets)",
                     "kernel_us": round(stream_us, 2),
                     "algorithmic_bytes": kv_bytes,
                     "call": {"us": round(attn_b2b_ms * 1e3, 2), "gbs": round(kv_gbs, 1),
                              "frac": round(kv_gbs / HBM_PEAK_GBS, 4),
                              "traffic": measured_traffic(args.config)}},
        "append_us": round((per["append"] if args.attn_only else extra["append"]) * 1e3, 2),
        "wall_s_timed": round(wall, 3),
    }
    if args.config == "cfg5":
        geo5 = case.geometry
        result["beam_fork_us"] = round(per["beam_fork"] * 1e3, 2)
        fork_ms = [ev[i][names.index("beam_fork")].elapsed_time(ev[i][names.index("beam_fork") + 1])
                   for i in range(args.steps)]
        host = beam["host_us"][-args.steps:]
        result["beam_fork"] = {"beam_width": BEAM_WIDTH, "parents": B,
                               "median_us": round(float(np.median(fork_ms)) * 1e3, 2),
                               "host_call_us_median": round(float(np.median(host)), 2),
                               "cow_pages_per_step": beam["copies"],
                               "cow_copy_bytes_per_step": beam["copies"] * 2 * args.layers *
                               geo5["block_bytes"],
                               "note": "host fork/CoW bookkeeping + one page-copy kernel, "
                                       "HIP events around the call"}
        # the decoder layer on the fp8 pool: kcmm_decode_layers_on_stream over
        # the pool's layers (bf16 activations and weights, fp8 KV with the
        # fp8 append), one weight set
        w = {name: (torch.randn((n, k), generator=g, device=dev) * 0.02).to(torch.bfloat16)
             for name, n, k in GEMMS}
        for name in ("attn_norm", "mlp_norm"):
            w[name] = (1.0 + 0.1 * torch.randn(HIDDEN, generator=g, device=dev)).to(torch.bfloat16)
        lw = KcmmLayerWeights(**{k: w[k].data_ptr() for k in
                                 ("attn_norm", "qkv", "o", "mlp_norm", "gate_up", "down")})
        hid5 = torch.randn((B, HIDDEN), generator=g, device=dev).to(torch.bfloat16)

        def fp8_layers():
            case.pool.decode_layers(first_layer=0, weights=[lw] * args.layers,
                                    hidden_ptr=hid5.data_ptr(), block_tables_ptr=dv["bt"].data_ptr(),
                                    seq_lens_ptr=dv["sl"].data_ptr(),
                                    block_offsets_f16_ptr=dv["offs"].data_ptr(),
                                    inv_freq_ptr=inv_freq.data_ptr(), batch=B, hidden_size=HIDDEN,
                                    num_q_heads=HQ, intermediate_size=INTER,
                                    max_blocks_per_seq=case.mbps, rms_eps=RMS_EPS, stream_ptr=sp)
        fp8_layers()
        torch.cuda.synchronize()
        reps = max(2, min(args.steps, 8))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fp8_layers()
        e1.record(stream)
        torch.cuda.synchronize()
        t_l = e0.elapsed_time(e1) / reps / args.layers
        assert torch.isfinite(hid5.float()).all(), "fp8 layer step produced non-finite hidden state"
        # the same with fp8-e4m3 projection weights (kcmm_decode_layers_fp8w_on_stream)
        w8, lw8 = quantize_layer_fp8(w)

        def fp8_layers_fp8w():
            case.pool.decode_layers_fp8w(first_layer=0, weights=[lw8] * args.layers,
                                         hidden_ptr=hid5.data_ptr(),
                                         block_tables_ptr=dv["bt"].data_ptr(),
                                         seq_lens_ptr=dv["sl"].data_ptr(),
                                         block_offsets_f16_ptr=dv["offs"].data_ptr(),
                                         inv_freq_ptr=inv_freq.data_ptr(), batch=B,
                                         hidden_size=HIDDEN, num_q_heads=HQ,
                                         intermediate_size=INTER, max_blocks_per_seq=case.mbps,
                                         rms_eps=RMS_EPS, stream_ptr=sp)
        fp8_layers_fp8w()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(reps):
            fp8_layers_fp8w()
        e1.record(stream)
        torch.cuda.synchronize()
        t_l8 = e0.elapsed_time(e1) / reps / args.layers
        assert torch.isfinite(hid5.float()).all(), "fp8-weight layer step produced non-finite state"
        del w8
        result["fp8_layer_step"] = {
            "t_layer_us": round(t_l * 1e3, 2), "layers_per_call": args.layers, "batch": B,
            "kv_bytes_per_layer": kv_bytes,
            "note": "kcmm_decode_layers_on_stream on the fp8 pool: RMSNorm, QKV (partials) + "
                    "RoPE + fp8 append, fp8 attention, O + residual + RMSNorm, gate/up + SwiGLU, "
                    "down + residual; HIP events around the calls",
            "t_layer_fp8_weights_us": round(t_l8 * 1e3, 2),
            "note_fp8_weights": "the same layers through kcmm_decode_layers_fp8w_on_stream with "
                                "fp8-e4m3 projection weights (per-row amax/448 scales)"}
        log(f"fp8 layer step: {t_l * 1e3:.1f} us per layer ({args.layers} layers per call); "
            f"with fp8 weights {t_l8 * 1e3:.1f} us")
        del w, hid5
    if not args.attn_only:
        t_step_s = extra["decode_step"] / 1e3
        result["decode_tokens_per_s"] = round(B / t_step_s, 1)
        result["t_decode_step_us"] = round(t_step_s * 1e6, 1)
        result["t_layer_us"] = round((t_step_s - extra["logits"] / 1e3) / MODEL_LAYERS * 1e6, 2)
        result["t_logits_us"] = round(extra["logits"] * 1e3, 2)
        if "decode_step_graph" in extra:
            tg = extra["decode_step_graph"] / 1e3
            result["decode_graph"] = {
                "decode_tokens_per_s": round(B / tg, 1), "t_decode_step_us": round(tg * 1e6, 1),
                "note": "the same decode step captured once in a HIP graph and replayed; every "
                        "replay checked bit-exact against the eager step before timing"}
        result["t_layer_single_call_us"] = round(extra["layer_step"] * 1e3, 2)
        result["t_layer_components_us"] = {n: round(per[n] * 1e3, 2) for n in names}
        if "decode_step_fp8w" in extra:
            t8 = extra["decode_step_fp8w"] / 1e3
            wbytes8 = sum(n * k + 4 * n for _, n, k in GEMMS)
            result["fp8_weight_decode"] = {
                "decode_tokens_per_s": round(B / t8, 1), "t_decode_step_us": round(t8 * 1e6, 1),
                "t_layer_us": round((t8 - extra["logits"] / 1e3) / MODEL_LAYERS * 1e6, 2),
                "projection_weight_bytes_per_layer": wbytes8,
                "note": "kcmm_decode_layers_fp8w_on_stream: the decode step with fp8-e4m3 "
                        "projection weights (fp32 row scales), bf16 KV pool, embedding and "
                        "bf16 lm_head as in decode_tokens_per_s; HIP events around each step"}
            log(f"fp8-weight decode step ms={extra['decode_step_fp8w']:.4f}")
        def gemm_report(times_ms, M, residual, plan=True):
            gem = {}
            for name, n, k in GEMMS:
                s = times_ms[name] / 1e3
                flops = 2.0 * M * n * k
                # W, X and Y; with a residual store O and down also read it
                res = 2 if residual and name in ("o", "down") else 1
                byts = 2.0 * (n * k + M * k + M * n * res)
                ceiling = min(BF16_PEAK_TFLOPS * 1e12, HBM_PEAK_GBS * 1e9 * flops / byts)
                gem[name] = {"us": round(times_ms[name] * 1e3, 2),
                             "tflops": round(flops / s / 1e12, 1),
                             "gbs": round(byts / s / 1e9, 1),
                             "frac_of_min_roofline": round(flops / s / ceiling, 4),
                             "frac_of_mfma_peak": round(flops / s / (BF16_PEAK_TFLOPS * 1e12), 4)}
                if plan:
                    # split-K partials: written by the GEMM, read back by the reduction
                    p = lib.gemm_plan(M, n, k)
                    gem[name]["splits"] = p["splits"]
                    gem[name]["partial_bytes"] = 2 * p["partial_bytes"]
                    gem[name]["gbs_incl_partials"] = round((byts + 2 * p["partial_bytes"]) / s / 1e9, 1)
            return gem
        result["gemm_m64"] = gemm_report(per, B, True)
        result["gemm_m256"] = gemm_report(m256, 256, False)
        result["gemm_m256"]["backend"] = "tiled MFMA kernel (gemm_tiled.hip)"
        result["gemm_m256"]["note"] = ("each timed call starts with the Infinity Cache flushed "
                                       "(512 MiB write outside the events), as in a layer loop")
        prev = os.environ.get("KCMM_GEMM_TILED")
        os.environ["KCMM_GEMM_TILED"] = "0"        # the weight-stream kernel's own plan
        lib.reload_tunables()
        result["gemm_m256_stream_kernel"] = gemm_report(m256_stream, 256, False)
        if prev is None:
            os.environ.pop("KCMM_GEMM_TILED", None)
        else:
            os.environ["KCMM_GEMM_TILED"] = prev
        lib.reload_tunables()
        result["gemm_m256_torch_reference"] = gemm_report(m256_torch, 256, False, plan=False)
        # plain products at M = 64 with the Infinity Cache flushed before each
        # call: this library's weight-stream kernel against torch.matmul
        result["gemm_m64_cold"] = {
            "kcmm": gemm_report(m64_cold, B, False),
            "torch_reference": gemm_report(m64_torch, B, False, plan=False),
            "note": "plain products (no residual), each timed call after a 512 MiB write that "
                    "flushes the Infinity Cache; torch.matmul is ROCm's GEMM library, timed "
                    "for comparison only"}
        result["tiering"] = tiering_report(lib, args)
    if not args.no_cpu_baseline:
        threads = len(os.sched_getaffinity(0))
        log(f"cpu baseline on {threads} threads ...")
        result["cpu_baseline"] = cpu_baseline(case, args.cpu_seconds, threads)
        result["cpu_baseline_detail"] = cpu_baseline_detail(lib, case, args, threads)
    else:
        result["cpu_baseline"] = None
    case.pool.destroy()
    if args.config == "cfg2" and not args.attn_only and not args.no_sub_configs:
        del case
        torch.cuda.empty_cache()
        # BASELINE configs[2] and configs[4], each timed in a child process
        result["cfg3_prefill"] = sub_config("cfg3", args)
        result["cfg5_fp8"] = sub_config("cfg5", args)
    print(json.dumps(result), flush=True)


def tiering_report(lib, args) -> dict:
    """HBM <-> host swap of whole blocks at the model shape: 32 layers of
    bf16 K and V pages (Hkv 8, D 128, 16 tokens: 32 KiB each, 2 MiB per block
    over all layers); kcmm_evict_blocks / kcmm_restore_evicted_blocks of 64
    blocks (the reference's default batch) timed on the host clock (both are
    synchronous), best of a few reps."""
    from lattice_amd.bindings import KV_BF16, make_config
    cfg = make_config(num_layers=MODEL_LAYERS, kv_heads=8, head_dim=128, max_batch=4,
                      max_seq_len=4096, tiering=True, max_blocks=512)
    pool = lib.create_pool(cfg, KV_BF16)
    try:
        n = 64
        blocks = pool.alloc_blocks(n)
        per_block = 2 * MODEL_LAYERS * pool.stats()["block_bytes"]
        ev, rs = [], []
        for rep in range(4):
            t0 = time.perf_counter()
            got = pool.evict_blocks(n)
            t1 = time.perf_counter()
            pool.restore_blocks(blocks)
            t2 = time.perf_counter()
            assert got == n
            ev.append(t1 - t0)
            rs.append(t2 - t1)
        gb = n * per_block / 1e9
        out = {"blocks_per_call": n, "bytes_per_call": n * per_block,
               "evict_ms": round(min(ev) * 1e3, 2), "restore_ms": round(min(rs) * 1e3, 2),
               "evict_gbs": round(gb / min(ev), 2), "restore_gbs": round(gb / min(rs), 2),
               "note": "host clock around the synchronous C calls; one gather/scatter launch per "
                       "64 blocks + one 2 MiB copy per block to/from page-locked swap memory; "
                       "host link PCIe Gen5 x16 (64 GB/s per direction)"}
        log(f"tiering: evict {out['evict_gbs']} GB/s, restore {out['restore_gbs']} GB/s "
            f"({n} blocks x {per_block >> 20} MiB)")
        return out
    finally:
        pool.destroy()


if __name__ == "__main__":
    main()
