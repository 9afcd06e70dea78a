"""BASELINE configs at their full workloads on the GPU, through the C ABI and
against the oracle:

* fp8-e4m3 pages, B = 128, 32/8 heads, head_dim 128, contexts
  80% U[1024, 8192] + 20% U[16384, 32768] (+ the appended token), pages
  filled on the device and read back; attention within 3e-2 of the fp64
  oracle, then one beam-width-4 fork of every sequence
  (kcmm_fork_beams_on_stream) against the oracle pool doing fork + CoW per
  child: child ids, every table, every refcount and every byte of both
  regions after the copy kernel;
* chunked prefill with a shared 1024-token prefix at its full
  batch of 16 (256-token suffix chunks), within 1e-2;
* configs[1]'s decoder layer: kcmm_decode_layer_step_on_stream at B = 64,
  hidden 4096, 32/8 heads, intermediate 14336, contexts U[512, 4096] + 1:
  every stage against the oracle's stage at 1e-2, the layer step equal to
  its components bit for bit, and the layer against the oracle's layer.
"""
import math

import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, KV_FP8, KcmmLayerWeights, memcpy_dtoh, memcpy_htod
from lattice_amd.workload import build_decode_case, build_prefix_shared_case
from tests import layer_stages as LS

pytestmark = pytest.mark.gpu

SB = 2 * 1024 * 1024
HQ, HKV, D, BS = 32, 8, 128, 16


def rel_err(got, ref):
    return float(np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30))


def regions(pool, layer=0):
    n = pool.stats()["superblock_count"] * SB
    return memcpy_dtoh(pool.va_k(layer), n), memcpy_dtoh(pool.va_v(layer), n)


def test_cfg5_fp8_full_attention_and_beam_fork(gpu_lib):
    import torch
    rng = np.random.default_rng(5)
    B, width = 128, 4
    long = rng.random(B) < 0.2
    ctx = np.where(long, rng.integers(16384, 32769, size=B), rng.integers(1024, 8193, size=B))
    L = ctx + 1
    print(f"cfg5: {int(L.sum())} tokens, max {int(L.max())}", flush=True)
    case = build_decode_case(gpu_lib, batch=B, num_q_heads=HQ, kv_heads=HKV, head_dim=D,
                             block_size=BS, ctx_lens=L, dtype=KV_FP8, seed=6, host_mirror=False)
    try:
        g = case.geometry
        kreg, vreg = regions(case.pool)
        case.dev["out"].fill_(float("nan"))
        case.run_attention(stream_ptr=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        got = O.decode(O.BF16, case.out_bits()).astype(np.float64)
        ref = O.attn_decode_f64(KV_FP8, case.q_bits, kreg, vreg, case.block_tables,
                                case.seq_lens, case.offsets_f16, HQ, HKV, D, BS, g["row_bytes"],
                                g["data_bytes"], 1 / math.sqrt(D))
        err = rel_err(got, ref)
        print(f"cfg5 fp8 attention rel err {err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= 3e-2
        # the oracle pool replays the workload's allocation and registrations
        opool = O.OraclePool(BS, 1, HKV, D, B, int(L.max()), O.FP8)
        pages = [max(1, -(-int(n) // BS)) for n in L]
        total = sum(pages)
        oids = []
        for start in range(0, total, 4096):
            oids += opool.alloc(min(4096, total - start))
        used = {int(case.block_tables[b, i]) for b in range(B) for i in range(pages[b])}
        assert used == set(oids)
        for b in range(B):
            s = opool.register(case.block_tables[b, :pages[b]].tolist())
            assert s == b
            opool.update_seq_len(s, int(L[b]))
        stream = torch.cuda.current_stream()
        children, ncopy = case.pool.fork_beams(list(range(B)), width,
                                               stream_ptr=stream.cuda_stream)
        stream.synchronize()
        ochildren, opairs = [], []
        for s in range(B):
            for _ in range(width - 1):
                c = opool.fork(s)
                ochildren.append(c)
                logical = int(L[s]) // BS
                if logical < len(opool.block_table(c)):
                    rc, pair = opool.cow(c, logical)
                    if rc == 1:
                        opairs.append(tuple(pair))
        assert children == ochildren and ncopy == len(opairs)
        print(f"beam fork: {len(children)} children, {ncopy} page copies", flush=True)
        seen = set()
        for s in list(range(B)) + children:
            t = case.pool.block_table(s)
            assert t == opool.block_table(s), s
            seen.update(t)
        for blk in seen:
            assert case.pool.refcount(blk) == opool.refcount(blk), blk
        # the copies' new pages may lie in superblocks the fork added: bytes
        # there that no copy wrote are whatever the region held
        gk, gv = regions(case.pool)
        kexp = np.concatenate([kreg, gk[kreg.size:]])
        vexp = np.concatenate([vreg, gv[vreg.size:]])
        O.copy_pages([kexp, vexp], [(opool.block_offset(a), opool.block_offset(b))
                                    for a, b in opairs], case.pool.stats()["block_bytes"])
        assert np.array_equal(gk, kexp) and np.array_equal(gv, vexp)
    finally:
        case.pool.destroy()


def test_cfg3_prefix_shared_prefill_full_batch(gpu_lib):
    import torch
    case = build_prefix_shared_case(gpu_lib, batch=16, prefix_tokens=1024, suffix_tokens=256,
                                    chunk=256, num_q_heads=HQ, kv_heads=HKV, head_dim=D,
                                    block_size=BS, dtype=KV_BF16, seed=33)
    try:
        pre = case.block_tables[:, :64]
        assert (pre == pre[0]).all() and case.pool.refcount(int(pre[0, 0])) == 16
        case.dev["out"].fill_(float("nan"))
        case.run(stream_ptr=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        kreg, vreg = regions(case.pool)
        got = O.decode(O.BF16, case.dev["out"].cpu().view(torch.int16).numpy().view(np.uint16))
        ref = O.attn_prefill_f64(KV_BF16, case.q_bits, kreg, vreg, case.block_tables,
                                 case.seq_lens, case.qsl, case.offsets_f16, HQ, HKV, D, BS,
                                 HKV * D * 2, HKV * D * 2 * BS, 1 / math.sqrt(D))
        err = rel_err(got.astype(np.float64), ref)
        print(f"cfg3 full batch prefill rel err {err:.3e}", flush=True)
        assert np.isfinite(got).all() and err <= 1e-2
    finally:
        case.pool.destroy()


def test_cfg2_decoder_layer_full_size(gpu_lib):
    """The Cfg2 layer (B = 64, Llama-3-8B dims) stage by stage against the
    oracle at 1e-2 (tests/layer_stages.py), then the layer step from the same
    pages: the components' bits, and the whole layer against the oracle's."""
    import torch
    rng = np.random.default_rng(21)
    B, H, I = 64, 4096, 14336
    L = rng.integers(512, 4097, size=B) + 1
    case = build_decode_case(gpu_lib, batch=B, num_q_heads=HQ, kv_heads=HKV, head_dim=D,
                             block_size=BS, ctx_lens=L, dtype=KV_BF16, seed=22, host_mirror=False)
    try:
        g = case.geometry
        enc = lambda shape, std: O.encode(O.BF16, rng.standard_normal(shape, dtype=np.float32) * std)
        w = {"attn_norm": O.encode(O.BF16, 1.0 + 0.1 * rng.standard_normal(H)),
             "qkv": enc(((HQ + 2 * HKV) * D, H), 0.02), "o": enc((H, HQ * D), 0.02),
             "mlp_norm": O.encode(O.BF16, 1.0 + 0.1 * rng.standard_normal(H)),
             "gate_up": enc((2 * I, H), 0.02), "down": enc((H, I), 0.02)}
        wdev = {k: torch.from_numpy(v.view(np.int16)).view(torch.bfloat16).cuda()
                for k, v in w.items()}
        lw = KcmmLayerWeights(**{k: t.data_ptr() for k, t in wdev.items()})
        hid = O.encode(O.BF16, rng.standard_normal((B, H)))
        inv = O.default_inv_freq(500000.0, D)
        invd = torch.from_numpy(inv.astype(np.float32)).cuda()
        stream = torch.cuda.current_stream().cuda_stream
        st = LS.run_stages(gpu_lib, case, wdev, hid, invd, HQ, H, I, 1e-5, stream)
        errs = LS.check_stages(st, case, w, inv, HQ, I, 1e-5, KV_BF16)
        print("cfg2 layer stages: " + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()),
              flush=True)
        kreg, vreg = st["kv0"]
        memcpy_htod(case.pool.va_k(0), kreg)
        memcpy_htod(case.pool.va_v(0), vreg)
        hd = torch.from_numpy(hid.view(np.int16)).view(torch.bfloat16).cuda()
        dv = case.dev
        case.pool.decode_layer_step(layer_idx=0, weights=lw, hidden_ptr=hd.data_ptr(),
                                    block_tables_ptr=dv["bt"].data_ptr(),
                                    seq_lens_ptr=dv["sl"].data_ptr(),
                                    block_offsets_f16_ptr=dv["offs"].data_ptr(),
                                    inv_freq_ptr=invd.data_ptr(), batch=B, hidden_size=H,
                                    num_q_heads=HQ, intermediate_size=I,
                                    max_blocks_per_seq=case.mbps, rms_eps=1e-5,
                                    stream_ptr=stream)
        torch.cuda.synchronize()
        out_bits = hd.cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(out_bits, st["out"]), "layer step != its components"
        got = O.decode(O.BF16, out_bits).astype(np.float64)
        ref = O.decode_layer_step_f64(hid, w, kreg, vreg, case.block_tables, case.seq_lens,
                                      case.offsets_f16, inv, HQ, HKV, D, I, BS, g["row_bytes"],
                                      1e-5, dtype=KV_BF16, data_bytes=g["data_bytes"])
        x = O.decode(O.BF16, hid).astype(np.float64)
        err, upd = rel_err(got, ref), rel_err(got - x, ref - x)
        print(f"cfg2 layer B={B} I={I}: err {err:.2e}, update err {upd:.2e}", flush=True)
        # every stage above holds 1e-2; the whole layer's update is bounded
        # at twice its measured error (MI355X: 1.03e-2)
        assert np.isfinite(got).all() and err <= 1e-2 and upd <= 2.1e-2
    finally:
        case.pool.destroy()
