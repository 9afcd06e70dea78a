"""KV append on the GPU through the C ABI: the reference's KAT (ref
scripts/kcmm/kv_write_ffi_smoke.py) replayed on libkcmm.so, region bytes
compared bit-exactly with the oracle after every step; then randomized
appends (16-bit and fp8 pages) against the oracle."""
import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import (KV_BF16, KV_F16, KV_FP8, make_config, memcpy_dtoh,
                                  memset_d8)
from tests import kat_kv_write as K

pytestmark = pytest.mark.gpu

SB = 2 * 1024 * 1024


def region_bytes(pool, layer=0):
    n = pool.stats()["superblock_count"] * SB
    return memcpy_dtoh(pool.va_k(layer), n), memcpy_dtoh(pool.va_v(layer), n)


def zero_regions(pool):
    n = pool.stats()["superblock_count"] * SB
    for l in range(pool.stats()["num_layers"]):
        memset_d8(pool.va_k(l), 0, n)
        memset_d8(pool.va_v(l), 0, n)


def t16(bits, torch):
    return torch.from_numpy(bits.view(np.int16)).view(torch.float16).cuda()


def test_kat_bit_exact_vs_oracle(gpu_lib):
    import torch
    ref = K.run_oracle()
    c = K.KAT["config"]
    bs, step = c["block_size"], c["kv_heads"] * c["head_dim"]
    pool = gpu_lib.create_pool(make_config(block_size=bs, max_blocks=c["max_blocks"],
                                           num_layers=c["num_layers"], kv_heads=c["kv_heads"],
                                           head_dim=c["head_dim"], max_batch=c["max_batch"],
                                           max_seq_len=c["max_seq_len"]), KV_F16)
    try:
        ids = pool.alloc_blocks(K.KAT["setup"]["alloc"])
        inactive = ids[K.KAT["setup"]["free_index"]]
        pool.free_blocks([inactive])
        blocks = ids[: K.KAT["setup"]["register_first"]]
        seq = pool.register_sequence(blocks)
        assert (blocks, inactive, seq) == (ref["blocks"], ref["inactive"], ref["seq"])
        assert pool.block_table(seq, 4) == blocks
        zero_regions(pool)
        stream = torch.cuda.current_stream()

        pw = K.KAT["position_write"]
        k, v = t16(K.f16_rows(2, step, pw["k_offset"]), torch), t16(K.f16_rows(2, step, pw["v_offset"]), torch)
        torch.cuda.synchronize()
        pool.append_kv_step(0, [seq, seq], pw["positions"], k.data_ptr(), v.data_ptr())
        pool.synchronize()
        got = region_bytes(pool)
        assert np.array_equal(got[0], ref["steps"][0][1]) and np.array_equal(got[1], ref["steps"][0][2])

        hs = K.KAT["host_slot_write"]
        k, v = t16(K.f16_rows(3, step, hs["k_offset"]), torch), t16(K.f16_rows(3, step, hs["v_offset"]), torch)
        pool.append_kv_slots(0, K.resolve_slots(hs["slots"], blocks, bs), k.data_ptr(), v.data_ptr(),
                             stream_ptr=stream.cuda_stream)
        stream.synchronize()
        got = region_bytes(pool)
        assert np.array_equal(got[0], ref["steps"][1][1]) and np.array_equal(got[1], ref["steps"][1][2])

        ds = K.KAT["device_slot_write"]
        k, v = t16(K.f16_rows(3, step, ds["k_offset"]), torch), t16(K.f16_rows(3, step, ds["v_offset"]), torch)
        offs = pool.all_block_offsets_f16()
        valid = pool.all_block_valid_flags()
        assert offs == ref["offsets"] and valid == ref["valid"]
        slots_t = torch.tensor(K.resolve_slots(ds["slots"], blocks, bs), dtype=torch.int64, device="cuda")
        offs_t = torch.tensor(offs, dtype=torch.int64, device="cuda")
        valid_t = torch.tensor(valid, dtype=torch.uint8, device="cuda")
        status = torch.zeros(1, dtype=torch.int32, device="cuda")
        common = dict(layer_idx=0, block_offsets_f16_ptr=offs_t.data_ptr(),
                      valid_blocks_ptr=valid_t.data_ptr(), block_offsets_f16_len=len(offs),
                      stream_ptr=stream.cuda_stream)
        pool.append_kv_device_slots_on_stream(slot_mapping_ptr=slots_t.data_ptr(), batch=3,
                                              k_src_ptr=k.data_ptr(), v_src_ptr=v.data_ptr(),
                                              status_ptr=status.data_ptr(), **common)
        stream.synchronize()
        assert int(status.item()) == ref["steps"][2][3] == 0
        got = region_bytes(pool)
        assert np.array_equal(got[0], ref["steps"][2][1]) and np.array_equal(got[1], ref["steps"][2][2])

        # bad slots (ref kv_write_ffi_smoke.py:423-505)
        invalid_slot = c["max_blocks"] * bs
        with pytest.raises(Exception):
            pool.append_kv_slots(0, [invalid_slot], k[:1].data_ptr(), v[:1].data_ptr(),
                                 stream_ptr=stream.cuda_stream)
        for slot, expect in ((inactive * bs, ref["inactive_status"]), (invalid_slot, ref["invalid_status"])):
            st = torch.zeros(1, dtype=torch.int32, device="cuda")
            sl = torch.tensor([slot], dtype=torch.int64, device="cuda")
            pool.append_kv_device_slots_on_stream(slot_mapping_ptr=sl.data_ptr(), batch=1,
                                                  k_src_ptr=k.data_ptr(), v_src_ptr=v.data_ptr(),
                                                  status_ptr=st.data_ptr(), **common)
            stream.synchronize()
            assert int(st.item()) == expect
        got = region_bytes(pool)
        assert np.array_equal(got[0], ref["final"][0]) and np.array_equal(got[1], ref["final"][1])
        pool.unregister_sequence(seq)
        assert pool.stats()["blocks_in_use"] == ref["blocks_in_use_after"] == 0
    finally:
        pool.destroy()


@pytest.mark.parametrize("dtype", [KV_BF16, KV_FP8])
def test_random_decode_appends_vs_oracle(gpu_lib, dtype):
    """Many decode steps of 1 token per sequence (device slots) into shuffled
    pages; region bytes bit-exact with the oracle after the run.  For fp8 the
    rows grow in magnitude now and then, exercising page re-scaling."""
    import torch
    rng = np.random.default_rng(10 + dtype)
    B, hk, d, bs, L = 6, 8, 128, 16, 2
    pool = gpu_lib.create_pool(make_config(num_layers=L, kv_heads=hk, head_dim=d, max_batch=B,
                                           max_seq_len=80), dtype)
    opool = O.OraclePool(bs, L, hk, d, B, 80, dtype)
    try:
        n_pages = 5
        ids = pool.alloc_blocks(B * n_pages)
        assert ids == opool.alloc(B * n_pages)
        perm = rng.permutation(ids)
        tables = [perm[i * n_pages:(i + 1) * n_pages].tolist() for i in range(B)]
        zero_regions(pool)
        nb = pool.stats()["superblock_count"] * SB
        oreg = [[np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)] for _ in range(L)]
        offs = pool.all_block_offsets_f16()
        offs_t = torch.tensor(offs, dtype=torch.int64, device="cuda")
        g_row = hk * d * (1 if dtype == KV_FP8 else 2)
        data_bytes = g_row * bs
        stream = torch.cuda.current_stream()
        for t in range(70):
            pos = np.full(B, t)
            slots = [tables[b][t // bs] * bs + t % bs for b in range(B)]
            for layer in range(L):
                mag = 4.0 if (dtype == KV_FP8 and rng.random() < 0.1) else 1.0
                x = (rng.standard_normal((2, B, hk * d)) * mag).astype(np.float32)
                bits = O.encode(O.BF16, x)
                k = torch.from_numpy(bits[0].view(np.int16)).view(torch.bfloat16).cuda()
                v = torch.from_numpy(bits[1].view(np.int16)).view(torch.bfloat16).cuda()
                sl = torch.tensor(slots, dtype=torch.int64, device="cuda")
                pool.append_kv_device_slots_on_stream(
                    layer_idx=layer, slot_mapping_ptr=sl.data_ptr(),
                    block_offsets_f16_ptr=offs_t.data_ptr(), valid_blocks_ptr=0,
                    block_offsets_f16_len=len(offs), batch=B, k_src_ptr=k.data_ptr(),
                    v_src_ptr=v.data_ptr(), status_ptr=0, stream_ptr=stream.cuda_stream)
                O.kv_write_device_slots(dtype, oreg[layer][0], oreg[layer][1], bits[0], bits[1],
                                        slots, np.asarray(offs, np.uint64), None, bs, hk, d,
                                        g_row, data_bytes)
                stream.synchronize()   # keep sources alive until the kernel ran
        for layer in range(L):
            gk, gv = region_bytes(pool, layer)
            assert np.array_equal(gk, oreg[layer][0]), f"K layer {layer}"
            assert np.array_equal(gv, oreg[layer][1]), f"V layer {layer}"
    finally:
        pool.destroy()


def test_host_variants_validate_before_writing(gpu_lib):
    """All rows are checked before any is enqueued (the reference applies
    the rows before a bad one, ref ffi.rs:1325-1343 -- not replicated)."""
    import torch
    pool = gpu_lib.create_pool(make_config(num_layers=1, kv_heads=2, head_dim=64, max_batch=2,
                                           max_seq_len=64), KV_BF16)
    try:
        ids = pool.alloc_blocks(2)
        seq = pool.register_sequence(ids[:1])
        zero_regions(pool)
        k = torch.ones((2, 128), dtype=torch.bfloat16, device="cuda")
        with pytest.raises(Exception):
            pool.append_kv_step(0, [seq, seq], [0, 16], k.data_ptr(), k.data_ptr())  # 2nd row: no block
        with pytest.raises(Exception):
            pool.append_kv_slots(0, [ids[0] * 16, 999 * 16], k.data_ptr(), k.data_ptr())
        pool.synchronize()
        kr, vr = region_bytes(pool)
        assert not kr.any() and not vr.any()
    finally:
        pool.destroy()


def _prefill_rows(rng, tables, bs, tokens, order):
    """Slot ids of `tokens` tokens per sequence, in one of several call orders:
    'seq' (each sequence's tokens in order, prefill style), 'interleaved'
    (token-major: the rows of one page are not adjacent), 'shuffled' (random
    order, some slots repeated and padding rows mixed in)."""
    per_seq = [[tables[b][t // bs] * bs + t % bs for t in range(tokens)]
               for b in range(len(tables))]
    if order == "seq":
        return [s for row in per_seq for s in row]
    if order == "interleaved":
        return [per_seq[b][t] for t in range(tokens) for b in range(len(tables))]
    flat = [s for row in per_seq for s in row]
    flat += [flat[i] for i in rng.choice(len(flat), size=len(flat) // 8, replace=False)]
    flat += [-1] * 5
    return [flat[i] for i in rng.permutation(len(flat))]


@pytest.mark.parametrize("geom", [(8, 128, 16), (2, 64, 8), (4, 256, 32), (1, 72, 16)],
                         ids=["hk8-d128-bs16", "hk2-d64-bs8", "hk4-d256-bs32", "hk1-d72-bs16"])
@pytest.mark.parametrize("order", ["seq", "interleaved", "shuffled"])
@pytest.mark.parametrize("path", ["device", "host"])
def test_fp8_multi_token_pages_vs_oracle(gpu_lib, order, path, geom):
    """fp8 pages written by calls that put many tokens of a sequence (two and
    a half pages' worth) into the same pages, in several row orders: the rows
    a call writes into a page act as one set (the last row for a repeated
    slot), bit-exact with the oracle, and every row the call wrote decodes
    (torch's e4m3 cast times the footer scale) within one e4m3 step of its
    bf16 input."""
    import torch
    rng = np.random.default_rng(77 + len(order) + (path == "host") + geom[1])
    B, L = 5, 1
    hk, d, bs = geom
    tokens = 2 * bs + bs // 2
    pool = gpu_lib.create_pool(make_config(num_layers=L, kv_heads=hk, head_dim=d, max_batch=B,
                                           max_seq_len=4 * bs, block_size=bs), KV_FP8)
    try:
        n_pages = 3
        ids = pool.alloc_blocks(B * n_pages)
        perm = rng.permutation(ids)
        tables = [perm[i * n_pages:(i + 1) * n_pages].tolist() for i in range(B)]
        for t in tables:
            pool.register_sequence(t)
        zero_regions(pool)
        nb = pool.stats()["superblock_count"] * SB
        ok, ov = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
        offs = pool.all_block_offsets_f16()
        offs_t = torch.tensor(offs, dtype=torch.int64, device="cuda")
        g_row, data_bytes = hk * d, hk * d * bs
        stream = torch.cuda.current_stream()
        for call in range(2):   # the second call rewrites the same pages from slot 0
            slots = _prefill_rows(rng, tables, bs, tokens, order)
            n = len(slots)
            mag = np.where(rng.random(n) < 0.2, 8.0, 1.0)[None, :, None]
            x = (rng.standard_normal((2, n, hk * d)) * mag).astype(np.float32)
            bits = O.encode(O.BF16, x)
            k = torch.from_numpy(bits[0].view(np.int16)).view(torch.bfloat16).cuda()
            v = torch.from_numpy(bits[1].view(np.int16)).view(torch.bfloat16).cuda()
            if path == "device":
                sl = torch.tensor(slots, dtype=torch.int64, device="cuda")
                st = torch.zeros(1, dtype=torch.int32, device="cuda")
                pool.append_kv_device_slots_on_stream(
                    layer_idx=0, slot_mapping_ptr=sl.data_ptr(),
                    block_offsets_f16_ptr=offs_t.data_ptr(), valid_blocks_ptr=0,
                    block_offsets_f16_len=len(offs), batch=n, k_src_ptr=k.data_ptr(),
                    v_src_ptr=v.data_ptr(), status_ptr=st.data_ptr(),
                    stream_ptr=stream.cuda_stream)
            else:
                pool.append_kv_slots(0, slots, k.data_ptr(), v.data_ptr(),
                                     stream_ptr=stream.cuda_stream)
            stream.synchronize()
            if path == "device":
                assert int(st.item()) == 0
            O.kv_write_device_slots(KV_FP8, ok, ov, bits[0], bits[1], slots,
                                    np.asarray(offs, np.uint64), None, bs, hk, d, g_row,
                                    data_bytes)
            gk, gv = region_bytes(pool)
            assert np.array_equal(gk, ok), f"K after call {call}"
            assert np.array_equal(gv, ov), f"V after call {call}"
            last = {sl_: i for i, sl_ in enumerate(slots) if sl_ >= 0}
            for which, reg in ((0, gk), (1, gv)):
                for sl_, i in last.items():
                    page = int(offs[sl_ // bs]) * 2
                    at = page + (sl_ % bs) * g_row
                    sc = reg[page + data_bytes:page + data_bytes + 4 * hk].view(np.float32)
                    codes = torch.from_numpy(reg[at:at + g_row].copy()).view(torch.float8_e4m3fn)
                    got = codes.float().numpy().reshape(hk, d) * sc[:, None]
                    want = O.decode(O.BF16, bits[which][i]).reshape(hk, d)
                    bound = 2.0 ** -3 * np.abs(want) + 2.0 ** -9 * sc[:, None]
                    assert np.all(np.abs(got - want) <= bound * (1 + 1e-6)), (call, which, sl_)
    finally:
        pool.destroy()


def test_fp8_device_slots_status_and_repeat_calls(gpu_lib):
    """The fp8 device-slot writer keeps its per-block row table zero between
    calls: an inactive block (status 2) and an id past the table (status 1,
    first error wins) are skipped, and later calls with other pages and batch
    sizes stay bit-exact with the oracle."""
    import torch
    rng = np.random.default_rng(5)
    hk, d, bs = 2, 128, 16
    pool = gpu_lib.create_pool(make_config(num_layers=1, kv_heads=hk, head_dim=d, max_batch=4,
                                           max_seq_len=128), KV_FP8)
    try:
        ids = pool.alloc_blocks(12)
        zero_regions(pool)
        nb = pool.stats()["superblock_count"] * SB
        ok, ov = np.zeros(nb, np.uint8), np.zeros(nb, np.uint8)
        offs = pool.all_block_offsets_f16()
        valid = np.ones(len(offs), np.uint8)
        valid[ids[3]] = 0
        offs_t = torch.tensor(offs, dtype=torch.int64, device="cuda")
        valid_t = torch.from_numpy(valid).cuda()
        stream = torch.cuda.current_stream()
        # "first error wins" is the first to arrive on the device (ref
        # kcmm_vllm_kv_write.cu: atomicCAS), so a call mixing both kinds may
        # report either; the oracle reports the first in row order
        calls = [(40, [ids[3] * bs + 2, ids[3] * bs + 9], {2}),
                 (7, [len(offs) * bs, len(offs) * bs + 40], {1}),
                 (33, [len(offs) * bs + 3, ids[3] * bs], {1, 2}), (90, [], {0})]
        for call, (n, bad, want) in enumerate(calls):
            good = [i for i in ids if i != ids[3]]
            slots = [int(rng.choice(good)) * bs + int(rng.integers(bs)) for _ in range(n)]
            for j, s in enumerate(bad):
                slots.insert(3 + 5 * j, s)
            x = rng.standard_normal((2, len(slots), hk * d)).astype(np.float32) * 3
            bits = O.encode(O.BF16, x)
            k = torch.from_numpy(bits[0].view(np.int16)).view(torch.bfloat16).cuda()
            v = torch.from_numpy(bits[1].view(np.int16)).view(torch.bfloat16).cuda()
            sl = torch.tensor(slots, dtype=torch.int64, device="cuda")
            st = torch.zeros(1, dtype=torch.int32, device="cuda")
            pool.append_kv_device_slots_on_stream(
                layer_idx=0, slot_mapping_ptr=sl.data_ptr(),
                block_offsets_f16_ptr=offs_t.data_ptr(), valid_blocks_ptr=valid_t.data_ptr(),
                block_offsets_f16_len=len(offs), batch=len(slots), k_src_ptr=k.data_ptr(),
                v_src_ptr=v.data_ptr(), status_ptr=st.data_ptr(), stream_ptr=stream.cuda_stream)
            stream.synchronize()
            ost = O.kv_write_device_slots(KV_FP8, ok, ov, bits[0], bits[1], slots,
                                          np.asarray(offs, np.uint64), valid, bs, hk, d, hk * d,
                                          hk * d * bs)
            assert int(st.item()) in want and ost in want
            gk, gv = region_bytes(pool)
            assert np.array_equal(gk, ok) and np.array_equal(gv, ov), f"call {call}"
    finally:
        pool.destroy()
