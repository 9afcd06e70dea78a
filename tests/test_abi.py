"""The drop-in boundary: every function declared in include/*.h is exported
by libkcmm.so (and by the host-check build), struct layouts match the
reference ABI (ref ffi.rs:2576-2602, kcmm_c_integration.c:29-40), and the
reference's null / argument checks behave as documented.  No GPU calls."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from lattice_amd.bindings import KcmmConfig, KcmmMetrics, KcmmPoolStats, SIGNATURES

ROOT = Path(__file__).resolve().parent.parent
HEADERS = [ROOT / "include" / "kcmm.h", ROOT / "include" / "kcmm_mi355x.h"]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(kcmm_\w+)\s*\(", text))
    return names


def exported(lib: Path):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True,
                         check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_header_lists_reference_surface():
    names = declared_functions()
    # the reference's header entry points plus its 4 unlisted exports (ref ffi.rs)
    ref = {"kcmm_pool_create", "kcmm_pool_destroy", "kcmm_get_last_error", "kcmm_clear_error",
           "kcmm_alloc_blocks", "kcmm_free_blocks", "kcmm_register_sequence",
           "kcmm_unregister_sequence", "kcmm_touch", "kcmm_cool", "kcmm_update_seq_len",
           "kcmm_get_seq_len", "kcmm_append_block_to_sequence", "kcmm_get_block_table",
           "kcmm_get_block_va_offset", "kcmm_get_all_block_offsets_f16", "kcmm_get_block_location",
           "kcmm_get_block_table_va_offsets", "kcmm_get_va_k", "kcmm_get_va_v",
           "kcmm_append_kv_step", "kcmm_append_kv_slots", "kcmm_append_kv_slots_on_stream",
           "kcmm_paged_attn_decode_f16", "kcmm_paged_attn_decode_f16_on_stream",
           "kcmm_paged_attn_decode_f16_on_current_context_stream",
           "kcmm_precompile_paged_attn_decode_f16", "kcmm_evict_blocks",
           "kcmm_restore_evicted_block", "kcmm_restore_evicted_blocks", "kcmm_is_gpu_resident",
           "kcmm_get_metrics", "kcmm_get_pool_stats", "kcmm_blocks_in_use", "kcmm_total_blocks",
           "kcmm_free_physical_blocks", "kcmm_has_free_blocks", "kcmm_active_sequences",
           "kcmm_set_eviction_policy", "kcmm_get_eviction_policy", "kcmm_is_tiering_enabled",
           "kcmm_hint", "kcmm_protect", "kcmm_share_prefix", "kcmm_below_low_watermark",
           "kcmm_synchronize", "kcmm_get_block_size", "kcmm_get_max_blocks_per_seq",
           "kcmm_get_block_bytes", "kcmm_get_num_layers", "kcmm_get_max_batch",
           "kcmm_get_max_seq_len", "kcmm_append_kv_device_slots_on_stream",
           "kcmm_get_all_block_valid", "kcmm_block_state_epoch",
           "kcmm_precompile_vllm_kv_write_f16"}
    assert ref <= names, ref - names


@pytest.mark.parametrize("which", ["product", "hostcheck"])
def test_library_exports_every_declared_symbol(which):
    from lattice_amd import build as b
    lib = b.LIB if which == "product" else b.HOSTCHECK_LIB
    if not lib.exists():
        (b.build_kcmm if which == "product" else b.build_hostcheck)()
    missing = declared_functions() - exported(lib)
    assert not missing, missing
    assert declared_functions() == set(SIGNATURES), set(SIGNATURES) ^ declared_functions()


def test_product_library_loads_without_gpu():
    from lattice_amd import build as b
    if not b.LIB.exists():
        b.build_kcmm()
    lib = C.CDLL(str(b.LIB))
    assert lib.kcmm_get_block_size(None) == 0      # NULL pool -> 0, no device touched


def test_struct_layouts():
    assert C.sizeof(KcmmConfig) == 376
    for field, off in [("max_seq_len", 336), ("low_watermark_threshold", 344),
                       ("background_evict_interval_ms", 352), ("attention_sink_blocks", 360),
                       ("recent_window_blocks", 368)]:
        assert getattr(KcmmConfig, field).offset == off
    assert C.sizeof(KcmmMetrics) == 72
    assert C.sizeof(KcmmPoolStats) == 56


def test_c_header_compiles_and_matches_layout(tmp_path):
    src = tmp_path / "t.c"
    src.write_text("""
#include "kcmm_mi355x.h"
#include <stddef.h>
_Static_assert(sizeof(kcmm_config_t) == 376, "size");
_Static_assert(offsetof(kcmm_config_t, max_seq_len) == 336, "a");
_Static_assert(offsetof(kcmm_config_t, low_watermark_threshold) == 344, "b");
_Static_assert(offsetof(kcmm_config_t, background_evict_interval_ms) == 352, "c");
_Static_assert(offsetof(kcmm_config_t, attention_sink_blocks) == 360, "d");
_Static_assert(offsetof(kcmm_config_t, recent_window_blocks) == 368, "e");
_Static_assert(sizeof(kcmm_pool_stats_t) == 56, "f");
int main(void) { return 0; }
""")
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", str(ROOT / "include"), "-c",
                    str(src), "-o", str(tmp_path / "t.o")], check=True)


def test_null_and_argument_checks(hostcheck_lib):
    """ref ffi.rs conventions on the host-check build (no device)."""
    from lattice_amd.bindings import make_config
    L = hostcheck_lib.lib
    assert L.kcmm_alloc_blocks(None, 1, None) == -1
    assert L.kcmm_free_blocks(None, None, 0) == 0
    assert L.kcmm_get_va_k(None, 0) == 0
    L.kcmm_pool_destroy(None)
    assert L.kcmm_pool_create(None) is None
    pool = hostcheck_lib.create_pool(make_config(num_layers=2, kv_heads=2, head_dim=64,
                                                 max_batch=2, max_seq_len=64))
    try:
        buf = C.create_string_buffer(64)
        assert L.kcmm_get_last_error(pool.handle, buf, 64) == 0 and buf.value == b""
        assert L.kcmm_alloc_blocks(pool.handle, 0, (C.c_uint32 * 1)()) == -1
        assert "zero count" in pool.last_error()
        L.kcmm_clear_error(pool.handle)
        assert pool.last_error() == ""
        assert L.kcmm_get_va_k(pool.handle, 2) == 0 and L.kcmm_get_va_k(pool.handle, 1) != 0
        assert L.kcmm_unregister_sequence(pool.handle, 12345) == 0
        assert L.kcmm_is_tiering_enabled(pool.handle) == 0
        assert L.kcmm_evict_blocks(pool.handle, 4) == 0
        assert L.kcmm_set_eviction_policy(pool.handle, b"lru") == -1
        assert L.kcmm_hint(pool.handle, 3, 1) == -1
        # attention argument validation happens before any device work
        args = [pool.handle, 0, 1, 1, 1, 1, 1, 1, 8, 2, 64, 16, 4, C.c_float(1.0)]
        assert L.kcmm_paged_attn_decode_f16(*args[:2], 0, *args[3:]) == -1
        assert "null pointer" in pool.last_error()
        bad = list(args)
        bad[10] = 512
        assert L.kcmm_paged_attn_decode_f16(*bad) == -1 and "256" in pool.last_error()
        bad = list(args)
        bad[1] = 7
        assert L.kcmm_paged_attn_decode_f16(*bad) == -1 and "layer_idx" in pool.last_error()
        bad = list(args)
        bad[9] = 3
        assert L.kcmm_paged_attn_decode_f16(*bad) == -1 and "geometry" in pool.last_error()
        assert L.kcmm_paged_attn_decode_bf16(*args) == -1 and "dtype" in pool.last_error()
        # small buffers are truncated and terminated (ref ffi.rs:412-422)
        small = C.create_string_buffer(5)
        assert L.kcmm_get_last_error(pool.handle, small, 5) == 4 and len(small.value) == 4
    finally:
        pool.destroy()


def test_decode_layer_entry_points_validate_before_device_work(hostcheck_lib):
    """The decode-layer, fused-GEMM and beam-fork entry points reject bad
    arguments (and say why) before any device work, on the host-check build."""
    from lattice_amd.bindings import KV_BF16, KcmmLayerWeights, KcmmLayerWeightsFp8, make_config
    L = hostcheck_lib.lib
    # pool-free entry points: shape rules
    assert L.kcmm_gemm_bf16_swiglu_on_stream(1, 1, 1, 4, 100, 256, 0) == -1      # inter % 32
    assert L.kcmm_gemm_bf16_add_rmsnorm_on_stream(1, 1, 1, 1, 1, 4, 100, 256,
                                                  C.c_float(1e-5), 0) == -1     # n % 8
    assert L.kcmm_decode_logits_bf16_on_stream(1, 1, 1, 1, 4, 4096, 1000, C.c_float(1e-5),
                                               0) == -1                          # vocab % 64
    assert L.kcmm_rmsnorm_bf16_on_stream(1, 1, 1, 4, 100, C.c_float(-1.0), 0) == -1
    cfg = make_config(num_layers=2, kv_heads=2, head_dim=64, max_batch=4, max_seq_len=64)
    w = KcmmLayerWeights(attn_norm=1, qkv=1, o=1, mlp_norm=1, gate_up=1, down=1)
    f16 = hostcheck_lib.create_pool(cfg)
    bf = hostcheck_lib.create_pool(cfg, KV_BF16)
    try:
        kw = dict(hidden_ptr=1, block_tables_ptr=1, seq_lens_ptr=1, block_offsets_f16_ptr=1,
                  inv_freq_ptr=1, batch=2, hidden_size=512, num_q_heads=8, intermediate_size=768,
                  max_blocks_per_seq=4, rms_eps=1e-5)
        with pytest.raises(Exception):
            f16.decode_layer_step(layer_idx=0, weights=w, **kw)
        assert "bf16" in f16.last_error()
        with pytest.raises(Exception):
            bf.decode_layer_step(layer_idx=0, weights=KcmmLayerWeights(), **kw)
        assert "null" in bf.last_error()
        with pytest.raises(Exception):
            bf.decode_layer_step(layer_idx=0, weights=w, **{**kw, "hidden_size": 500})
        assert "multiples of 256" in bf.last_error()
        with pytest.raises(Exception):
            bf.decode_layer_step(layer_idx=0, weights=w, **{**kw, "num_q_heads": 7})
        with pytest.raises(Exception):
            bf.decode_layers(first_layer=1, weights=[w, w], **kw)            # layers 1..2 of 2
        assert "layer" in bf.last_error()
        with pytest.raises(Exception):
            bf.decode_layers(first_layer=0, weights=[], **kw)
        # fp8-weight layers: every row-scale pointer is required
        w8 = KcmmLayerWeightsFp8(attn_norm=1, qkv=1, qkv_scale=1, o=1, o_scale=1, mlp_norm=1,
                                 gate_up=1, gate_up_scale=1, down=1, down_scale=1)
        for missing in ("qkv_scale", "o_scale", "gate_up_scale", "down_scale"):
            bad = KcmmLayerWeightsFp8(**{f: getattr(w8, f) for f, _ in w8._fields_})
            setattr(bad, missing, 0)
            with pytest.raises(Exception):
                bf.decode_layers_fp8w(first_layer=0, weights=[w8, bad], **kw)
            assert "null weight pointer at layer 1" in bf.last_error()
        with pytest.raises(Exception):
            bf.decode_layers_fp8w(first_layer=0, weights=[w8], **{**kw, "hidden_size": 500})
        assert "multiples of 256" in bf.last_error()
        with pytest.raises(Exception):
            f16.decode_layers_fp8w(first_layer=0, weights=[w8], **kw)
        assert "bf16" in f16.last_error()
        # beam fork: bad width and an unknown parent are errors; a parent whose
        # next token opens a new page forks with no copy (so no device work)
        ids = bf.alloc_blocks(2)
        s = bf.register_sequence(ids)
        bf.update_seq_len(s, 32)
        with pytest.raises(Exception):
            bf.fork_beams([s], 0)
        with pytest.raises(Exception):
            bf.fork_beams([12345], 4)
        children, copies = bf.fork_beams([s], 4)
        assert copies == 0 and len(children) == 3
        for c in children:
            assert bf.block_table(c) == ids
        assert [bf.refcount(i) for i in ids] == [4, 4]
    finally:
        f16.destroy()
        bf.destroy()


def test_fork_beams_all_or_nothing(hostcheck_lib):
    """kcmm_fork_beams_on_stream checks parents, pages and capacity before it
    changes anything: a call that would run out of pages partway through (or
    names an unknown parent after valid ones) fails and leaves tables,
    refcounts, sequences and the free lists exactly as they were."""
    from lattice_amd.bindings import KV_BF16, make_config
    # 64 blocks of capacity at this geometry: bs 16, max_batch 2 x 512 tokens
    cfg = make_config(num_layers=2, kv_heads=2, head_dim=64, max_batch=2, max_seq_len=512)
    pool = hostcheck_lib.create_pool(cfg, KV_BF16)
    try:
        cap = pool.stats()["blocks_per_superblock"]
        parents = []
        for _ in range(4):
            ids = pool.alloc_blocks(3)
            s = pool.register_sequence(ids)
            pool.update_seq_len(s, 40)          # next token in logical block 2 (allocated)
            parents.append(s)
        def snapshot():
            st = pool.stats()
            return (st, [pool.block_table(s) for s in parents],
                    [pool.refcount(i) for i in range(pool.total_blocks())])
        before = snapshot()
        free = before[0]["free_physical_blocks"]
        width = 2 + free // len(parents)        # needs more new pages than are free
        assert len(parents) * (width - 1) > free and cap >= 12
        with pytest.raises(Exception):
            pool.fork_beams(parents, width)
        assert "new pages needed" in pool.last_error()
        assert snapshot() == before
        with pytest.raises(Exception):
            pool.fork_beams(parents + [10 ** 6], 2)
        assert "out of bounds" in pool.last_error()
        assert snapshot() == before
        # the pool still works: a fork with no page copy (no device work) goes through
        pool.update_seq_len(parents[0], 48)
        children, copies = pool.fork_beams(parents[:1], 3)
        assert copies == 0 and [pool.block_table(c) for c in children] == [before[1][0]] * 2
    finally:
        pool.destroy()
