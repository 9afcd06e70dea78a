"""ctypes bindings of libkcmm.so -- the host-side mirror of the reference's
Python seam (ref scripts/kcmm/bindings.py: KcmmConfig, KcmmLibrary, KcmmPool,
KcmmError), over this build's C ABI (include/kcmm.h, include/kcmm_mi355x.h).

The HIP runtime: libkcmm.so and PyTorch-ROCm both need libamdhip64.so.7; the
loader resolves that soname to whichever copy is loaded first, so this module
imports torch (when installed) before opening libkcmm.so to keep one runtime
per process.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

try:  # load torch's HIP runtime first (see module docstring)
    import torch  # noqa: F401
except Exception:  # pragma: no cover - torch is optional for the host-check tier
    torch = None

PKG = Path(__file__).resolve().parent
DEFAULT_LIB = PKG / "libkcmm.so"

KV_F16, KV_BF16, KV_FP8, KV_F32 = 0, 1, 2, 3


class KcmmError(RuntimeError):
    """A libkcmm call returned failure (message from kcmm_get_last_error)."""


class KcmmConfig(C.Structure):
    """kcmm_config_t (ref kcmm.h:81-144); 376 bytes on LP64."""

    _fields_ = [
        ("block_size", C.c_size_t),
        ("max_blocks", C.c_size_t),
        ("cpu_cache_path", C.c_char * 256),
        ("tiering", C.c_int32),
        ("eviction_policy", C.c_int32),
        ("prefetch_window", C.c_size_t),
        ("max_batch_blocks", C.c_size_t),
        ("device_ordinal", C.c_size_t),
        ("num_layers", C.c_size_t),
        ("kv_heads", C.c_size_t),
        ("head_dim", C.c_size_t),
        ("max_batch", C.c_size_t),
        ("max_seq_len", C.c_size_t),
        ("low_watermark_threshold", C.c_float),
        ("background_evict_interval_ms", C.c_uint64),
        ("attention_sink_blocks", C.c_size_t),
        ("recent_window_blocks", C.c_size_t),
    ]


class KcmmMetrics(C.Structure):
    _fields_ = [("ifr", C.c_double), ("pme", C.c_double), ("bu", C.c_double),
                ("rfi", C.c_double), ("gpu_blocks", C.c_uint64), ("cpu_blocks", C.c_uint64),
                ("nvme_blocks", C.c_uint64), ("eviction_count", C.c_uint64),
                ("restoration_count", C.c_uint64)]


class KcmmPoolStats(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "blocks_in_use", "total_blocks", "total_physical_blocks", "free_physical_blocks",
        "active_sequences", "num_layers", "blocks_per_superblock", "superblock_count",
        "block_size", "max_blocks_per_seq", "block_bytes")] + [
        ("tiering_enabled", C.c_int32), ("sharing_enabled", C.c_int32),
        ("physical_idle_ratio", C.c_float)]


def make_config(*, num_layers, kv_heads, head_dim, max_batch, max_seq_len, block_size=16,
                max_blocks=0, device_ordinal=0, tiering=False, eviction_policy=0,
                max_batch_blocks=0) -> KcmmConfig:
    cfg = KcmmConfig()
    cfg.block_size = block_size
    cfg.max_blocks = max_blocks
    cfg.tiering = 1 if tiering else 0
    cfg.eviction_policy = eviction_policy
    cfg.max_batch_blocks = max_batch_blocks
    cfg.num_layers = num_layers
    cfg.kv_heads = kv_heads
    cfg.head_dim = head_dim
    cfg.max_batch = max_batch
    cfg.max_seq_len = max_seq_len
    cfg.device_ordinal = device_ordinal
    return cfg


class KcmmLayerWeights(C.Structure):
    """kcmm_layer_weights_t (include/kcmm_mi355x.h): device addresses of one
    layer's bf16 weights."""
    _fields_ = [("attn_norm", C.c_uint64), ("qkv", C.c_uint64), ("o", C.c_uint64),
                ("mlp_norm", C.c_uint64), ("gate_up", C.c_uint64), ("down", C.c_uint64)]


class KcmmLayerWeightsFp8(C.Structure):
    """kcmm_layer_weights_fp8_t (include/kcmm_mi355x.h): device addresses of
    one layer's weights with fp8-e4m3 projections (codes [out][in] plus an
    fp32 scale per output row) and bf16 RMSNorm weights."""
    _fields_ = [(name, C.c_uint64) for name in
                ("attn_norm", "qkv", "qkv_scale", "o", "o_scale", "mlp_norm", "gate_up",
                 "gate_up_scale", "down", "down_scale")]


_P, _U32, _U64, _I32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int32
_ATTN = [_P, _U32, _U64, _U64, _U64, _U64, _U64] + [_U32] * 6 + [C.c_float]

SIGNATURES = {
    "kcmm_pool_create": ([C.POINTER(KcmmConfig)], _P),
    "kcmm_pool_create_typed": ([C.POINTER(KcmmConfig), _I32], _P),
    "kcmm_pool_destroy": ([_P], None),
    "kcmm_last_create_error": ([C.c_char_p, C.c_size_t], C.c_size_t),
    "kcmm_get_kv_dtype": ([_P], _I32),
    "kcmm_get_backing_kind": ([_P], _I32),
    "kcmm_get_last_error": ([_P, C.c_char_p, C.c_size_t], C.c_size_t),
    "kcmm_clear_error": ([_P], None),
    "kcmm_alloc_blocks": ([_P, _U32, _P], C.c_int),
    "kcmm_free_blocks": ([_P, _P, _U32], C.c_int),
    "kcmm_register_sequence": ([_P, _P, _U32, _P], C.c_int),
    "kcmm_unregister_sequence": ([_P, _U32], C.c_int),
    "kcmm_touch": ([_P, _U32], None),
    "kcmm_cool": ([_P, _U32], None),
    "kcmm_update_seq_len": ([_P, _U32, _U32], None),
    "kcmm_get_seq_len": ([_P, _U32], _U32),
    "kcmm_append_block_to_sequence": ([_P, _U32, _U32], C.c_int),
    "kcmm_get_block_table": ([_P, _U32, _P, _U32, _P], C.c_int),
    "kcmm_get_block_va_offset": ([_P, _U32], _U64),
    "kcmm_get_all_block_offsets_f16": ([_P, _P, _U32, _P], C.c_int),
    "kcmm_get_all_block_valid": ([_P, _P, _U32, _P], C.c_int),
    "kcmm_get_block_location": ([_P, _U32, _P], C.c_int),
    "kcmm_get_block_table_va_offsets": ([_P, _U32, _P, _U32, _P], C.c_int),
    "kcmm_get_va_k": ([_P, _U32], _U64),
    "kcmm_get_va_v": ([_P, _U32], _U64),
    "kcmm_append_kv_step": ([_P, _U32, _P, _P, _U32, _U64, _U64], C.c_int),
    "kcmm_append_kv_slots": ([_P, _U32, _P, _U32, _U64, _U64], C.c_int),
    "kcmm_append_kv_slots_on_stream": ([_P, _U32, _P, _U32, _U64, _U64, _U64], C.c_int),
    "kcmm_append_kv_device_slots_on_stream": ([_P, _U32, _U64, _U64, _U64, _U32, _U32, _U64,
                                               _U64, _U64, _U64], C.c_int),
    "kcmm_precompile_vllm_kv_write_f16": ([_P], C.c_int),
    "kcmm_paged_attn_decode_f16": (_ATTN, C.c_int),
    "kcmm_paged_attn_decode_f16_on_stream": (_ATTN + [_U64], C.c_int),
    "kcmm_paged_attn_decode_f16_on_current_context_stream": (_ATTN + [_U64], C.c_int),
    "kcmm_paged_attn_decode_bf16": (_ATTN, C.c_int),
    "kcmm_paged_attn_decode_bf16_on_stream": (_ATTN + [_U64], C.c_int),
    "kcmm_paged_attn_decode_fp8_on_stream": (_ATTN + [_U64], C.c_int),
    "kcmm_paged_attn_decode_bf16_noalloc_on_stream": (_ATTN + [_U64], C.c_int),
    "kcmm_paged_attn_decode_f32": (_ATTN, C.c_int),
    "kcmm_paged_attn_decode_f32_on_stream": (_ATTN + [_U64], C.c_int),
    "kcmm_paged_attn_prefill_on_stream": ([_P, _U32, _U64, _U64, _U64, _U64, _U64, _U64, _U32,
                                           _U32, _U32, _U32, _U32, _U32, _U32, C.c_float, _U64],
                                          C.c_int),
    "kcmm_precompile_paged_attn_decode_f16": ([_P], C.c_int),
    "kcmm_evict_blocks": ([_P, _U32], _U32),
    "kcmm_restore_evicted_block": ([_P, _U32], _U64),
    "kcmm_restore_evicted_blocks": ([_P, _P, _U32], C.c_int),
    "kcmm_is_gpu_resident": ([_P, _U32], C.c_int),
    "kcmm_get_metrics": ([_P, C.POINTER(KcmmMetrics)], C.c_int),
    "kcmm_get_pool_stats": ([_P, C.POINTER(KcmmPoolStats)], C.c_int),
    "kcmm_blocks_in_use": ([_P], _U32),
    "kcmm_total_blocks": ([_P], _U32),
    "kcmm_block_state_epoch": ([_P], _U64),
    "kcmm_free_physical_blocks": ([_P], _U32),
    "kcmm_has_free_blocks": ([_P], C.c_int),
    "kcmm_active_sequences": ([_P], _U32),
    "kcmm_set_eviction_policy": ([_P, C.c_char_p], C.c_int),
    "kcmm_get_eviction_policy": ([_P, C.c_char_p, _U32], _U32),
    "kcmm_is_tiering_enabled": ([_P], C.c_int),
    "kcmm_hint": ([_P, _U32, C.c_int], C.c_int),
    "kcmm_protect": ([_P, _U32, _P, _U32, C.c_int], C.c_int),
    "kcmm_share_prefix": ([_P, _U32, _U32, _U32, _P], C.c_int),
    "kcmm_fork_sequence": ([_P, _U32, _P], C.c_int),
    "kcmm_get_block_refcount": ([_P, _U32], _U32),
    "kcmm_cow_block_for_append": ([_P, _U32, _U32, _P, _P], C.c_int),
    "kcmm_fork_beams_on_stream": ([_P, C.POINTER(C.c_uint32), _U32, _U32, C.POINTER(C.c_uint32),
                                   _U64], C.c_int),
    "kcmm_copy_blocks_on_stream": ([_P, _P, _U32, _U64], C.c_int),
    "kcmm_copy_blocks_device_on_stream": ([_P, _U64, _U64, _U32, _U64], C.c_int),
    "kcmm_gemm_bf16_on_stream": ([_U64, _U64, _U64, _U32, _U32, _U32, _U64], C.c_int),
    "kcmm_gemm_fp8w_bf16_on_stream": ([_U64, _U64, _U64, _U64, _U32, _U32, _U32, _U64], C.c_int),
    "kcmm_gemm_plan": ([_U32, _U32, _U32, _U32, C.POINTER(C.c_int64)], C.c_int),
    "kcmm_attn_stream_timing_start": ([_U32], C.c_int),
    "kcmm_attn_stream_timing_stop": ([C.POINTER(C.c_double), C.POINTER(C.c_uint32)], C.c_int),
    "kcmm_prefix_hash_blocks": ([_P, _U32, _U32, _U64, _P, _U32, C.POINTER(_U32)], C.c_int),
    "kcmm_prefix_register": ([_P, _U32, _P, _U32, C.POINTER(_U32)], C.c_int),
    "kcmm_prefix_match": ([_P, _P, _U32, _P, C.POINTER(_U32)], C.c_int),
    "kcmm_prefix_attach": ([_P, _U32, _P, _U32, _P, C.POINTER(_U32)], C.c_int),
    "kcmm_prefix_evict": ([_P, _U32, C.POINTER(_U32)], C.c_int),
    "kcmm_prefix_cached_blocks": ([_P], _U32),
    "kcmm_gemm_bf16_add_on_stream": ([_U64, _U64, _U64, _U64, _U32, _U32, _U32, _U64], C.c_int),
    "kcmm_rmsnorm_bf16_on_stream": ([_U64, _U64, _U64, _U32, _U32, C.c_float, _U64], C.c_int),
    "kcmm_silu_mul_bf16_on_stream": ([_U64, _U64, _U32, _U32, _U64], C.c_int),
    "kcmm_embed_tokens_bf16_on_stream": ([_U64, _U64, _U64, _U32, _U32, _U32, _U64], C.c_int),
    "kcmm_gemm_bf16_swiglu_on_stream": ([_U64, _U64, _U64, _U32, _U32, _U32, _U64], C.c_int),
    "kcmm_decode_logits_bf16_on_stream": ([_U64, _U64, _U64, _U64, _U32, _U32, _U32, C.c_float,
                                           _U64], C.c_int),
    "kcmm_gemm_bf16_add_rmsnorm_on_stream": ([_U64, _U64, _U64, _U64, _U64, _U32, _U32, _U32,
                                              C.c_float, _U64], C.c_int),
    "kcmm_qkv_rope_append_bf16_on_stream": ([_P, _U32, _U64, _U64, _U64, _U64, _U64, _U64, _U64,
                                             _U32, _U32, _U32, _U32, _U64], C.c_int),
    "kcmm_rope_append_bf16_on_stream": ([_P, _U32, _U64, _U64, _U64, _U64, _U64, _U64, _U32,
                                         _U32, _U32, _U64], C.c_int),
    "kcmm_decode_layer_step_on_stream": ([_P, _U32, C.POINTER(KcmmLayerWeights), _U64, _U64, _U64,
                                          _U64, _U64, _U32, _U32, _U32, _U32, _U32, C.c_float,
                                          _U64], C.c_int),
    "kcmm_decode_layers_on_stream": ([_P, _U32, _U32, C.POINTER(KcmmLayerWeights), _U64, _U64,
                                      _U64, _U64, _U64, _U32, _U32, _U32, _U32, _U32, C.c_float,
                                      _U64], C.c_int),
    "kcmm_decode_layers_fp8w_on_stream": ([_P, _U32, _U32, C.POINTER(KcmmLayerWeightsFp8), _U64,
                                           _U64, _U64, _U64, _U64, _U32, _U32, _U32, _U32, _U32,
                                           C.c_float, _U64], C.c_int),
    "kcmm_below_low_watermark": ([_P, C.c_float], C.c_int),
    "kcmm_synchronize": ([_P], C.c_int),
    "kcmm_get_block_size": ([_P], _U32),
    "kcmm_get_max_blocks_per_seq": ([_P], _U32),
    "kcmm_get_block_bytes": ([_P], _U32),
    "kcmm_get_num_layers": ([_P], _U32),
    "kcmm_get_max_batch": ([_P], _U32),
    "kcmm_get_max_seq_len": ([_P], _U32),
    "kcmm_reload_tunables": ([], None),
}


def _arr(ctype, values):
    values = list(values)
    return (ctype * max(1, len(values)))(*values)


class KcmmLibrary:
    """Loads libkcmm.so (or the host-check build) and declares every entry point."""

    def __init__(self, path: str | os.PathLike | None = None):
        path = Path(path) if path else Path(os.environ.get("KCMM_LIB_PATH", DEFAULT_LIB))
        if not path.exists():
            raise KcmmError(f"{path} not built: run `python -m lattice_amd.build`")
        self.path = path
        self.lib = C.CDLL(str(path))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(self.lib, name)
            fn.argtypes = args
            fn.restype = res

    def reload_tunables(self) -> None:
        """Re-read the KCMM_* tuning variables (the library reads them once)."""
        self.lib.kcmm_reload_tunables()

    def create_pool(self, config: KcmmConfig, kv_dtype: int = KV_F16) -> "KcmmPool":
        h = self.lib.kcmm_pool_create_typed(C.byref(config), kv_dtype)
        if not h:
            buf = C.create_string_buffer(512)
            self.lib.kcmm_last_create_error(buf, 512)
            raise KcmmError(f"kcmm_pool_create failed: {buf.value.decode()}")
        return KcmmPool(self, h)

    def gemm_bf16(self, x_ptr, w_ptr, y_ptr, m, n, k, stream_ptr=0) -> None:
        if self.lib.kcmm_gemm_bf16_on_stream(x_ptr, w_ptr, y_ptr, m, n, k, stream_ptr) != 0:
            raise KcmmError("kcmm_gemm_bf16_on_stream failed")

    def prefix_hash_blocks(self, tokens, block_size, seed=0):
        """Chained content hashes of the full blocks of a token sequence
        (numpy uint64 array)."""
        import numpy as np
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros(max(len(t) // block_size, 1), dtype=np.uint64)
        cnt = _U32(0)
        if self.lib.kcmm_prefix_hash_blocks(t.ctypes.data if t.size else None, t.size, block_size,
                                            seed, out.ctypes.data, out.size, C.byref(cnt)) != 0:
            raise KcmmError("kcmm_prefix_hash_blocks failed")
        return out[: cnt.value]

    def attn_stream_timing_start(self, max_calls: int) -> None:
        """Start HIP-event timing of the decode-attention streaming kernel."""
        if self.lib.kcmm_attn_stream_timing_start(max_calls) != 0:
            raise KcmmError("kcmm_attn_stream_timing_start failed")

    def attn_stream_timing_stop(self) -> tuple[float, int]:
        """(average streaming-kernel duration in us, launches timed)."""
        avg, n = C.c_double(), C.c_uint32()
        if self.lib.kcmm_attn_stream_timing_stop(C.byref(avg), C.byref(n)) != 0:
            raise KcmmError("kcmm_attn_stream_timing_stop failed")
        return float(avg.value), int(n.value)

    def gemm_plan(self, m, n, k, fp8_weights=False) -> dict:
        """How a plain product of this shape runs: kernel ('stream' / 'tiled'),
        K splits, tiling, bytes of fp32 split partials."""
        out = (C.c_int64 * 4)()
        if self.lib.kcmm_gemm_plan(m, n, k, int(bool(fp8_weights)), out) != 0:
            raise KcmmError("kcmm_gemm_plan failed")
        return {"kernel": ("stream", "tiled")[out[0]], "splits": int(out[1]), "tile": int(out[2]),
                "partial_bytes": int(out[3])}

    def gemm_fp8w_bf16(self, x_ptr, w8_ptr, wscale_ptr, y_ptr, m, n, k, stream_ptr=0) -> None:
        """Y = X (W8 diag(wscale))^T: fp8-e4m3 weights with an fp32 scale per row."""
        if self.lib.kcmm_gemm_fp8w_bf16_on_stream(x_ptr, w8_ptr, wscale_ptr, y_ptr, m, n, k,
                                                  stream_ptr) != 0:
            raise KcmmError("kcmm_gemm_fp8w_bf16_on_stream failed")

    def gemm_bf16_add(self, x_ptr, w_ptr, residual_ptr, y_ptr, m, n, k, stream_ptr=0) -> None:
        """Y = R + X W^T (R may be Y)."""
        if self.lib.kcmm_gemm_bf16_add_on_stream(x_ptr, w_ptr, residual_ptr, y_ptr, m, n, k,
                                                 stream_ptr) != 0:
            raise KcmmError("kcmm_gemm_bf16_add_on_stream failed")

    def rmsnorm_bf16(self, x_ptr, w_ptr, y_ptr, rows, hidden, eps, stream_ptr=0) -> None:
        if self.lib.kcmm_rmsnorm_bf16_on_stream(x_ptr, w_ptr, y_ptr, rows, hidden, C.c_float(eps),
                                                stream_ptr) != 0:
            raise KcmmError("kcmm_rmsnorm_bf16_on_stream failed")

    def embed_tokens_bf16(self, embed_ptr, token_ids_ptr, hidden_ptr, batch, hidden_size, vocab,
                          stream_ptr=0) -> None:
        """hidden[b] = embed[token_ids[b]] (device int32 ids; out-of-range ids: zero rows)."""
        if self.lib.kcmm_embed_tokens_bf16_on_stream(embed_ptr, token_ids_ptr, hidden_ptr, batch,
                                                     hidden_size, vocab, stream_ptr) != 0:
            raise KcmmError("kcmm_embed_tokens_bf16_on_stream failed")

    def silu_mul_bf16(self, gate_up_ptr, act_ptr, rows, intermediate, stream_ptr=0) -> None:
        if self.lib.kcmm_silu_mul_bf16_on_stream(gate_up_ptr, act_ptr, rows, intermediate,
                                                 stream_ptr) != 0:
            raise KcmmError("kcmm_silu_mul_bf16_on_stream failed")

    def decode_logits_bf16(self, hidden_ptr, norm_w_ptr, lm_head_ptr, logits_ptr, batch,
                           hidden_size, vocab_size, eps, stream_ptr=0) -> None:
        """logits = lm_head(rmsnorm(hidden)), bf16 on the device."""
        if self.lib.kcmm_decode_logits_bf16_on_stream(hidden_ptr, norm_w_ptr, lm_head_ptr,
                                                      logits_ptr, batch, hidden_size, vocab_size,
                                                      C.c_float(eps), stream_ptr) != 0:
            raise KcmmError("kcmm_decode_logits_bf16_on_stream failed")

    def gemm_bf16_add_rmsnorm(self, x_ptr, w_ptr, hidden_ptr, norm_w_ptr, normed_ptr, m, n, k,
                              eps, stream_ptr=0) -> None:
        """hidden += x W^T (bf16 rounding of a bf16 model); normed = rmsnorm(hidden)."""
        if self.lib.kcmm_gemm_bf16_add_rmsnorm_on_stream(x_ptr, w_ptr, hidden_ptr, norm_w_ptr,
                                                         normed_ptr, m, n, k, C.c_float(eps),
                                                         stream_ptr) != 0:
            raise KcmmError("kcmm_gemm_bf16_add_rmsnorm_on_stream failed")

    def gemm_bf16_swiglu(self, x_ptr, w_gate_up_ptr, act_ptr, m, intermediate, k,
                         stream_ptr=0) -> None:
        """act = bf16(bf16(silu(x Wg^T)) * (x Wu^T)), W = [Wg; Wu]."""
        if self.lib.kcmm_gemm_bf16_swiglu_on_stream(x_ptr, w_gate_up_ptr, act_ptr, m,
                                                    intermediate, k, stream_ptr) != 0:
            raise KcmmError("kcmm_gemm_bf16_swiglu_on_stream failed")


class KcmmPool:
    """One KCMM pool handle (ref scripts/kcmm/bindings.py KcmmPool)."""

    def __init__(self, library: KcmmLibrary, handle):
        self.library = library
        self.lib = library.lib
        self.handle = C.c_void_p(handle)

    # -- lifecycle / errors --
    def destroy(self) -> None:
        if self.handle:
            self.lib.kcmm_pool_destroy(self.handle)
            self.handle = C.c_void_p(0)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()

    def last_error(self) -> str:
        buf = C.create_string_buffer(1024)
        self.lib.kcmm_get_last_error(self.handle, buf, 1024)
        return buf.value.decode()

    def _check(self, rc: int, op: str) -> None:
        if rc != 0:
            raise KcmmError(f"{op} failed: {self.last_error()}")

    # -- tiering (ref ffi.rs:1900-2008, 2195-2272) --
    LOCATIONS = {0: "gpu", 1: "cpu", 2: "nvme", 3: "evicting", 4: "restoring"}

    def tiering_enabled(self) -> bool:
        return bool(self.lib.kcmm_is_tiering_enabled(self.handle))

    def evict_blocks(self, count: int) -> int:
        return self.lib.kcmm_evict_blocks(self.handle, count)

    def restore_block(self, blk: int) -> int:
        va = self.lib.kcmm_restore_evicted_block(self.handle, blk)
        if va == 0:
            raise KcmmError(f"kcmm_restore_evicted_block failed: {self.last_error()}")
        return va

    def restore_blocks(self, blocks) -> None:
        blocks = list(blocks)
        self._check(self.lib.kcmm_restore_evicted_blocks(self.handle, _arr(C.c_uint32, blocks),
                                                         len(blocks)),
                    "kcmm_restore_evicted_blocks")

    def block_location(self, blk: int):
        v = C.c_int(0)
        if self.lib.kcmm_get_block_location(self.handle, blk, C.byref(v)) != 0:
            return None
        return self.LOCATIONS[v.value]

    def is_gpu_resident(self, blk: int) -> bool:
        return bool(self.lib.kcmm_is_gpu_resident(self.handle, blk))

    def set_eviction_policy(self, name: str) -> None:
        self._check(self.lib.kcmm_set_eviction_policy(self.handle, name.encode()),
                    "kcmm_set_eviction_policy")

    def eviction_policy(self) -> str:
        buf = C.create_string_buffer(64)
        self.lib.kcmm_get_eviction_policy(self.handle, buf, 64)
        return buf.value.decode()

    def hint(self, seq: int, hint: int) -> None:
        self._check(self.lib.kcmm_hint(self.handle, seq, hint), "kcmm_hint")

    def protect(self, seq: int, blocks, level: int) -> None:
        blocks = list(blocks)
        self._check(self.lib.kcmm_protect(self.handle, seq, _arr(C.c_uint32, blocks), len(blocks),
                                          level), "kcmm_protect")

    # -- allocation / sequences --
    def alloc_blocks(self, n: int) -> list[int]:
        out = (C.c_uint32 * max(1, n))()
        self._check(self.lib.kcmm_alloc_blocks(self.handle, n, out), "kcmm_alloc_blocks")
        return list(out[:n])

    def free_blocks(self, blocks) -> None:
        a = _arr(C.c_uint32, blocks)
        self._check(self.lib.kcmm_free_blocks(self.handle, a, len(list(blocks))), "kcmm_free_blocks")

    def register_sequence(self, table) -> int:
        table = list(table)
        out = C.c_uint32(0)
        self._check(self.lib.kcmm_register_sequence(self.handle, _arr(C.c_uint32, table),
                                                    len(table), C.byref(out)),
                    "kcmm_register_sequence")
        return out.value

    def unregister_sequence(self, seq: int) -> None:
        self._check(self.lib.kcmm_unregister_sequence(self.handle, seq), "kcmm_unregister_sequence")

    def append_block_to_sequence(self, seq: int, blk: int) -> None:
        self._check(self.lib.kcmm_append_block_to_sequence(self.handle, seq, blk),
                    "kcmm_append_block_to_sequence")

    def update_seq_len(self, seq: int, n: int) -> None:
        self.lib.kcmm_update_seq_len(self.handle, seq, n)

    def seq_len(self, seq: int) -> int:
        return self.lib.kcmm_get_seq_len(self.handle, seq)

    def block_table(self, seq: int, max_blocks: int = 1 << 16) -> list[int]:
        out = (C.c_uint32 * max_blocks)()
        cnt = C.c_uint32(0)
        self._check(self.lib.kcmm_get_block_table(self.handle, seq, out, max_blocks, C.byref(cnt)),
                    "kcmm_get_block_table")
        return list(out[: cnt.value])

    def block_table_va_offsets(self, seq: int, max_blocks: int = 1 << 16) -> list[int]:
        out = (C.c_uint64 * max_blocks)()
        cnt = C.c_uint32(0)
        self._check(self.lib.kcmm_get_block_table_va_offsets(self.handle, seq, out, max_blocks,
                                                             C.byref(cnt)),
                    "kcmm_get_block_table_va_offsets")
        return list(out[: cnt.value])

    def block_va_offset(self, blk: int) -> int:
        return self.lib.kcmm_get_block_va_offset(self.handle, blk)

    def all_block_offsets_f16(self, max_blocks: int | None = None) -> list[int]:
        n = max_blocks if max_blocks is not None else max(1, self.total_blocks())
        out = (C.c_uint64 * n)()
        cnt = C.c_uint32(0)
        self._check(self.lib.kcmm_get_all_block_offsets_f16(self.handle, out, n, C.byref(cnt)),
                    "kcmm_get_all_block_offsets_f16")
        return list(out[: cnt.value])

    def all_block_valid_flags(self, max_blocks: int | None = None) -> list[int]:
        n = max_blocks if max_blocks is not None else max(1, self.total_blocks())
        out = (C.c_uint8 * n)()
        cnt = C.c_uint32(0)
        self._check(self.lib.kcmm_get_all_block_valid(self.handle, out, n, C.byref(cnt)),
                    "kcmm_get_all_block_valid")
        return list(out[: cnt.value])

    def va_k(self, layer: int) -> int:
        return self.lib.kcmm_get_va_k(self.handle, layer)

    def va_v(self, layer: int) -> int:
        return self.lib.kcmm_get_va_v(self.handle, layer)

    def total_blocks(self) -> int:
        return self.lib.kcmm_total_blocks(self.handle)

    def blocks_in_use(self) -> int:
        return self.lib.kcmm_blocks_in_use(self.handle)

    def epoch(self) -> int:
        return self.lib.kcmm_block_state_epoch(self.handle)

    def kv_dtype(self) -> int:
        return self.lib.kcmm_get_kv_dtype(self.handle)

    def backing_kind(self) -> int:
        return self.lib.kcmm_get_backing_kind(self.handle)

    def stats(self) -> dict:
        s = KcmmPoolStats()
        self._check(self.lib.kcmm_get_pool_stats(self.handle, C.byref(s)), "kcmm_get_pool_stats")
        return {name: getattr(s, name) for name, _ in s._fields_}

    def metrics(self) -> dict:
        m = KcmmMetrics()
        self._check(self.lib.kcmm_get_metrics(self.handle, C.byref(m)), "kcmm_get_metrics")
        return {name: getattr(m, name) for name, _ in m._fields_}

    def synchronize(self) -> None:
        self._check(self.lib.kcmm_synchronize(self.handle), "kcmm_synchronize")

    # -- KV write --
    def append_kv_step(self, layer_idx, seq_indices, positions, k_src_ptr, v_src_ptr) -> None:
        seq_indices, positions = list(seq_indices), list(positions)
        self._check(self.lib.kcmm_append_kv_step(self.handle, layer_idx, _arr(C.c_uint32, seq_indices),
                                                 _arr(C.c_uint32, positions), len(seq_indices),
                                                 k_src_ptr, v_src_ptr), "kcmm_append_kv_step")

    def append_kv_slots(self, layer_idx, slot_mapping, k_src_ptr, v_src_ptr, stream_ptr=None):
        slot_mapping = list(slot_mapping)
        a = _arr(C.c_int64, slot_mapping)
        if stream_ptr is None:
            rc = self.lib.kcmm_append_kv_slots(self.handle, layer_idx, a, len(slot_mapping),
                                               k_src_ptr, v_src_ptr)
        else:
            rc = self.lib.kcmm_append_kv_slots_on_stream(self.handle, layer_idx, a,
                                                         len(slot_mapping), k_src_ptr, v_src_ptr,
                                                         stream_ptr)
        self._check(rc, "kcmm_append_kv_slots")

    def append_kv_device_slots_on_stream(self, *, layer_idx, slot_mapping_ptr,
                                         block_offsets_f16_ptr, valid_blocks_ptr,
                                         block_offsets_f16_len, batch, k_src_ptr, v_src_ptr,
                                         status_ptr, stream_ptr) -> None:
        self._check(self.lib.kcmm_append_kv_device_slots_on_stream(
            self.handle, layer_idx, slot_mapping_ptr, block_offsets_f16_ptr, valid_blocks_ptr,
            block_offsets_f16_len, batch, k_src_ptr, v_src_ptr, status_ptr, stream_ptr),
            "kcmm_append_kv_device_slots_on_stream")

    # -- attention --
    def paged_attn_decode(self, *, layer_idx, query_ptr, out_ptr, block_tables_ptr, seq_lens_ptr,
                          block_offsets_f16_ptr, batch, num_q_heads, kv_heads, head_dim,
                          block_size, max_blocks_per_seq, scale, stream_ptr=None,
                          variant="auto") -> None:
        """Dispatch to the entry point matching the pool dtype (f16/bf16/fp8/fp32)."""
        dt = self.kv_dtype()
        args = (self.handle, layer_idx, query_ptr, out_ptr, block_tables_ptr, seq_lens_ptr,
                block_offsets_f16_ptr, batch, num_q_heads, kv_heads, head_dim, block_size,
                max_blocks_per_seq, C.c_float(scale))
        if dt == KV_F16:
            if stream_ptr is None:
                rc = self.lib.kcmm_paged_attn_decode_f16(*args)
            elif variant == "current_context":
                rc = self.lib.kcmm_paged_attn_decode_f16_on_current_context_stream(*args, stream_ptr)
            else:
                rc = self.lib.kcmm_paged_attn_decode_f16_on_stream(*args, stream_ptr)
        elif dt == KV_BF16:
            if stream_ptr is None:
                rc = self.lib.kcmm_paged_attn_decode_bf16(*args)
            else:
                rc = self.lib.kcmm_paged_attn_decode_bf16_on_stream(*args, stream_ptr)
        elif dt == KV_F32:
            if stream_ptr is None:
                rc = self.lib.kcmm_paged_attn_decode_f32(*args)
            else:
                rc = self.lib.kcmm_paged_attn_decode_f32_on_stream(*args, stream_ptr)
        else:
            rc = self.lib.kcmm_paged_attn_decode_fp8_on_stream(*args, stream_ptr or 0)
        self._check(rc, "paged_attn_decode")

    def paged_attn_prefill(self, *, layer_idx, query_ptr, out_ptr, block_tables_ptr,
                           seq_lens_ptr, query_start_loc_ptr, block_offsets_f16_ptr, batch,
                           total_query_tokens, num_q_heads, kv_heads, head_dim, block_size,
                           max_blocks_per_seq, scale, stream_ptr=0) -> None:
        """Causal chunked prefill (q/out f16 for f16 pools, fp32 for fp32 pools, bf16
        otherwise)."""
        rc = self.lib.kcmm_paged_attn_prefill_on_stream(
            self.handle, layer_idx, query_ptr, out_ptr, block_tables_ptr, seq_lens_ptr,
            query_start_loc_ptr, block_offsets_f16_ptr, batch, total_query_tokens, num_q_heads,
            kv_heads, head_dim, block_size, max_blocks_per_seq, C.c_float(scale), stream_ptr)
        self._check(rc, "paged_attn_prefill")

    # -- decode-step glue and the layer step --
    def rope_append(self, *, layer_idx, qkv_ptr, q_out_ptr, block_tables_ptr, seq_lens_ptr,
                    block_offsets_f16_ptr, inv_freq_ptr, batch, num_q_heads, max_blocks_per_seq,
                    stream_ptr=0) -> None:
        """RoPE of the decode token's q / k, k and v appended to its page row."""
        rc = self.lib.kcmm_rope_append_bf16_on_stream(
            self.handle, layer_idx, qkv_ptr, q_out_ptr, block_tables_ptr, seq_lens_ptr,
            block_offsets_f16_ptr, inv_freq_ptr, batch, num_q_heads, max_blocks_per_seq,
            stream_ptr)
        self._check(rc, "rope_append")

    def qkv_rope_append(self, *, layer_idx, x_ptr, w_qkv_ptr, q_out_ptr, block_tables_ptr,
                        seq_lens_ptr, block_offsets_f16_ptr, inv_freq_ptr, batch, hidden_size,
                        num_q_heads, max_blocks_per_seq, stream_ptr=0) -> None:
        """QKV projection with RoPE and the KV append fused into its store."""
        rc = self.lib.kcmm_qkv_rope_append_bf16_on_stream(
            self.handle, layer_idx, x_ptr, w_qkv_ptr, q_out_ptr, block_tables_ptr, seq_lens_ptr,
            block_offsets_f16_ptr, inv_freq_ptr, batch, hidden_size, num_q_heads,
            max_blocks_per_seq, stream_ptr)
        self._check(rc, "qkv_rope_append")

    def decode_layer_step(self, *, layer_idx, weights: KcmmLayerWeights, hidden_ptr,
                          block_tables_ptr, seq_lens_ptr, block_offsets_f16_ptr, inv_freq_ptr,
                          batch, hidden_size, num_q_heads, intermediate_size, max_blocks_per_seq,
                          rms_eps, stream_ptr=0) -> None:
        """One decoder layer of a decode step, in place on hidden ([batch][hidden] bf16)."""
        rc = self.lib.kcmm_decode_layer_step_on_stream(
            self.handle, layer_idx, C.byref(weights), hidden_ptr, block_tables_ptr, seq_lens_ptr,
            block_offsets_f16_ptr, inv_freq_ptr, batch, hidden_size, num_q_heads,
            intermediate_size, max_blocks_per_seq, C.c_float(rms_eps), stream_ptr)
        self._check(rc, "decode_layer_step")

    def decode_layers(self, *, first_layer, weights, hidden_ptr, block_tables_ptr, seq_lens_ptr,
                      block_offsets_f16_ptr, inv_freq_ptr, batch, hidden_size, num_q_heads,
                      intermediate_size, max_blocks_per_seq, rms_eps, stream_ptr=0) -> None:
        """Layers first_layer .. first_layer + len(weights) - 1 in one call."""
        arr = (KcmmLayerWeights * len(weights))(*weights)
        rc = self.lib.kcmm_decode_layers_on_stream(
            self.handle, first_layer, len(weights), arr, hidden_ptr, block_tables_ptr,
            seq_lens_ptr, block_offsets_f16_ptr, inv_freq_ptr, batch, hidden_size, num_q_heads,
            intermediate_size, max_blocks_per_seq, C.c_float(rms_eps), stream_ptr)
        self._check(rc, "decode_layers")

    def decode_layers_fp8w(self, *, first_layer, weights, hidden_ptr, block_tables_ptr,
                           seq_lens_ptr, block_offsets_f16_ptr, inv_freq_ptr, batch, hidden_size,
                           num_q_heads, intermediate_size, max_blocks_per_seq, rms_eps,
                           stream_ptr=0) -> None:
        """decode_layers with fp8-e4m3 projection weights (KcmmLayerWeightsFp8)."""
        arr = (KcmmLayerWeightsFp8 * len(weights))(*weights)
        rc = self.lib.kcmm_decode_layers_fp8w_on_stream(
            self.handle, first_layer, len(weights), arr, hidden_ptr, block_tables_ptr,
            seq_lens_ptr, block_offsets_f16_ptr, inv_freq_ptr, batch, hidden_size, num_q_heads,
            intermediate_size, max_blocks_per_seq, C.c_float(rms_eps), stream_ptr)
        self._check(rc, "decode_layers_fp8w")

    # -- copy-on-write --
    def fork_sequence(self, src: int) -> int:
        out = C.c_uint32(0)
        self._check(self.lib.kcmm_fork_sequence(self.handle, src, C.byref(out)), "kcmm_fork_sequence")
        return out.value

    def fork_beams(self, parents, beam_width: int, stream_ptr: int = 0):
        """Children (parent-major) and the number of pages copied."""
        n = len(parents)
        par = (C.c_uint32 * max(1, n))(*parents)
        out = (C.c_uint32 * max(1, n * max(0, beam_width - 1)))()
        rc = self.lib.kcmm_fork_beams_on_stream(self.handle, par, n, beam_width, out, stream_ptr)
        if rc < 0:
            raise KcmmError(f"kcmm_fork_beams_on_stream: {self.last_error()}")
        return list(out[:n * max(0, beam_width - 1)]), rc

    def share_prefix(self, src: int, dst: int, n: int) -> list[int]:
        out = (C.c_uint32 * max(1, n))()
        self._check(self.lib.kcmm_share_prefix(self.handle, src, dst, n, out), "kcmm_share_prefix")
        return list(out[:n])

    def refcount(self, blk: int) -> int:
        return self.lib.kcmm_get_block_refcount(self.handle, blk)

    # ---- prefix cache (kcmm_prefix_*) ----
    @staticmethod
    def _hashes(hashes):
        import numpy as np
        h = np.ascontiguousarray(hashes, dtype=np.uint64)
        return h, (h.ctypes.data if h.size else None)

    def prefix_register(self, seq: int, hashes) -> int:
        h, hp = self._hashes(hashes)
        added = C.c_uint32(0)
        self._check(self.lib.kcmm_prefix_register(self.handle, seq, hp, h.size, C.byref(added)),
                    "kcmm_prefix_register")
        return added.value

    def prefix_match(self, hashes) -> list[int]:
        h, hp = self._hashes(hashes)
        out = (C.c_uint32 * max(1, h.size))()
        m = C.c_uint32(0)
        self._check(self.lib.kcmm_prefix_match(self.handle, hp, h.size, out, C.byref(m)),
                    "kcmm_prefix_match")
        return list(out[: m.value])

    def prefix_attach(self, dst: int, hashes) -> list[int]:
        h, hp = self._hashes(hashes)
        out = (C.c_uint32 * max(1, h.size))()
        m = C.c_uint32(0)
        self._check(self.lib.kcmm_prefix_attach(self.handle, dst, hp, h.size, out, C.byref(m)),
                    "kcmm_prefix_attach")
        return list(out[: m.value])

    def prefix_evict(self, n: int = 0xFFFFFFFF) -> int:
        k = C.c_uint32(0)
        self._check(self.lib.kcmm_prefix_evict(self.handle, n, C.byref(k)), "kcmm_prefix_evict")
        return k.value

    def prefix_entries(self) -> int:
        return self.lib.kcmm_prefix_cached_blocks(self.handle)

    def cow_block_for_append(self, seq: int, logical: int):
        s, d = C.c_uint32(0), C.c_uint32(0)
        rc = self.lib.kcmm_cow_block_for_append(self.handle, seq, logical, C.byref(s), C.byref(d))
        if rc < 0:
            raise KcmmError(f"kcmm_cow_block_for_append failed: {self.last_error()}")
        return (s.value, d.value) if rc == 1 else None

    def copy_blocks(self, pairs, stream_ptr=0) -> None:
        flat = [v for p in pairs for v in p]
        self._check(self.lib.kcmm_copy_blocks_on_stream(self.handle, _arr(C.c_uint32, flat),
                                                        len(flat) // 2, stream_ptr),
                    "kcmm_copy_blocks_on_stream")

    def copy_blocks_device(self, pairs_ptr, offsets_ptr, n, stream_ptr=0) -> None:
        self._check(self.lib.kcmm_copy_blocks_device_on_stream(self.handle, pairs_ptr, offsets_ptr,
                                                               n, stream_ptr),
                    "kcmm_copy_blocks_device_on_stream")


# ---- raw HIP helpers (test/bench plumbing for pool-owned device memory) ----

_hip = None


def hip() -> C.CDLL:
    """The process's HIP runtime (torch's copy when torch is loaded)."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipMemcpy.restype = C.c_int
        _hip.hipDeviceSynchronize.restype = C.c_int
        _hip.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        _hip.hipMemset.restype = C.c_int
    return _hip


def memset_d8(ptr: int, value: int, nbytes: int) -> None:
    rc = hip().hipMemset(C.c_void_p(ptr), value, nbytes)
    if rc != 0:
        raise KcmmError(f"hipMemset failed ({rc})")


def memcpy_htod(dst_ptr: int, src) -> None:
    import numpy as np
    src = np.ascontiguousarray(src)
    rc = hip().hipMemcpy(C.c_void_p(dst_ptr), src.ctypes.data_as(C.c_void_p), src.nbytes, 1)
    if rc != 0:
        raise KcmmError(f"hipMemcpy H2D failed ({rc})")


def memcpy_dtoh(src_ptr: int, nbytes: int):
    import numpy as np
    out = np.empty(nbytes, dtype=np.uint8)
    rc = hip().hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(src_ptr), nbytes, 2)
    if rc != 0:
        raise KcmmError(f"hipMemcpy D2H failed ({rc})")
    return out
