/*
 * kcmm.h -- C ABI of the KV-cache memory manager (KCMM), MI355X build.
 *
 * Every declaration below keeps the name, C types and struct layout of the
 * reference header (Vitalrubbish/Lattice include/kcmm.h), so that an existing
 * caller (ctypes, C, a Rust FFI crate) links against this libkcmm.so without
 * change.  Each entry point cites the reference declaration it replaces as
 * "ref kcmm.h:LINE" and the Rust body it re-implements as "ref ffi.rs:LINE".
 *
 * Conventions (ref kcmm.h:1-18, ffi.rs:1-20):
 *   - int-returning calls: 0 on success, -1 on failure; the message is kept
 *     per pool and read with kcmm_get_last_error().
 *   - getters return 0 on an invalid pool / index.
 *   - pointer-returning calls return NULL on failure.
 *   - every call is thread-safe; a pool handle may be shared across threads.
 *   - `uint64_t` "ptr" arguments are device virtual addresses (HIP), and
 *     `stream_ptr` is a hipStream_t (0 = the null stream).
 *
 * MI355X additions (bf16 / fp8 pools, copy-on-write fork, projection GEMM,
 * chunked prefill) live in kcmm_mi355x.h.
 */
#ifndef KCMM_H
#define KCMM_H

#ifdef __cplusplus
extern "C" {
#endif

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

/** Opaque pool handle (ref kcmm.h:36). */
typedef struct kcmm_pool_t kcmm_pool_t;

/** Eviction hints (ref kcmm.h:43-52).  With tiering on, protect-class hints
 *  record an access of the sequence's blocks (ref ffi.rs:2296-2379). */
typedef enum {
    KCMM_HINT_MULTI_TURN     = 1,
    KCMM_HINT_NEAR_END       = 2,
    KCMM_HINT_SYSTEM_PROMPT  = 3,
    KCMM_HINT_HIGH_PRIORITY  = 4,
    KCMM_HINT_LOW_PRIORITY   = 5,
    KCMM_HINT_ATTENTION_SINK = 6,
    KCMM_HINT_HEAVY_HITTER   = 7,
    KCMM_HINT_EVICTABLE      = 8,
} kcmm_hint_t;

/** Block protection levels (ref kcmm.h:55-59). */
typedef enum {
    KCMM_PROTECT_NEVER_EVICT = 0,
    KCMM_PROTECT_PREFERRED   = 1,
    KCMM_EVICT_PREFERRED     = 2,
} kcmm_protection_t;

/** Where a block's bytes live (ref kcmm.h:62-68).  With tiering on, blocks
 *  move between HBM and page-locked host memory (CPU_RESIDENT); this build
 *  has no NVMe tier, so NVME_RESIDENT is never reported. */
typedef enum {
    KCMM_LOC_GPU_RESIDENT  = 0,
    KCMM_LOC_CPU_RESIDENT  = 1,
    KCMM_LOC_NVME_RESIDENT = 2,
    KCMM_LOC_EVICTING      = 3,
    KCMM_LOC_RESTORING     = 4,
} kcmm_block_location_t;

/**
 * Pool configuration (ref kcmm.h:81-144).  Layout is part of the ABI:
 * sizeof == 376 on LP64 with max_seq_len at 336, low_watermark_threshold at
 * 344, background_evict_interval_ms at 352, attention_sink_blocks at 360 and
 * recent_window_blocks at 368 (ref ffi.rs:2576-2602).  Zero / non-positive
 * optional fields take the defaults of ref ffi.rs:476-490.
 */
typedef struct {
    size_t block_size;                /* tokens per block; default 16 */
    size_t max_blocks;                /* default 16384 (informational, as in the reference) */
    char cpu_cache_path[256];         /* unused: the swap space is page-locked host memory */
    int32_t tiering;                  /* non-zero: evict / restore between HBM and host */
    int32_t eviction_policy;          /* 0 lru, 1 lfu, 2 fifo */
    size_t prefetch_window;           /* default 4 */
    size_t max_batch_blocks;          /* default 64 */
    size_t device_ordinal;            /* HIP device ordinal; default 0 */
    size_t num_layers;                /* required */
    size_t kv_heads;                  /* required */
    size_t head_dim;                  /* required */
    size_t max_batch;                 /* required */
    size_t max_seq_len;               /* required */
    float low_watermark_threshold;    /* default 0.2 */
    uint64_t background_evict_interval_ms; /* default 100 */
    size_t attention_sink_blocks;     /* default 1 */
    size_t recent_window_blocks;      /* default 4 */
} kcmm_config_t;

/** UFS fragmentation metrics (ref kcmm.h:151-161). */
typedef struct {
    double ifr;
    double pme;
    double bu;
    double rfi;
    uint64_t gpu_blocks;
    uint64_t cpu_blocks;
    uint64_t nvme_blocks;
    uint64_t eviction_count;
    uint64_t restoration_count;
} kcmm_metrics_t;

/** Pool statistics (ref kcmm.h:164-179). */
typedef struct {
    uint32_t blocks_in_use;
    uint32_t total_blocks;
    uint32_t total_physical_blocks;
    uint32_t free_physical_blocks;
    uint32_t active_sequences;
    uint32_t num_layers;
    uint32_t blocks_per_superblock;
    uint32_t superblock_count;
    uint32_t block_size;
    uint32_t max_blocks_per_seq;
    uint32_t block_bytes;
    int32_t  tiering_enabled;
    int32_t  sharing_enabled;
    float    physical_idle_ratio;
} kcmm_pool_stats_t;

/* ---- lifecycle ---------------------------------------------------------- */

/** ref kcmm.h:193, ffi.rs:470-532.  Creates an f16 pool on the configured
 *  device: per layer one K and one V virtual-address region, backed by 2 MiB
 *  HIP VMM superblocks mapped on demand.  NULL on failure. */
kcmm_pool_t *kcmm_pool_create(const kcmm_config_t *config);

/** ref kcmm.h:203, ffi.rs:540-556.  Synchronizes the device, then unmaps and
 *  releases every superblock and VA reservation.  NULL is a no-op. */
void kcmm_pool_destroy(kcmm_pool_t *pool);

/* ---- errors ------------------------------------------------------------- */

/** ref kcmm.h:218, ffi.rs:563-579. */
size_t kcmm_get_last_error(kcmm_pool_t *pool, char *buf, size_t max_len);
/** ref kcmm.h:225, ffi.rs:584-590. */
void kcmm_clear_error(kcmm_pool_t *pool);

/* ---- block allocation --------------------------------------------------- */

/** ref kcmm.h:239, ffi.rs:605-632.  -1 on num_blocks == 0 or NULL output. */
int kcmm_alloc_blocks(kcmm_pool_t *pool, uint32_t num_blocks, uint32_t *out_blocks);
/** ref kcmm.h:249, ffi.rs:643-656.  0 even for NULL / empty input.  A block
 *  shared by a fork is released only when its last holder frees it. */
int kcmm_free_blocks(kcmm_pool_t *pool, const uint32_t *blocks, uint32_t num);

/* ---- sequences ---------------------------------------------------------- */

/** ref kcmm.h:264, ffi.rs:671-690.  Sequence indices are never reused. */
int kcmm_register_sequence(kcmm_pool_t *pool, const uint32_t *block_table,
                           uint32_t num_blocks, uint32_t *out_seq_idx);
/** ref kcmm.h:277, ffi.rs:699-709.  Out-of-range index: no-op, returns 0. */
int kcmm_unregister_sequence(kcmm_pool_t *pool, uint32_t seq_idx);
/** ref kcmm.h:288, ffi.rs:719-726. */
void kcmm_touch(kcmm_pool_t *pool, uint32_t seq_idx);
/** ref kcmm.h:299, ffi.rs:735-741. */
void kcmm_cool(kcmm_pool_t *pool, uint32_t seq_idx);
/** ref kcmm.h:308, ffi.rs:748-758. */
void kcmm_update_seq_len(kcmm_pool_t *pool, uint32_t seq_idx, uint32_t len);
/** ref kcmm.h:317, ffi.rs:767-776. */
uint32_t kcmm_get_seq_len(kcmm_pool_t *pool, uint32_t seq_idx);
/** ref kcmm.h:327, ffi.rs:785-806. */
int kcmm_append_block_to_sequence(kcmm_pool_t *pool, uint32_t seq_idx, uint32_t block_idx);
/** ref kcmm.h:340, ffi.rs:817-850. */
int kcmm_get_block_table(kcmm_pool_t *pool, uint32_t seq_idx, uint32_t *out_table,
                         uint32_t max_blocks, uint32_t *out_count);

/* ---- block queries ------------------------------------------------------ */

/** ref kcmm.h:355, ffi.rs:861-874.  Byte offset inside every layer's K and V
 *  region (the regions are allocated in lockstep); 0 if not in use. */
uint64_t kcmm_get_block_va_offset(kcmm_pool_t *pool, uint32_t block_idx);
/** ref kcmm.h:369, ffi.rs:887-911.  Entry i = byte offset of block i / 2, or
 *  0 when block i is not in use (ref pool.rs:724-737). */
int kcmm_get_all_block_offsets_f16(kcmm_pool_t *pool, uint64_t *out_offsets,
                                   uint32_t max_blocks, uint32_t *out_count);
/** ref kcmm.h:381, ffi.rs:951-974. */
int kcmm_get_block_location(kcmm_pool_t *pool, uint32_t block_idx,
                            kcmm_block_location_t *out_location);
/** ref kcmm.h:394, ffi.rs:983-1020. */
int kcmm_get_block_table_va_offsets(kcmm_pool_t *pool, uint32_t seq_idx,
                                    uint64_t *out_offsets, uint32_t max_blocks,
                                    uint32_t *out_count);

/* ---- region bases ------------------------------------------------------- */

/** ref kcmm.h:409, ffi.rs:1029-1042. */
uint64_t kcmm_get_va_k(kcmm_pool_t *pool, uint32_t layer);
/** ref kcmm.h:418, ffi.rs:1051-1064. */
uint64_t kcmm_get_va_v(kcmm_pool_t *pool, uint32_t layer);

/* ---- KV write (reshape-and-cache) -------------------------------------- */

/** ref kcmm.h:438, ffi.rs:1088-1200.  Row b of k/v_src ([batch][kv_heads *
 *  head_dim] elements of the pool dtype) is written at token `positions[b]`
 *  of sequence `seq_indices[b]`, on the null stream.  All rows are validated
 *  before anything is enqueued; one HIP kernel moves every row. */
int kcmm_append_kv_step(kcmm_pool_t *pool, uint32_t layer_idx,
                        const uint32_t *seq_indices, const uint32_t *positions,
                        uint32_t batch, uint64_t k_src_ptr, uint64_t v_src_ptr);

/** ref kcmm.h:459, ffi.rs:1217-1240.  Host slot ids: slot = block*block_size +
 *  offset; negative slots are padding.  Null stream. */
int kcmm_append_kv_slots(kcmm_pool_t *pool, uint32_t layer_idx,
                         const int64_t *slot_mapping, uint32_t batch,
                         uint64_t k_src_ptr, uint64_t v_src_ptr);

/** ref kcmm.h:475, ffi.rs:1249-1383.  As above on `stream_ptr`; returns
 *  without synchronizing. */
int kcmm_append_kv_slots_on_stream(kcmm_pool_t *pool, uint32_t layer_idx,
                                   const int64_t *slot_mapping, uint32_t batch,
                                   uint64_t k_src_ptr, uint64_t v_src_ptr,
                                   uint64_t stream_ptr);

/** Exported by the reference without a header entry (ref ffi.rs:1399-1551,
 *  kernel ref kcmm_vllm_kv_write.cu:8-66).  Device-resident int64 slots; the
 *  int32 word at status_ptr (if non-zero) is set once, first error wins:
 *  1 = block id >= block_offsets_f16_len, 2 = valid_blocks[id] == 0. */
int kcmm_append_kv_device_slots_on_stream(kcmm_pool_t *pool, uint32_t layer_idx,
                                          uint64_t slot_mapping_ptr,
                                          uint64_t block_offsets_f16_ptr,
                                          uint64_t valid_blocks_ptr,
                                          uint32_t block_offsets_f16_len,
                                          uint32_t batch, uint64_t k_src_ptr,
                                          uint64_t v_src_ptr, uint64_t status_ptr,
                                          uint64_t stream_ptr);

/** Exported without a header entry (ref ffi.rs:210).  Kernels are compiled
 *  ahead of time for gfx950, so this only validates the pool. */
int kcmm_precompile_vllm_kv_write_f16(kcmm_pool_t *pool);

/* ---- paged decode attention -------------------------------------------- */

/** ref kcmm.h:505, ffi.rs:1569-1609 (kernel ref kcmm_vllm_paged_attn.cu:10-102).
 *  q/out f16 [batch][num_q_heads][head_dim] (contiguous), block_tables int32
 *  [batch][max_blocks_per_seq], seq_lens int32 [batch], block_offsets_f16
 *  u64 [n_block_ids].  out[b][h] = softmax(scale * q.K^T) V over the first
 *  seq_lens[b] tokens of sequence b, kv head = h * kv_heads / num_q_heads;
 *  seq_lens[b] <= 0 writes zeros.  Synchronizes before returning. */
int kcmm_paged_attn_decode_f16(kcmm_pool_t *pool, uint32_t layer_idx,
                               uint64_t query_ptr, uint64_t out_ptr,
                               uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
                               uint64_t block_offsets_f16_ptr,
                               uint32_t batch, uint32_t num_q_heads,
                               uint32_t kv_heads, uint32_t head_dim,
                               uint32_t block_size, uint32_t max_blocks_per_seq,
                               float scale);

/** ref kcmm.h:525, ffi.rs:1618-1661.  Enqueue on stream_ptr, no sync. */
int kcmm_paged_attn_decode_f16_on_stream(
    kcmm_pool_t *pool, uint32_t layer_idx, uint64_t query_ptr, uint64_t out_ptr,
    uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
    uint64_t block_offsets_f16_ptr, uint32_t batch, uint32_t num_q_heads,
    uint32_t kv_heads, uint32_t head_dim, uint32_t block_size,
    uint32_t max_blocks_per_seq, float scale, uint64_t stream_ptr);

/** ref kcmm.h:544, ffi.rs:1670-1713.  As _on_stream without making the
 *  pool's device current first. */
int kcmm_paged_attn_decode_f16_on_current_context_stream(
    kcmm_pool_t *pool, uint32_t layer_idx, uint64_t query_ptr, uint64_t out_ptr,
    uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
    uint64_t block_offsets_f16_ptr, uint32_t batch, uint32_t num_q_heads,
    uint32_t kv_heads, uint32_t head_dim, uint32_t block_size,
    uint32_t max_blocks_per_seq, float scale, uint64_t stream_ptr);

/** ref kcmm.h:559, ffi.rs:182-205.  Idempotent; validates the pool. */
int kcmm_precompile_paged_attn_decode_f16(kcmm_pool_t *pool);

/* ---- tiering (ref kcmm.h:577-613): HBM <-> page-locked host memory ------ */

/** ref kcmm.h:577, ffi.rs:1900-1945.  Moves up to `count` policy-chosen
 *  blocks to host swap slots; returns how many moved (0 with tiering off).
 *  Synchronous. */
uint32_t kcmm_evict_blocks(kcmm_pool_t *pool, uint32_t count);
/** ref kcmm.h:590, ffi.rs:1954-1972.  Brings a swapped-out block back to a
 *  new page; returns its VA offset (a resident block: its offset; 0 on
 *  error).  Synchronous. */
uint64_t kcmm_restore_evicted_block(kcmm_pool_t *pool, uint32_t block_idx);
/** ref kcmm.h:603, ffi.rs:1984-2002.  Restores every swapped-out block of the
 *  list (each once); 0 on success, -1 if any failed.  Synchronous. */
int kcmm_restore_evicted_blocks(kcmm_pool_t *pool, const uint32_t *block_indices,
                                uint32_t count);
/** ref kcmm.h:613, ffi.rs:2011-2025. */
int kcmm_is_gpu_resident(kcmm_pool_t *pool, uint32_t block_idx);

/* ---- metrics ------------------------------------------------------------ */

/** ref kcmm.h:626, ffi.rs:2037-2070 (formulas ref pool.rs:1179-1240). */
int kcmm_get_metrics(kcmm_pool_t *pool, kcmm_metrics_t *out);
/** ref kcmm.h:635, ffi.rs:2079-2107. */
int kcmm_get_pool_stats(kcmm_pool_t *pool, kcmm_pool_stats_t *out);
/** ref kcmm.h:638, ffi.rs:2116. */
uint32_t kcmm_blocks_in_use(kcmm_pool_t *pool);
/** ref kcmm.h:641, ffi.rs:2128. */
uint32_t kcmm_total_blocks(kcmm_pool_t *pool);
/** Exported without a header entry (ref ffi.rs:2143): bumps whenever a block's
 *  in-use state or mapping changes. */
uint64_t kcmm_block_state_epoch(kcmm_pool_t *pool);
/** ref kcmm.h:644, ffi.rs:2155. */
uint32_t kcmm_free_physical_blocks(kcmm_pool_t *pool);
/** ref kcmm.h:647, ffi.rs:2169. */
int kcmm_has_free_blocks(kcmm_pool_t *pool);
/** ref kcmm.h:650, ffi.rs:2181. */
uint32_t kcmm_active_sequences(kcmm_pool_t *pool);
/** Exported without a header entry (ref ffi.rs:920-941). */
int kcmm_get_all_block_valid(kcmm_pool_t *pool, uint8_t *out_valid,
                             uint32_t max_blocks, uint32_t *out_count);

/* ---- policy / hints (tiering-dependent) --------------------------------- */

/** ref kcmm.h:664, ffi.rs:2200-2234.  lru, lfu, fifo, arc or sink_window;
 *  -1 when tiering is disabled or the name is unknown. */
int kcmm_set_eviction_policy(kcmm_pool_t *pool, const char *policy);
/** ref kcmm.h:674, ffi.rs:2243-2259.  Name length; 0 when tiering is disabled. */
uint32_t kcmm_get_eviction_policy(kcmm_pool_t *pool, char *out_policy, uint32_t max_len);
/** ref kcmm.h:683, ffi.rs:2268. */
int kcmm_is_tiering_enabled(kcmm_pool_t *pool);
/** ref kcmm.h:704, ffi.rs:2296-2379. */
int kcmm_hint(kcmm_pool_t *pool, uint32_t seq_idx, kcmm_hint_t hint);
/** ref kcmm.h:722, ffi.rs:2388-2442. */
int kcmm_protect(kcmm_pool_t *pool, uint32_t seq_idx, const uint32_t *block_ids,
                 uint32_t num_blocks, kcmm_protection_t level);

/* ---- prefix sharing ----------------------------------------------------- */

/** ref kcmm.h:744, ffi.rs:2451-2481 (a placeholder there).  Here it is real:
 *  the first num_blocks entries of src_seq's table are appended to dst_seq's
 *  table, each shared block's reference count is incremented, and the ids are
 *  written to out_blocks.  -1 if either sequence is unknown or src_seq holds
 *  fewer than num_blocks blocks. */
int kcmm_share_prefix(kcmm_pool_t *pool, uint32_t src_seq, uint32_t dst_seq,
                      uint32_t num_blocks, uint32_t *out_blocks);

/* ---- utilities ---------------------------------------------------------- */

/** ref kcmm.h:761, ffi.rs:2488-2498. */
int kcmm_below_low_watermark(kcmm_pool_t *pool, float threshold);
/** ref kcmm.h:771, ffi.rs:2547-2560.  Synchronizes the pool's device. */
int kcmm_synchronize(kcmm_pool_t *pool);

/** ref kcmm.h:778-793, ffi.rs:2505-2538. */
uint32_t kcmm_get_block_size(kcmm_pool_t *pool);
uint32_t kcmm_get_max_blocks_per_seq(kcmm_pool_t *pool);
uint32_t kcmm_get_block_bytes(kcmm_pool_t *pool);
uint32_t kcmm_get_num_layers(kcmm_pool_t *pool);
uint32_t kcmm_get_max_batch(kcmm_pool_t *pool);
uint32_t kcmm_get_max_seq_len(kcmm_pool_t *pool);

#ifdef __cplusplus
}
#endif

#endif /* KCMM_H */
