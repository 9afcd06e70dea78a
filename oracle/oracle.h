/*
 * oracle.h -- CPU restatement of the reference's decode-step data path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (lattice_amd/, libkcmm.so)
 * may link, load or call this code.  It is used by tests/ (as the checker),
 * by __graft_entry__.smoke() (as the checker) and by bench.py's cpu_baseline
 * leg (timed beside the GPU, never in place of it).
 *
 * Every function names the reference file:line it restates.  The reference
 * is Rust + CUDA and cannot be built here (no rustc/cargo, no nvcc), so there
 * is no oracle/_ref build; each function is pinned instead by the reference's
 * own unit-test constants and KATs, by closed forms, and by library routines
 * (numpy, torch dtype casts) -- see tests/test_oracle_*.py.
 */
#ifndef LATTICE_ORACLE_H
#define LATTICE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element codes: 0 f16, 1 bf16, 2 fp8-e4m3 (+ page-footer scales), 3 f32 */

/* ---- numeric formats ---- */
uint16_t oracle_f32_to_bf16(float x);
float oracle_bf16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);
uint8_t oracle_f32_to_e4m3(float x);
float oracle_e4m3_to_f32(uint8_t b);
void oracle_encode_array(int dtype, const float *src, void *dst, size_t n);
void oracle_decode_array(int dtype, const void *src, float *dst, size_t n);

/* ---- page allocator (ref superblock.rs, pool.rs:199-757) ---- */
typedef struct OPool OPool;
OPool *opool_new(size_t block_size, size_t num_layers, size_t kv_heads, size_t head_dim,
                 size_t max_batch, size_t max_seq_len, int dtype, int rollback_on_failure);
void opool_delete(OPool *p);
int opool_alloc(OPool *p, uint32_t n, uint32_t *out);
void opool_release(OPool *p, const uint32_t *ids, uint32_t n);
uint32_t opool_register(OPool *p, const uint32_t *table, uint32_t n);
void opool_unregister(OPool *p, uint32_t seq);
int opool_append_block(OPool *p, uint32_t seq, uint32_t blk);
void opool_update_seq_len(OPool *p, uint32_t seq, uint32_t len);
int opool_block_table(OPool *p, uint32_t seq, uint32_t *out, uint32_t max, uint32_t *count);
int opool_block_offset(OPool *p, uint32_t blk, uint64_t *out);
uint32_t opool_offsets_f16(OPool *p, uint64_t *out, uint32_t max);
uint32_t opool_valid_flags(OPool *p, uint8_t *out, uint32_t max);
int opool_table_offsets(OPool *p, uint32_t seq, uint64_t *out, uint32_t max, uint32_t *count);
int opool_fork(OPool *p, uint32_t src, uint32_t *out_seq);
int opool_share_prefix(OPool *p, uint32_t src, uint32_t dst, uint32_t n, uint32_t *out);
int opool_cow(OPool *p, uint32_t seq, uint32_t logical, uint32_t *src, uint32_t *dst);
uint32_t opool_refcount(OPool *p, uint32_t blk);
int opool_incref(OPool *p, uint32_t blk);
uint32_t opool_seq_len(OPool *p, uint32_t seq);
/* stats[14]: blocks_in_use, total_blocks, total_physical, free_physical,
 * active_sequences, num_layers, bps, superblocks, block_size,
 * max_blocks_per_seq, block_bytes, (float bits) idle ratio,
 * max_physical_blocks, region_bytes/2MiB */
void opool_stats(OPool *p, uint64_t *stats);
/* metrics[4] as float: ifr, pme, bu, rfi */
void opool_metrics(OPool *p, float *m);
int opool_below_low_watermark(OPool *p, float threshold);

/* ---- tiering: HBM <-> host swap (ref tiering.rs, pool.rs:824-1002, ffi.rs:1900-2008) ---- */
/* policy: 0 lru, 1 lfu, 2 fifo (anything else lru); 0 max_* = reference defaults */
int opool_enable_tiering(OPool *p, int policy, size_t max_blocks, size_t max_batch_blocks);
int opool_set_policy(OPool *p, const char *name);   /* lru lfu fifo arc sink_window */
const char *opool_policy_name(OPool *p);
int opool_location(OPool *p, uint32_t blk);          /* -1 not in use, else 0/1/3/4 */
uint64_t opool_cpu_offset(OPool *p, uint32_t blk);   /* UINT64_MAX unless swapped out */
int opool_access(OPool *p, uint32_t blk);            /* hint/protect on_access */
uint32_t opool_evict(OPool *p, uint32_t count, uint32_t *out_blocks);
int opool_restore_one(OPool *p, uint32_t blk, uint64_t *va);
int opool_restore(OPool *p, const uint32_t *ids, uint32_t n);
/* standalone policy (0 lru, 1 lfu, 2 fifo, 3 arc, 4 sink_window) and swap-slot
 * allocator; handles are (superblock, index) pairs */
typedef struct OTier OTier;
OTier *otier_new(int policy, size_t arc_cap, uint64_t swap_size, uint64_t per_block);
void otier_free(OTier *t);
void otier_event(OTier *t, int kind, uint32_t sb, uint32_t idx);  /* 0 alloc 1 access 2 evict */
size_t otier_select(OTier *t, const uint32_t *hs, size_t n, size_t count, uint32_t *out);
int otier_slot_alloc(OTier *t, uint64_t size, uint64_t *off);
void otier_slot_free(OTier *t, uint64_t off, uint64_t size);
size_t otier_ranges(OTier *t, uint64_t *out, size_t max);
size_t otier_arc_list(OTier *t, int which, uint32_t *out, size_t max);  /* 0 t1 1 t2 2 b1 3 b2 */
size_t otier_arc_p(OTier *t);

/* ---- KV write (ref pool.rs:1036-1098, ffi.rs:1088-1551, kcmm_vllm_kv_write.cu) ---- */
/* rows: destination page byte offset, slot in page, source row. */
int oracle_kv_write_rows(int dtype, uint8_t *k_region, uint8_t *v_region,
                         const uint8_t *k_src, const uint8_t *v_src,
                         const uint64_t *page_offsets, const uint32_t *slots,
                         const uint32_t *src_rows, uint32_t n, uint32_t kv_heads,
                         uint32_t head_dim, uint32_t row_bytes, uint32_t data_bytes);
int oracle_kv_write_device_slots(int dtype, uint8_t *k_region, uint8_t *v_region,
                                 const uint8_t *k_src, const uint8_t *v_src,
                                 const int64_t *slots, uint32_t batch,
                                 const uint64_t *offsets_f16, const uint8_t *valid,
                                 uint32_t offsets_len, uint32_t block_size, uint32_t kv_heads,
                                 uint32_t head_dim, uint32_t row_bytes, uint32_t data_bytes,
                                 int32_t *status);

/* ---- page copy (ref kv_gather.cu:9-43 as a page primitive) ---- */
void oracle_copy_pages(uint8_t *const *regions, uint32_t n_regions, const uint64_t *pairs,
                       uint32_t n_pairs, uint32_t block_bytes);

/* ---- paged decode attention (ref kcmm_vllm_paged_attn.cu:10-102) ---- */
/* Textbook two-pass softmax in fp64 over the decoded page contents. */
int oracle_attn_decode_f64(int dtype, const void *q, double *out, const uint8_t *k_region,
                           const uint8_t *v_region, const int32_t *block_tables,
                           const int32_t *seq_lens, const uint64_t *offsets_f16, uint32_t batch,
                           uint32_t num_q_heads, uint32_t kv_heads, uint32_t head_dim,
                           uint32_t block_size, uint32_t mbps, uint32_t row_bytes,
                           uint32_t data_bytes, double scale);
/* Causal chunked prefill over paged K/V (textbook; the reference has no
 * chunked prefill).  qsl = int32 [batch+1] query row offsets; the queries of
 * b are the last qsl[b+1]-qsl[b] of its seq_lens[b] cached tokens. */
int oracle_attn_prefill_f64(int dtype, const void *q, double *out, const uint8_t *k_region,
                            const uint8_t *v_region, const int32_t *block_tables,
                            const int32_t *seq_lens, const int32_t *qsl,
                            const uint64_t *offsets_f16, uint32_t batch, uint32_t num_q_heads,
                            uint32_t kv_heads, uint32_t head_dim, uint32_t block_size,
                            uint32_t mbps, uint32_t row_bytes, uint32_t data_bytes, double scale);
/* The reference kernel's own loop (one task per (b, q head), online softmax
 * in fp32) parallelised over tasks with OpenMP: the CPU baseline. */
int oracle_attn_decode_ref_f32(int dtype, const void *q, float *out, const uint8_t *k_region,
                               const uint8_t *v_region, const int32_t *block_tables,
                               const int32_t *seq_lens, const uint64_t *offsets_f16,
                               uint32_t batch, uint32_t num_q_heads, uint32_t kv_heads,
                               uint32_t head_dim, uint32_t block_size, uint32_t mbps,
                               uint32_t row_bytes, float scale, int threads);

/* ---- projection GEMM (intended semantics of ref runtime.rs:17-41) ---- */
/* Y[m][n] = sum_k X[m][k] W[n][k], bf16 inputs, fp64 accumulation. */
void oracle_gemm_fp8w_f64(const uint16_t *x, const uint8_t *w8, const float *s, double *y,
                          uint32_t m, uint32_t n, uint32_t k);
void oracle_gemm_bf16_f64(const uint16_t *x, const uint16_t *w, double *y, uint32_t m,
                          uint32_t n, uint32_t k);

#ifdef __cplusplus
}
#endif

#endif
