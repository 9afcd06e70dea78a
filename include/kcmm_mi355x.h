/*
 * kcmm_mi355x.h -- MI355X additions to the KCMM C ABI.
 *
 * The reference ships an f16-only cache (ref pool.rs:203-204), a placeholder
 * prefix-sharing manager (ref sharing.rs:24-65) and runs its projections
 * through cuBLAS (ref runtime.rs:17-41).  The entry points below add what the
 * decode-step data path needs on MI355X, next to the reference ABI in
 * kcmm.h and with the same conventions (0 / -1, per-pool error text,
 * device addresses as uint64_t, stream_ptr = hipStream_t).
 */
#ifndef KCMM_MI355X_H
#define KCMM_MI355X_H

#include "kcmm.h"

#ifdef __cplusplus
extern "C" {
#endif

/** Element type of a pool's K/V pages. */
typedef enum {
    KCMM_KV_F16 = 0,       /* IEEE half (the reference's only type) */
    KCMM_KV_BF16 = 1,      /* bfloat16 */
    KCMM_KV_FP8_E4M3 = 2,  /* OCP e4m3fn + one fp32 scale per (page, kv head) */
    KCMM_KV_F32 = 3,       /* IEEE single */
} kcmm_kv_dtype_t;

/**
 * Create a pool whose pages hold `kv_dtype` elements.  Page layout in every
 * layer's K and V region: [block_size][kv_heads][head_dim] elements, token
 * major, exactly as the reference (ref pool.rs:1036-1098).  fp8 pages add a
 * footer of kv_heads fp32 scales at byte bs*kv_heads*head_dim and are padded
 * to a multiple of 256 bytes, so a page copy moves its scales with it.
 * Extends kcmm_pool_create (ref kcmm.h:193), which is the KCMM_KV_F16 case.
 *
 * fp8 page writes (every KV append on an fp8 pool) take bf16 rows.  The rows
 * one call writes into a page are applied as one set -- for each token slot
 * the call's last row for it -- so the bytes do not depend on row order.
 * Per (page, kv head), with amax = max |x| over the rows written:
 *   - a call that writes slot 0, or that finds a footer scale that is not a
 *     finite positive number, starts the page: scale = amax / 448 (1 if 0);
 *     the page's other slots are undefined afterwards;
 *   - any other call keeps the scale, or raises it to amax / 448 when
 *     amax > 448 * scale and then re-encodes every slot it does not write;
 * each written element is e4m3(x / scale), round to nearest even, so no
 * value is clipped.  A page must therefore be started by a write of slot 0.
 * Limits: block_size <= 4096 and head_dim <= 256; a host-slot call writes at
 * most 64 distinct slots of one page.
 */
kcmm_pool_t *kcmm_pool_create_typed(const kcmm_config_t *config, int32_t kv_dtype);

/** Pool element type (kcmm_kv_dtype_t), or -1 for NULL. */
int32_t kcmm_get_kv_dtype(kcmm_pool_t *pool);

/** 1 = one hipMalloc per region holding the full capacity (the only backing
 *  this build creates), -1 for NULL.  Value 0 is reserved for HIP VMM 2 MiB
 *  superblocks mapped on demand (the reference design, ref cuda_vmm.rs);
 *  KCMM_BACKING=vmm makes kcmm_pool_create* fail, because that backing is
 *  disabled (unexplained hipMemSetAccess failures after repeated pool
 *  create/destroy in one process).  Block ids and offsets do not depend on
 *  the backing. */
int32_t kcmm_get_backing_kind(kcmm_pool_t *pool);

/** Why the last kcmm_pool_create* on this thread returned NULL (the reference
 *  has no channel for this, ref ffi.rs:500-531). */
size_t kcmm_last_create_error(char *buf, size_t max_len);

/* ---- decode attention for bf16 / fp8 pools ------------------------------ */

/** Same tensor contract as kcmm_paged_attn_decode_f16 (ref kcmm.h:505) with
 *  bf16 q/out and a bf16 pool.  Synchronizes before returning. */
int kcmm_paged_attn_decode_bf16(kcmm_pool_t *pool, uint32_t layer_idx,
                                uint64_t query_ptr, uint64_t out_ptr,
                                uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
                                uint64_t block_offsets_f16_ptr,
                                uint32_t batch, uint32_t num_q_heads,
                                uint32_t kv_heads, uint32_t head_dim,
                                uint32_t block_size, uint32_t max_blocks_per_seq,
                                float scale);

/** As kcmm_paged_attn_decode_f16_on_stream (ref kcmm.h:525) for bf16. */
int kcmm_paged_attn_decode_bf16_on_stream(
    kcmm_pool_t *pool, uint32_t layer_idx, uint64_t query_ptr, uint64_t out_ptr,
    uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
    uint64_t block_offsets_f16_ptr, uint32_t batch, uint32_t num_q_heads,
    uint32_t kv_heads, uint32_t head_dim, uint32_t block_size,
    uint32_t max_blocks_per_seq, float scale, uint64_t stream_ptr);

/** fp8-e4m3 pool: bf16 q/out; K/V are dequantized in registers with the
 *  page-footer scale of their (page, kv head).  Enqueue only. */
int kcmm_paged_attn_decode_fp8_on_stream(
    kcmm_pool_t *pool, uint32_t layer_idx, uint64_t query_ptr, uint64_t out_ptr,
    uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
    uint64_t block_offsets_f16_ptr, uint32_t batch, uint32_t num_q_heads,
    uint32_t kv_heads, uint32_t head_dim, uint32_t block_size,
    uint32_t max_blocks_per_seq, float scale, uint64_t stream_ptr);

/**
 * kcmm_paged_attn_decode_bf16_on_stream without any device allocation: the
 * kernels' scratch (partial results, segment table) is a static 24 MiB device
 * array in the library instead of a per-stream workspace.  No counterpart in
 * the reference: for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  A batch
 * whose scratch would exceed 24 MiB is refused (-1, error text names the
 * sizes); at the Llama-3-8B decode shape (32/8 heads, head_dim 128) that is
 * about 300 sequences.  Every call on a GPU shares that GPU's array, so
 * calls take turns with it: a call on a different stream from the previous
 * call on that GPU first waits (hipStreamWaitEvent on one event per GPU,
 * created with the array's address on the first call) for that call's
 * kernels, and the array keeps the last call's contents.  Under HIP graph
 * capture no event is recorded or waited on: a graph that holds two such
 * calls on parallel branches must order them itself.  Enqueue only.
 */
int kcmm_paged_attn_decode_bf16_noalloc_on_stream(
    kcmm_pool_t *pool, uint32_t layer_idx, uint64_t query_ptr, uint64_t out_ptr,
    uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
    uint64_t block_offsets_f16_ptr, uint32_t batch, uint32_t num_q_heads,
    uint32_t kv_heads, uint32_t head_dim, uint32_t block_size,
    uint32_t max_blocks_per_seq, float scale, uint64_t stream_ptr);

/** Measurement: HIP-event timing of the decode-attention streaming kernel
 *  alone (the kernel that reads the KV pages; the attention call also runs
 *  a log-sum-exp merge after it).  start creates max_calls (1..65536) event
 *  pairs on the current device; each streaming-kernel launch on that device
 *  after it, by any decode-attention entry point and not under graph
 *  capture, is bracketed by the next free pair.  stop waits for the
 *  recorded pairs, writes their average duration in microseconds and their
 *  number, and frees the events.  Call stop after the timed calls have
 *  returned; not for concurrent use from several threads.  Off by default
 *  (a launch then only reads one atomic flag).  No counterpart in the
 *  reference (it has no per-kernel timing); for bench.py's roofline of the
 *  dominant kernel.  0 on success, -1 on error (stop without start, bad
 *  arguments, an event query that failed). */
int kcmm_attn_stream_timing_start(uint32_t max_calls);
int kcmm_attn_stream_timing_stop(double *avg_us, uint32_t *count);

/** Reads the KCMM_* tuning variables (KCMM_ATTN_*, KCMM_GEMM_*) again.  The
 *  library reads them once, on first use, so that launch paths make no
 *  getenv call; tests and tuning runs that change them call this after the
 *  change.  Not to be called while other threads launch.  No counterpart
 *  in the reference. */
void kcmm_reload_tunables(void);

/** fp32 pool: fp32 q/out, same tensor contract as
 *  kcmm_paged_attn_decode_f16 (ref kcmm.h:505).  Synchronizes before
 *  returning. */
int kcmm_paged_attn_decode_f32(kcmm_pool_t *pool, uint32_t layer_idx,
                               uint64_t query_ptr, uint64_t out_ptr,
                               uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
                               uint64_t block_offsets_f16_ptr,
                               uint32_t batch, uint32_t num_q_heads,
                               uint32_t kv_heads, uint32_t head_dim,
                               uint32_t block_size, uint32_t max_blocks_per_seq,
                               float scale);

/** As kcmm_paged_attn_decode_f16_on_stream (ref kcmm.h:525) for fp32 pools.
 *  Enqueue only. */
int kcmm_paged_attn_decode_f32_on_stream(
    kcmm_pool_t *pool, uint32_t layer_idx, uint64_t query_ptr, uint64_t out_ptr,
    uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
    uint64_t block_offsets_f16_ptr, uint32_t batch, uint32_t num_q_heads,
    uint32_t kv_heads, uint32_t head_dim, uint32_t block_size,
    uint32_t max_blocks_per_seq, float scale, uint64_t stream_ptr);

/* ---- chunked prefill attention ----------------------------------------- */

/**
 * Causal chunked-prefill attention over the pool's pages (the reference
 * prefills one token per decode step, ref transformer.rs:50-65; this is the
 * varlen-with-paged-KV form of vLLM's chunked prefill).  Sequence b holds
 * seq_lens[b] cached tokens, the last (query_start_loc[b+1] -
 * query_start_loc[b]) of which are this chunk's queries, already appended.
 * Query i of b (row query_start_loc[b] + i of q/out, [rows][Hq][D]) is at
 * position seq_lens[b] - len_b + i and attends to keys 0..position.  q/out
 * are f16 for f16 pools and bf16 otherwise; seq_lens and query_start_loc are
 * device int32 arrays; rows without a valid position are written as zeros.
 * fp32 pools take fp32 q/out.
 * Enqueue only.
 */
int kcmm_paged_attn_prefill_on_stream(
    kcmm_pool_t *pool, uint32_t layer_idx, uint64_t query_ptr, uint64_t out_ptr,
    uint64_t block_tables_ptr, uint64_t seq_lens_ptr, uint64_t query_start_loc_ptr,
    uint64_t block_offsets_f16_ptr, uint32_t batch, uint32_t total_query_tokens,
    uint32_t num_q_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t block_size,
    uint32_t max_blocks_per_seq, float scale, uint64_t stream_ptr);

/* ---- copy-on-write fork ------------------------------------------------- */

/** Fork `src_seq` (beam search): a new sequence holding the same block ids
 *  and seq_len; every shared block's reference count is incremented.  The
 *  reference has only a placeholder (ref sharing.rs:24-65); semantics follow
 *  the vLLM fork it mirrors (ref patch_vllm.py:1092-1101,
 *  shadow_allocator.py:63-73). */
int kcmm_fork_sequence(kcmm_pool_t *pool, uint32_t src_seq, uint32_t *out_seq);

/** Reference count of a block (0 if not in use). */
uint32_t kcmm_get_block_refcount(kcmm_pool_t *pool, uint32_t block_idx);

/**
 * Make logical block `logical_block` of `seq_idx` private before an append
 * (ref patch_vllm.py:1083-1090, shadow_allocator.py:94-118).  Returns 1 when
 * the block was shared: a fresh block is allocated, the sequence's table is
 * repointed to it, the old block's count drops by one and (*out_src,
 * *out_dst) name the page copy the caller must enqueue with
 * kcmm_copy_blocks_on_stream.  Returns 0 when the block is already private
 * (nothing to copy), -1 on error.
 */
int kcmm_cow_block_for_append(kcmm_pool_t *pool, uint32_t seq_idx,
                              uint32_t logical_block, uint32_t *out_src,
                              uint32_t *out_dst);

/** Copy whole pages src->dst for every layer's K and V region (and fp8
 *  scale footers), one HIP kernel launch per 192 pairs.  `src_dst` is a host array of
 *  num_pairs (src, dst) block ids; both ids must be in use.  Enqueue only. */
int kcmm_copy_blocks_on_stream(kcmm_pool_t *pool, const uint32_t *src_dst,
                               uint32_t num_pairs, uint64_t stream_ptr);

/** Beam-search fork of one decode step in one call (the vLLM block manager's
 *  fork + copy-on-write + copy_blocks, patch_vllm.py:1083-1101; ref
 *  sharing.rs:24-65 leaves it a placeholder).  Each parents[i] gets
 *  beam_width - 1 children (written to children_out, parent-major) that
 *  share its pages; each child's page for its next token (logical block
 *  seq_len / block_size, when already allocated) is made private as
 *  kcmm_cow_block_for_append does, in the same order as the separate calls
 *  (fork child, CoW child, next child), and all the page copies (every
 *  layer's K and V) are enqueued on stream_ptr (one kernel launch per 192
 *  pages).  The parent keeps the original page, private again once its
 *  children have copied.  The children share the parent's table up to that
 *  page instead of copying it, so the call costs O(children) on the host,
 *  not O(table length); refcounts reported afterwards are exact.
 *  Returns the number of pages copied, or -1. */
int kcmm_fork_beams_on_stream(kcmm_pool_t *pool, const uint32_t *parents, uint32_t n_parents,
                              uint32_t beam_width, uint32_t *children_out,
                              uint64_t stream_ptr);

/** Device-side variant (vLLM copy_blocks contract): `pairs_ptr` is a device
 *  int64 [num_pairs][2] array of block ids, translated through the device
 *  f16-unit offset table (which must cover every id the pool has issued).
 *  A pair with an id outside [0, ids issued at enqueue time) is skipped.
 *  Enqueue only; apart from that id count no host state is read. */
int kcmm_copy_blocks_device_on_stream(kcmm_pool_t *pool, uint64_t pairs_ptr,
                                      uint64_t block_offsets_f16_ptr,
                                      uint32_t num_pairs, uint64_t stream_ptr);

/* ---- prefix cache ------------------------------------------------------- */

/* The reference's prefix-sharing manager (src/kcmm/sharing.rs:9-65: content
 * hash -> the blocks of a prefix, reference counted for sharing; a
 * placeholder there) over the copy-on-write pages above.  Keys are chained
 * content hashes of full blocks; every cache entry holds one reference on its
 * block, so a cached prefix outlives the sequence that registered it and a
 * later request with the same tokens attaches the same pages instead of
 * recomputing them.  Cached blocks are full and shared: writes into them are
 * refused like writes into any shared block. */

/** Chained content hashes of the full blocks of tokens[0..n_tokens): hash i
 *  = FNV-1a-64 over the 8 little-endian bytes of hash i-1 (seed for i = 0)
 *  followed by the 4 little-endian bytes of each of the block's block_size
 *  token ids.  Writes min(n_tokens / block_size, max_hashes) hashes to
 *  out_hashes and their count to *count.  Host-only.  -1 on null pointers or
 *  block_size 0. */
int kcmm_prefix_hash_blocks(const int32_t *tokens, uint32_t n_tokens, uint32_t block_size,
                            uint64_t seed, uint64_t *out_hashes, uint32_t max_hashes,
                            uint32_t *count);

/** Cache the first num_blocks blocks of seq_idx's table under
 *  hashes[0..num_blocks).  Only full blocks: num_blocks * block_size must not
 *  exceed the sequence's seq_len.  A key already cached is left as it is (the
 *  first registration wins); each new entry takes one reference on its block.
 *  *out_added = entries created.  -1 on an unknown sequence, too many blocks,
 *  a partial block or a block not in use (nothing cached then). */
int kcmm_prefix_register(kcmm_pool_t *pool, uint32_t seq_idx, const uint64_t *hashes,
                         uint32_t num_blocks, uint32_t *out_added);

/** The longest cached run hashes[0..m): block ids to out_blocks[0..m)
 *  (out_blocks may be NULL), m to *out_matched.  Marks the run as used now
 *  (eviction order).  No reference changes. */
int kcmm_prefix_match(kcmm_pool_t *pool, const uint64_t *hashes, uint32_t num_blocks,
                      uint32_t *out_blocks, uint32_t *out_matched);

/** kcmm_prefix_match, then append the m matched blocks to dst_seq's table
 *  with one reference each (as kcmm_share_prefix).  out_blocks may be NULL.
 *  The caller sets dst_seq's seq_len; blocks swapped out to host memory must
 *  be restored before attention reads them. */
int kcmm_prefix_attach(kcmm_pool_t *pool, uint32_t dst_seq, const uint64_t *hashes,
                       uint32_t num_blocks, uint32_t *out_blocks, uint32_t *out_matched);

/** Drop up to max_entries cache entries, least recently used first (the
 *  deepest first among entries registered or matched together), releasing
 *  each entry's reference (a block no sequence holds is freed).
 *  UINT32_MAX drops every entry.  *out_evicted = entries dropped. */
int kcmm_prefix_evict(kcmm_pool_t *pool, uint32_t max_entries, uint32_t *out_evicted);

/** Number of cache entries (0 for NULL). */
uint32_t kcmm_prefix_cached_blocks(kcmm_pool_t *pool);

/* ---- projection GEMM ---------------------------------------------------- */

/** Y[m][n] = X[m][k] * W[n][k]^T (row major, the HF Linear layout used by
 *  ref llama_transformer.rs:115-120), bf16 inputs and output, fp32
 *  accumulation on MFMA.  Replaces the cuBLAS call of ref runtime.rs:17-41
 *  (whose column-major arguments equal this product only at m == 1).
 *  m <= 128 runs the weight-stream MFMA kernel (weights streamed into
 *  registers); m > 128 the LDS-tiled MFMA kernel (same product, fp32
 *  accumulation, not the same bits; KCMM_GEMM_TILED=0 keeps the
 *  weight-stream kernel).  Enqueue only; requires k % 256 == 0 and
 *  n % 64 == 0. */
int kcmm_gemm_bf16_on_stream(uint64_t x_ptr, uint64_t w_ptr, uint64_t y_ptr,
                             uint32_t m, uint32_t n, uint32_t k,
                             uint64_t stream_ptr);

/** How kcmm_gemm_bf16_on_stream (fp8_weights = 0) or
 *  kcmm_gemm_fp8w_bf16_on_stream (fp8_weights = 1) runs a product of this
 *  shape under the current KCMM_GEMM_* settings, written to out[4]: kernel
 *  (0 weight-stream, 1 LDS-tiled), K splits, tiling of the tiled kernel (-1
 *  otherwise), bytes of fp32 split partials written and read back by the
 *  reduction (0 without a split).  No reference counterpart (the reference's
 *  cuBLAS call, runtime.rs:17-41, exposes no plan); for sizing workspaces and
 *  for counting a product's HBM bytes.  Host-only, no device work.  0 on
 *  success, -1 on a shape the kernels do not take. */
int kcmm_gemm_plan(uint32_t m, uint32_t n, uint32_t k, uint32_t fp8_weights, int64_t* out);

/** Y[m][n] = X[m][k] * (W8[n][k] * wscale[n])^T with fp8-e4m3 (OCP e4m3fn)
 *  weights W8 and one fp32 scale per weight row: the projection with
 *  weight-only fp8 quantization (half the weight bytes a decode step
 *  streams).  bf16 activations and output, fp32 accumulation on bf16 MFMA
 *  (the weights are converted to bf16 exactly in registers; the row scale
 *  multiplies the accumulated dot product).  m <= 128 runs the
 *  weight-stream kernel, m > 128 the LDS-tiled kernel (codes staged in LDS,
 *  converted as they are read; KCMM_GEMM_TILED=0 keeps the weight-stream
 *  kernel).  Enqueue only; k % 256 == 0, n % 64 == 0. */
int kcmm_gemm_fp8w_bf16_on_stream(uint64_t x_ptr, uint64_t w8_ptr, uint64_t wscale_ptr,
                                  uint64_t y_ptr, uint32_t m, uint32_t n, uint32_t k,
                                  uint64_t stream_ptr);

/** Y = R + X * W^T: the O / down projections with the residual add of ref
 *  llama_transformer.rs:358-360,377-379 (add.cu) in the GEMM's store.  The product
 *  is rounded to bf16 before the add, as a bf16 model computes it; R may be
 *  the same buffer as Y.  Same shape rules as kcmm_gemm_bf16_on_stream. */
int kcmm_gemm_bf16_add_on_stream(uint64_t x_ptr, uint64_t w_ptr, uint64_t residual_ptr,
                                 uint64_t y_ptr, uint32_t m, uint32_t n, uint32_t k,
                                 uint64_t stream_ptr);

/* ---- decode-step glue and the layer step -------------------------------- */
/* The steps of one decoder layer around the GEMMs and the attention (ref
 * LlamaTransformer::forward_step_paged, llama_transformer.rs:262-391, and
 * its rms_norm.cu / rope.cu / silu_mul.cu / add.cu), with Hugging Face Llama
 * semantics.  bf16 activations, fp32 arithmetic, enqueue only; pointers are
 * device addresses aligned to 16 bytes. */

/** The O projection with its residual add and the post-attention RMSNorm
 *  (ref llama_transformer.rs:356-362: o GEMM, add.cu, rms_norm.cu):
 *  hidden = bf16(hidden + bf16(x * w^T)) in place ([m][n]), then normed =
 *  rmsnorm(hidden) with weight norm_w.  Bit-identical to
 *  kcmm_gemm_bf16_add_on_stream followed by kcmm_rmsnorm_bf16_on_stream; the
 *  split-K partial sums are finished inside the RMSNorm kernel.  n % 64 ==
 *  0, k % 256 == 0. */
int kcmm_gemm_bf16_add_rmsnorm_on_stream(uint64_t x_ptr, uint64_t w_ptr, uint64_t hidden_ptr,
                                         uint64_t norm_w_ptr, uint64_t normed_ptr, uint32_t m,
                                         uint32_t n, uint32_t k, float eps,
                                         uint64_t stream_ptr);

/** y[r] = w * bf16(x[r] * rsqrt(mean(x[r]^2) + eps)) for each of `rows` rows
 *  of `hidden` elements (HF LlamaRMSNorm).  hidden % 8 == 0. */
int kcmm_rmsnorm_bf16_on_stream(uint64_t x_ptr, uint64_t w_ptr, uint64_t y_ptr,
                                uint32_t rows, uint32_t hidden, float eps,
                                uint64_t stream_ptr);

/** Token embedding of a decode step (ref llama_transformer.rs:264-275, one
 *  device copy per token there): hidden[b][:] = embed[token_ids[b]][:] for
 *  b < batch, bf16 rows of hidden_size (% 8 == 0) elements; token_ids is a
 *  device int32 array (e.g. the previous step's sampled tokens); an id
 *  outside [0, vocab) gives a zero row.  Enqueue only. */
int kcmm_embed_tokens_bf16_on_stream(uint64_t embed_ptr, uint64_t token_ids_ptr,
                                     uint64_t hidden_ptr, uint32_t batch, uint32_t hidden_size,
                                     uint32_t vocab, uint64_t stream_ptr);

/** act[r][j] = bf16(bf16(silu(g)) * u) with g = gate_up[r][j] and
 *  u = gate_up[r][intermediate + j] (the fused [gate | up] projection
 *  output; F.silu on a bf16 tensor rounds before the multiply).
 *  intermediate % 8 == 0. */
int kcmm_silu_mul_bf16_on_stream(uint64_t gate_up_ptr, uint64_t act_ptr, uint32_t rows,
                                 uint32_t intermediate, uint64_t stream_ptr);

/** The gate/up projection with SwiGLU in its store (ref
 *  llama_transformer.rs:370-375: gate and up GEMMs, silu_mul.cu): act[m][j]
 *  = bf16(bf16(silu(G)) * U) with G, U the bf16-rounded projections
 *  x * w[j]^T and x * w[intermediate + j]^T; w_gate_up = [gate rows; up
 *  rows], [2 intermediate][k].  Bit-identical to kcmm_gemm_bf16_on_stream
 *  (on the weight-stream kernel: m <= 128 or KCMM_GEMM_TILED=0)
 *  followed by kcmm_silu_mul_bf16_on_stream, without the [m][2 intermediate]
 *  intermediate.  intermediate % 32 == 0, k % 256 == 0. */
int kcmm_gemm_bf16_swiglu_on_stream(uint64_t x_ptr, uint64_t w_gate_up_ptr, uint64_t act_ptr,
                                    uint32_t m, uint32_t intermediate, uint32_t k,
                                    uint64_t stream_ptr);

/** RoPE fused with the KV append for the decode token of every sequence of a
 *  bf16 or fp8 pool (bf16 activations; on an fp8 pool the rotated k and the
 *  v rows go through the fp8 page writer of kcmm_append_kv_device_slots,
 *  scales included): row b of qkv_ptr holds [q heads | k heads | v heads] x
 *  head_dim; the token's position is seq_lens[b] - 1 (seq_lens include it).
 *  q is rotated into q_out_ptr ([batch][num_q_heads][head_dim], the layout
 *  the attention reads); k is rotated and written, with v, into the token's
 *  page row (the vLLM reshape_and_cache slot block_tables[b][pos / bs] * bs
 *  + pos % bs).  Rotation: HF rotate_half pairs (i, i + head_dim/2) at angle
 *  pos * inv_freq[i], inv_freq an fp32 device array of head_dim/2 (so any
 *  HF rope_type works).  Sequences with seq_lens <= 0 or a position past
 *  the table are skipped.  The caller makes shared pages private first. */
int kcmm_rope_append_bf16_on_stream(kcmm_pool_t *pool, uint32_t layer_idx, uint64_t qkv_ptr,
                                    uint64_t q_out_ptr, uint64_t block_tables_ptr,
                                    uint64_t seq_lens_ptr, uint64_t block_offsets_f16_ptr,
                                    uint64_t inv_freq_ptr, uint32_t batch,
                                    uint32_t num_q_heads, uint32_t max_blocks_per_seq,
                                    uint64_t stream_ptr);

/** The QKV projection of a decode step with RoPE and the KV append in its
 *  store (ref llama_transformer.rs:315-333: q/k/v GEMMs, rope.cu, the cache
 *  write): x_ptr [batch][hidden] times w_qkv_ptr [(Hq + 2 Hkv) head_dim]
 *  [hidden] (q rows, k rows, v rows), each product rounded to bf16 and then
 *  treated exactly as kcmm_rope_append_bf16_on_stream treats a qkv row, so
 *  the pair gives identical bits without the qkv intermediate (with the
 *  pair's GEMM on the weight-stream kernel: batch <= 128 or
 *  KCMM_GEMM_TILED=0).  head_dim %
 *  16 == 0, hidden % 256 == 0, (Hq + 2 Hkv) head_dim % 64 == 0. */
int kcmm_qkv_rope_append_bf16_on_stream(kcmm_pool_t *pool, uint32_t layer_idx, uint64_t x_ptr,
                                        uint64_t w_qkv_ptr, uint64_t q_out_ptr,
                                        uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
                                        uint64_t block_offsets_f16_ptr, uint64_t inv_freq_ptr,
                                        uint32_t batch, uint32_t hidden_size,
                                        uint32_t num_q_heads, uint32_t max_blocks_per_seq,
                                        uint64_t stream_ptr);

/** The end of a decode step (ref llama_transformer.rs:382-390: final norm,
 *  lm_head GEMM): logits[b] = lm_head * rmsnorm(hidden[b]) with weight
 *  norm_w, bf16 [batch][vocab_size] on the device (the reference copies fp32
 *  logits to the host; the caller converts or samples where it needs them).
 *  hidden_size % 256 == 0, vocab_size % 64 == 0.  Enqueue only. */
int kcmm_decode_logits_bf16_on_stream(uint64_t hidden_ptr, uint64_t norm_w_ptr,
                                      uint64_t lm_head_ptr, uint64_t logits_ptr, uint32_t batch,
                                      uint32_t hidden_size, uint32_t vocab_size, float rms_eps,
                                      uint64_t stream_ptr);

/** Device addresses of one layer's weights (bf16, row-major [out][in]). */
typedef struct kcmm_layer_weights {
    uint64_t attn_norm; /**< [hidden] */
    uint64_t qkv;       /**< [(Hq + 2 Hkv) head_dim][hidden]: q rows, k rows, v rows */
    uint64_t o;         /**< [hidden][Hq head_dim] */
    uint64_t mlp_norm;  /**< [hidden] */
    uint64_t gate_up;   /**< [2 intermediate][hidden]: gate rows, then up rows */
    uint64_t down;      /**< [hidden][intermediate] */
} kcmm_layer_weights_t;

/** One decoder layer of a decode step, in place on hidden_ptr
 *  ([batch][hidden] bf16), for layer `layer_idx` of a bf16 or fp8 pool (ref
 *  LlamaTransformer::forward_step_paged, llama_transformer.rs:262-391, per
 *  layer): h += o(attn(rope(qkv(rmsnorm(h))))), with this token's k / v
 *  appended to the pages; h += down(silu(gate) * up(rmsnorm(h))).  kv
 *  heads, head_dim and block size are the pool's; attention scale is
 *  1/sqrt(head_dim).  seq_lens include the new token (its position is
 *  seq_lens[b] - 1).  hidden, intermediate and q_heads * head_dim must be
 *  multiples of 256.  Activations use a per-stream workspace of the library. */
int kcmm_decode_layer_step_on_stream(kcmm_pool_t *pool, uint32_t layer_idx,
                                     const kcmm_layer_weights_t *weights, uint64_t hidden_ptr,
                                     uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
                                     uint64_t block_offsets_f16_ptr, uint64_t inv_freq_ptr,
                                     uint32_t batch, uint32_t hidden_size,
                                     uint32_t num_q_heads, uint32_t intermediate_size,
                                     uint32_t max_blocks_per_seq, float rms_eps,
                                     uint64_t stream_ptr);

/** Layers first_layer .. first_layer + num_layers - 1 of a decode step in one
 *  call (the loop of ref LlamaTransformer::forward_step_paged over its
 *  layers, llama_transformer.rs:262-391), in place on hidden_ptr: the same
 *  arithmetic as num_layers calls of kcmm_decode_layer_step_on_stream, with
 *  one kernel fewer per layer boundary (a layer's down projection leaves
 *  fp32 partials whose residual add the next layer's first RMSNorm
 *  finishes).  weights points to num_layers host structs; layer i uses
 *  weights[i] and pool layer first_layer + i.  Same shape rules. */
int kcmm_decode_layers_on_stream(kcmm_pool_t *pool, uint32_t first_layer, uint32_t num_layers,
                                 const kcmm_layer_weights_t *weights, uint64_t hidden_ptr,
                                 uint64_t block_tables_ptr, uint64_t seq_lens_ptr,
                                 uint64_t block_offsets_f16_ptr, uint64_t inv_freq_ptr,
                                 uint32_t batch, uint32_t hidden_size, uint32_t num_q_heads,
                                 uint32_t intermediate_size, uint32_t max_blocks_per_seq,
                                 float rms_eps, uint64_t stream_ptr);

/** Device addresses of one layer's weights with fp8-e4m3 (OCP e4m3fn)
 *  projections: each projection matrix as e4m3 codes, row-major [out][in],
 *  with an fp32 scale per output row (weight[r][c] = decode(code[r][c]) *
 *  scale[r]); the RMSNorm weights stay bf16.  Shapes as kcmm_layer_weights_t. */
typedef struct kcmm_layer_weights_fp8 {
    uint64_t attn_norm;     /**< bf16 [hidden] */
    uint64_t qkv;           /**< e4m3 [(Hq + 2 Hkv) head_dim][hidden] */
    uint64_t qkv_scale;     /**< fp32 [(Hq + 2 Hkv) head_dim] */
    uint64_t o;             /**< e4m3 [hidden][Hq head_dim] */
    uint64_t o_scale;       /**< fp32 [hidden] */
    uint64_t mlp_norm;      /**< bf16 [hidden] */
    uint64_t gate_up;       /**< e4m3 [2 intermediate][hidden]: gate rows, then up rows */
    uint64_t gate_up_scale; /**< fp32 [2 intermediate] */
    uint64_t down;          /**< e4m3 [hidden][intermediate] */
    uint64_t down_scale;    /**< fp32 [hidden] */
} kcmm_layer_weights_fp8_t;

/** kcmm_decode_layers_on_stream with fp8-e4m3 projection weights (the same
 *  layer loop, ref LlamaTransformer::forward_step_paged,
 *  llama_transformer.rs:262-391, whose GEMMs are bf16 cuBLAS calls there; the
 *  fp8-weight form has no counterpart in the reference).  Every projection
 *  streams half the weight bytes of the bf16 form; activations, the RMSNorm
 *  weights and the pool's pages are as in kcmm_decode_layers_on_stream, and
 *  each product is sum(x * code) * scale in fp32 before the same bf16
 *  rounding.  All four scale pointers of every layer must be set. */
int kcmm_decode_layers_fp8w_on_stream(kcmm_pool_t *pool, uint32_t first_layer,
                                      uint32_t num_layers,
                                      const kcmm_layer_weights_fp8_t *weights,
                                      uint64_t hidden_ptr, uint64_t block_tables_ptr,
                                      uint64_t seq_lens_ptr, uint64_t block_offsets_f16_ptr,
                                      uint64_t inv_freq_ptr, uint32_t batch,
                                      uint32_t hidden_size, uint32_t num_q_heads,
                                      uint32_t intermediate_size, uint32_t max_blocks_per_seq,
                                      float rms_eps, uint64_t stream_ptr);

#ifdef __cplusplus
}
#endif

#endif /* KCMM_MI355X_H */
