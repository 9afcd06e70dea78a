// Device-side entry points used by the C ABI layer (ffi.cpp).  Plain C++
// types only: the HIP implementation lives in device_hip.cpp and kernels/*.hip,
// so ffi.cpp and pool_core.cpp compile without HIP headers.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "pool_core.hpp"

namespace kcmm {
namespace dev {

// Page backing for `device`: HIP VMM superblocks, or one hipMalloc per
// region when VMM is unavailable or KCMM_BACKING=flat.
std::unique_ptr<PageBacking> make_backing(int device, std::string* err);

bool set_device(int device, std::string* err);

// KCMM_* tunables, read once per process on first use (tunables.cpp).
enum class Tun {
    kAttnWaves,     // KCMM_ATTN_WAVES
    kAttnHw,        // KCMM_ATTN_HW
    kAttnMinTiles,  // KCMM_ATTN_MIN_TILES
    kAttnDepth,     // KCMM_ATTN_DEPTH
    kAttnGeneric,   // KCMM_ATTN_GENERIC (set: force the any-shape kernels)
    kGemmSplits,    // KCMM_GEMM_SPLITS
    kGemmWgs,       // KCMM_GEMM_WGS
    kGemmTiled,     // KCMM_GEMM_TILED
    kGemmTile,      // KCMM_GEMM_TILE
    kGemmWaves,     // KCMM_GEMM_WAVES (waves per workgroup of unsplit plain / SwiGLU products)
    kGemmHelpers,   // KCMM_GEMM_HELPERS (0: split products without activation-staging helper waves)
    kCount
};
// true and *value = atoi(variable) when the variable is set.
bool tunable(Tun t, int* value);
int tunable_or(Tun t, int dflt);
void reload_tunables();

// Per-(device, stream, slot, host thread) device scratch; grown on demand
// (slot 0: decode attention partials, 1: GEMM split partials, 2: decode
// attention segment table, 3: decode layer-step activations, 4: the final
// norm's output, 5: unused, 6: tiering staging on
// the null stream, 7: fp8 RoPE/append staging, 8: fp8 page-writer row
// table).  `zero_fill` buffers start zeroed by a fill kernel, and their
// users leave them zeroed.  Keyed by host thread as well, so a thread that
// grows a buffer never frees one another thread has been handed.  Growth
// synchronizes the stream and calls hipMalloc, so it cannot happen under
// graph capture: run each shape once before capturing it.
bool stream_workspace(uint64_t stream, int slot, size_t bytes, void** out, bool zero_fill,
                      std::string* err);
// Buffers of exited threads are freed by the next workspace allocation;
// this frees them now (device synchronize first).  Count of those pending.
bool release_orphaned_workspaces(std::string* err);
size_t orphaned_workspaces();
bool synchronize_device(int device, std::string* err);

// Paged decode attention over one layer's K/V regions.
struct AttnDecodeArgs {
    int32_t dtype;          // pool dtype (kF16: f16 q/out; kBF16, kFP8: bf16 q/out)
    uint64_t q, out;        // [batch][num_q_heads][head_dim]
    uint64_t k_base, v_base;
    uint64_t block_tables;  // int32 [batch][mbps]
    uint64_t seq_lens;      // int32 [batch]
    uint64_t offsets_f16;   // u64 [ids], page byte offset / 2
    uint32_t batch, num_q_heads, kv_heads, head_dim, block_size, mbps;
    uint32_t row_bytes;     // token stride inside a page
    uint32_t data_bytes;    // bytes of page data before the fp8 scale footer
    float scale;
    uint64_t stream;
    bool no_alloc = false;  // scratch from the static array, never the workspace
};
bool attn_decode(const AttnDecodeArgs& a, std::string* err);

// Event timing of the decode-attention streaming kernel, for measurement:
// start creates `max_calls` event pairs on the current device, and each
// streaming-kernel launch after it (not under graph capture) is bracketed by
// the next pair; stop waits for the recorded pairs and returns their average
// duration in microseconds and how many there were, then frees the events.
bool attn_stream_timing_start(uint32_t max_calls, std::string* err);
bool attn_stream_timing_stop(double* avg_us, uint32_t* count, std::string* err);

// Causal chunked-prefill attention over one layer's K/V regions: sequence b's
// last qsl[b+1]-qsl[b] cached tokens are the queries (rows qsl[b]..).
struct AttnPrefillArgs {
    int32_t dtype;            // pool dtype (kF16: f16 q/out; kBF16, kFP8: bf16 q/out)
    uint64_t q, out;          // [total_query_tokens][num_q_heads][head_dim]
    uint64_t k_base, v_base;
    uint64_t block_tables;    // int32 [batch][mbps]
    uint64_t seq_lens;        // int32 [batch], cached tokens including the chunk
    uint64_t query_start_loc; // int32 [batch + 1]
    uint64_t offsets_f16;
    uint32_t batch, total_query_tokens, num_q_heads, kv_heads, head_dim, block_size, mbps;
    uint32_t row_bytes, data_bytes;
    float scale;
    uint64_t stream;
};
bool attn_prefill(const AttnPrefillArgs& a, std::string* err);

// KV append of host-resolved rows: source row r (elements of the pool dtype;
// bf16 for fp8 pools) lands at page_offset + slot*row_bytes in both regions.
struct KvRowsArgs {
    int32_t dtype;
    uint64_t k_base, v_base, k_src, v_src;
    uint32_t block_size, kv_heads, head_dim, row_bytes, data_bytes;
    const RowDst* rows;
    size_t num_rows;
    uint64_t stream;
};
bool kv_write_rows(const KvRowsArgs& a, std::string* err);

// KV append from device-resident int64 slot ids (ref kcmm_vllm_kv_write.cu).
struct KvDeviceSlotsArgs {
    int32_t dtype;
    uint64_t k_base, v_base, k_src, v_src;
    uint64_t slot_mapping, offsets_f16, valid_blocks, status;
    uint32_t offsets_len, batch, block_size;
    uint32_t kv_heads, head_dim, row_bytes, data_bytes;
    uint64_t stream;
};
bool kv_write_device_slots(const KvDeviceSlotsArgs& a, std::string* err);

// Page copies: every (src, dst) byte-offset pair is copied in every region.
bool copy_pages(const std::vector<uint64_t>& region_bases, const uint64_t* pair_offsets,
                size_t num_pairs, uint32_t block_bytes, uint64_t stream, std::string* err);
// Pairs of block ids read on the device; ids outside [0, n_ids) are skipped.
bool copy_pages_device(const std::vector<uint64_t>& region_bases, uint64_t pairs_ptr,
                       uint64_t offsets_f16, size_t num_pairs, uint32_t n_ids,
                       uint32_t block_bytes, uint64_t stream, std::string* err);

// Tiering moves (kernels/tier_copy.hip): n whole blocks between the pool's
// regions (page byte offset pages[b] in every region) and host swap memory
// (host[b]: the block's slot, regions in order, block_bytes each).  On the
// null stream; returns when the copies have finished.
bool tier_evict_copy(const std::vector<uint64_t>& region_bases, const uint64_t* pages,
                     uint8_t* const* host, size_t n, uint32_t block_bytes, std::string* err);
bool tier_restore_copy(const std::vector<uint64_t>& region_bases, const uint64_t* pages,
                       uint8_t* const* host, size_t n, uint32_t block_bytes, std::string* err);
// Page-locked host memory for the swap buffer (hipHostMalloc), freed only by
// host_pinned_free.
bool host_pinned_alloc(size_t bytes, void** out, std::string* err);
void host_pinned_free(void* p);

// Y = X W^T (+ R when residual != 0; R may be Y), bf16, fp32 accumulate.  With a
// residual the product is rounded to bf16 before the add, as a bf16 model does.
bool gemm_bf16(uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t n, uint32_t k,
               uint64_t stream, std::string* err, uint64_t residual = 0);

// The same product for many tokens (m > 128) on the LDS-tiled MFMA kernel
// (kernels/gemm_tiled.hip); n % 64 == 0, k % 64 == 0.
bool gemm_bf16_tiled(uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t n, uint32_t k,
                     uint64_t stream, uint64_t residual, std::string* err);
void gemm_tiled_plan(uint32_t m, uint32_t n, uint32_t k, int* splits, int* tile);
// The tiled kernel for either weight type: bf16 W (wscale == 0) or fp8-e4m3
// W [n][k] with an fp32 scale per row (as gemm_fp8w_bf16).
bool gemm_tiled(uint64_t x, uint64_t w, uint64_t wscale, uint64_t y, uint32_t m, uint32_t n,
                uint32_t k, uint64_t stream, uint64_t residual, std::string* err);

// How a plain product of this shape runs (under the current KCMM_GEMM_*
// settings): kernel 0 = weight-stream, 1 = LDS-tiled; K splits; tiling (tiled
// kernel only, else -1); bytes of fp32 split partials written (and read
// back by the reduction), 0 without a split.
struct GemmPlan {
    int kernel = 0, splits = 1, tile = -1;
    uint64_t partial_bytes = 0;
};
bool gemm_plan(uint32_t m, uint32_t n, uint32_t k, bool fp8_weights, GemmPlan* plan,
               std::string* err);
// Y = X (W8 diag(wscale))^T (+ R when residual != 0, as gemm_bf16): fp8-e4m3
// weights W8 [n][k] with an fp32 scale per weight row, bf16 activations and
// result, fp32 accumulate (weight-stream kernel; the weights are converted to
// bf16 exactly in registers, the row scale multiplies each dot product).
bool gemm_fp8w_bf16(uint64_t x, uint64_t w8, uint64_t wscale, uint64_t y, uint32_t m, uint32_t n,
                    uint32_t k, uint64_t stream, std::string* err, uint64_t residual = 0);
// Y = bf16(sum of `splits` fp32 partials [splits][MN]) (+ R), in split order.
bool gemm_split_reduce_launch(const float* part, uint16_t* y, const uint16_t* r, int mn,
                              int splits, uint64_t stream, std::string* err);


// Decode-step glue (kernels/glue.hip), bf16.
bool rmsnorm_bf16(uint64_t x, uint64_t w, uint64_t y, uint32_t rows, uint32_t hidden, float eps,
                  uint64_t stream, std::string* err);
struct RopeAppendArgs {
    uint64_t qkv;             // [batch][(Hq + 2 Hkv) D]: q heads, k heads, v heads
    uint64_t q_out;           // [batch][Hq][D]
    uint64_t k_base, v_base;  // the layer's regions
    uint64_t block_tables, seq_lens, offsets_f16;
    uint64_t inv_freq;        // fp32 [D/2]
    uint32_t batch, num_q_heads, kv_heads, head_dim, block_size, mbps, row_bytes;
    uint64_t stream;
    int32_t dtype = 1;        // page type: 1 bf16 (rows stored in the pages), 2 fp8
                              // (rows staged, then the fp8 page writer: workspace slot 7)
    uint32_t data_bytes = 0;  // fp8: page bytes before the scale footer
    uint32_t n_ids = 0;       // fp8: block ids the pool has issued (rows naming
                              // a larger id are skipped)
};
bool rope_append_bf16(const RopeAppendArgs& a, std::string* err);
// hidden[b] = embed[ids[b]] (bf16 rows of hidden_size; ids int32 on the
// device; an id outside [0, vocab) gives a zero row).
bool embed_bf16(uint64_t embed, uint64_t ids, uint64_t hidden, uint32_t batch, uint32_t hidden_size,
                uint32_t vocab, uint64_t stream, std::string* err);
bool silu_mul_bf16(uint64_t gate_up, uint64_t act, uint32_t rows, uint32_t inter,
                   uint64_t stream, std::string* err);

// The same two steps fed by a split GEMM's fp32 partials [splits][rows][n]
// (summed in split order and rounded to bf16 first, as the GEMM's own store
// would): RoPE/append of the QKV projection, and the O projection's residual
// add (hidden = bf16(hidden + bf16(sum)), written back) followed by RMSNorm.
bool rope_append_from_partials(const RopeAppendArgs& a, const float* part, int splits,
                               std::string* err);
bool residual_rmsnorm_from_partials(const float* part, int splits, uint64_t hidden, uint64_t w,
                                    uint64_t y, uint32_t rows, uint32_t H, float eps,
                                    uint64_t stream, std::string* err);

// X W^T as fp32 partials [*splits][m][n] in the stream's workspace (slot 1),
// for a consumer that finishes the sum itself.  The projections below take
// fp8-e4m3 weights with fp32 row scales when wscale != 0 (as gemm_fp8w_bf16).
bool gemm_bf16_partials(uint64_t x, uint64_t w, uint32_t m, uint32_t n, uint32_t k,
                        uint64_t stream, float** part, int* splits, std::string* err,
                        uint64_t wscale = 0);

// Fused projections (kernels/gemm.hip): the QKV GEMM whose store does what
// rope_append_bf16 does with its result (a.qkv unused; one token per
// sequence, m == a.batch; head_dim % 16 == 0), and the gate/up GEMM whose
// store does what silu_mul_bf16 does (w_gate_up = [gate; up], [2 inter][k]).
// With a K split the finishing step runs as a second kernel over the partials.
bool gemm_bf16_rope_append(uint64_t x, uint64_t w_qkv, uint32_t m, uint32_t k,
                           const RopeAppendArgs& a, std::string* err, uint64_t wscale = 0);
bool gemm_bf16_swiglu(uint64_t x, uint64_t w_gate_up, uint64_t act, uint32_t m, uint32_t inter,
                      uint32_t k, uint64_t stream, std::string* err, uint64_t wscale = 0);

}  // namespace dev
}  // namespace kcmm
