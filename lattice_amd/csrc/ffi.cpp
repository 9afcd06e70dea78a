// The KCMM C ABI (include/kcmm.h, include/kcmm_mi355x.h).  Argument checks,
// error channel and return conventions follow the reference's Rust FFI
// (ref src/kcmm/ffi.rs); bookkeeping is PoolCore, device work goes through
// device_api.hpp.  This file has no HIP dependency.
#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/kcmm.h"
#include "../../include/kcmm_mi355x.h"
#include "device_api.hpp"
#include "pool_core.hpp"

struct kcmm_pool_t {
    std::unique_ptr<kcmm::PoolCore> core;
    int device = 0;
    std::mutex err_mu;
    std::string last_error;
    // Host swap buffer of the tiering engine: page-locked chunks of
    // kSwapChunkBlocks slots, allocated when a slot in them is first used
    // and kept until the pool is destroyed.  Slots are whole blocks at
    // multiples of the slot size, so none straddles two chunks.
    static constexpr size_t kSwapChunkBlocks = 64;
    std::vector<uint8_t*> swap_chunks;
    size_t swap_slot_bytes = 0;
    std::mutex tier_mu;   // one evict / restore data move at a time

    void set_error(const std::string& s) {
        std::lock_guard<std::mutex> lk(err_mu);
        last_error = s;
    }
    // host address of the swap slot at byte offset off (chunk allocated on demand)
    uint8_t* swap_slot(uint64_t off, std::string* err) {
        const size_t chunk_bytes = kSwapChunkBlocks * swap_slot_bytes;
        const size_t c = static_cast<size_t>(off / chunk_bytes);
        if (c >= swap_chunks.size()) swap_chunks.resize(c + 1, nullptr);
        if (swap_chunks[c] == nullptr) {
            void* p = nullptr;
            if (!kcmm::dev::host_pinned_alloc(chunk_bytes, &p, err)) return nullptr;
            swap_chunks[c] = static_cast<uint8_t*>(p);
        }
        return swap_chunks[c] + (off - c * chunk_bytes);
    }
    ~kcmm_pool_t() {
        for (uint8_t* c : swap_chunks) kcmm::dev::host_pinned_free(c);
    }
};

namespace {

thread_local std::string g_create_error;

size_t write_c_str(char* buf, size_t max_len, const std::string& s) {
    // ref ffi.rs:412-422: copy at most max_len-1 bytes and terminate.
    if (buf == nullptr || max_len == 0) return 0;
    const size_t n = s.size() < max_len - 1 ? s.size() : max_len - 1;
    std::memcpy(buf, s.data(), n);
    buf[n] = '\0';
    return n;
}

std::string fmtu(const char* f, unsigned long long a = 0, unsigned long long b = 0) {
    char buf[256];
    std::snprintf(buf, sizeof(buf), f, a, b);
    return buf;
}

bool layer_ok(kcmm_pool_t* p, uint32_t layer, const char* fn) {
    if (layer < p->core->geo().num_layers) return true;
    p->set_error(std::string(fn) + fmtu(": layer_idx %llu out of bounds", layer));
    return false;
}

// Shared body of every decode-attention entry point (ref ffi.rs:1710-1895).
int attn_impl(kcmm_pool_t* pool, int32_t want_dtype, const char* fn, uint32_t layer_idx,
              uint64_t q, uint64_t out, uint64_t bt, uint64_t sl, uint64_t offs, uint32_t batch,
              uint32_t hq, uint32_t hkv, uint32_t d, uint32_t bs, uint32_t mbps, float scale,
              uint64_t stream, bool sync_after, bool bind_device, bool no_alloc = false) {
    if (pool == nullptr || q == 0 || out == 0 || bt == 0 || sl == 0 || offs == 0) {
        if (pool) pool->set_error(std::string(fn) + ": null pointer argument");
        return -1;
    }
    if (batch == 0 || hq == 0 || hkv == 0 || d == 0 || bs == 0 || mbps == 0) {
        pool->set_error(std::string(fn) + ": shape arguments must be positive");
        return -1;
    }
    if (d > 256) {
        pool->set_error(std::string(fn) + fmtu(": head_dim %llu exceeds kernel limit 256", d));
        return -1;
    }
    if (hq > 0xFFFF || hkv > 0xFFFF || bs > 0xFFFF || mbps > 0xFFFF) {
        pool->set_error(std::string(fn) + ": packed shape argument exceeds 65535");
        return -1;
    }
    if (!layer_ok(pool, layer_idx, fn)) return -1;
    const kcmm::PoolGeometry& g = pool->core->geo();
    if (g.dtype != want_dtype) {
        pool->set_error(std::string(fn) + fmtu(": pool holds kv dtype %llu, this entry point "
                                               "reads dtype %llu",
                                               (unsigned long long)g.dtype,
                                               (unsigned long long)want_dtype));
        return -1;
    }
    // The kernels address pages with the pool's own geometry; a mismatching
    // shape would read past the mapped pages.
    if (hkv != g.kv_heads || d != g.head_dim || bs != g.block_size) {
        pool->set_error(std::string(fn) +
                        ": kv_heads/head_dim/block_size differ from the pool's geometry");
        return -1;
    }
    std::string err;
    if (bind_device && !kcmm::dev::set_device(pool->device, &err)) {
        pool->set_error(std::string(fn) + ": bind device failed: " + err);
        return -1;
    }
    kcmm::dev::AttnDecodeArgs a{};
    a.dtype = g.dtype;
    a.q = q;
    a.out = out;
    a.k_base = pool->core->va_k(layer_idx);
    a.v_base = pool->core->va_v(layer_idx);
    a.block_tables = bt;
    a.seq_lens = sl;
    a.offsets_f16 = offs;
    a.batch = batch;
    a.num_q_heads = hq;
    a.kv_heads = hkv;
    a.head_dim = d;
    a.block_size = bs;
    a.mbps = mbps;
    a.row_bytes = static_cast<uint32_t>(g.row_bytes);
    a.data_bytes = static_cast<uint32_t>(g.data_bytes);
    a.scale = scale;
    a.stream = stream;
    a.no_alloc = no_alloc;
    if (!kcmm::dev::attn_decode(a, &err)) {
        pool->set_error(std::string(fn) + ": launch failed: " + err);
        return -1;
    }
    if (sync_after && !kcmm::dev::synchronize_device(pool->device, &err)) {
        pool->set_error(std::string(fn) + ": synchronize failed: " + err);
        return -1;
    }
    return 0;
}

int write_rows(kcmm_pool_t* pool, const char* fn, uint32_t layer_idx,
               const std::vector<kcmm::RowDst>& rows, uint64_t k_src, uint64_t v_src,
               uint64_t stream) {
    if (rows.empty()) return 0;
    if (k_src == 0 || v_src == 0) {
        pool->set_error(std::string(fn) + ": null source pointer");
        return -1;
    }
    const kcmm::PoolGeometry& g = pool->core->geo();
    std::string err;
    if (!kcmm::dev::set_device(pool->device, &err)) {
        pool->set_error(std::string(fn) + ": bind device failed: " + err);
        return -1;
    }
    kcmm::dev::KvRowsArgs a{};
    a.dtype = g.dtype;
    a.k_base = pool->core->va_k(layer_idx);
    a.v_base = pool->core->va_v(layer_idx);
    a.k_src = k_src;
    a.v_src = v_src;
    a.block_size = static_cast<uint32_t>(g.block_size);
    a.kv_heads = static_cast<uint32_t>(g.kv_heads);
    a.head_dim = static_cast<uint32_t>(g.head_dim);
    a.row_bytes = static_cast<uint32_t>(g.row_bytes);
    a.data_bytes = static_cast<uint32_t>(g.data_bytes);
    a.rows = rows.data();
    a.num_rows = rows.size();
    a.stream = stream;
    if (!kcmm::dev::kv_write_rows(a, &err)) {
        pool->set_error(std::string(fn) + ": " + err);
        return -1;
    }
    return 0;
}

int slots_impl(kcmm_pool_t* pool, uint32_t layer_idx, const int64_t* slots, uint32_t batch,
               uint64_t k, uint64_t v, uint64_t stream) {
    // ref ffi.rs:1258-1383
    if (pool == nullptr || slots == nullptr) {
        if (pool) pool->set_error("kcmm_append_kv_slots: null arguments");
        return -1;
    }
    if (!layer_ok(pool, layer_idx, "kcmm_append_kv_slots")) return -1;
    std::vector<kcmm::RowDst> rows;
    std::string err;
    if (!pool->core->resolve_slots(slots, batch, &rows, &err)) {
        pool->set_error(err);
        return -1;
    }
    return write_rows(pool, "kcmm_append_kv_slots", layer_idx, rows, k, v, stream);
}

}  // namespace

extern "C" {

// ---- lifecycle -----------------------------------------------------------

kcmm_pool_t* kcmm_pool_create_typed(const kcmm_config_t* cfg, int32_t kv_dtype) {
    g_create_error.clear();
    if (cfg == nullptr) {
        g_create_error = "kcmm_pool_create: null config";
        return nullptr;
    }
    kcmm::PoolGeometry g;
    g.block_size = cfg->block_size ? cfg->block_size : 16;  // ref ffi.rs:477
    g.num_layers = cfg->num_layers;
    g.kv_heads = cfg->kv_heads;
    g.head_dim = cfg->head_dim;
    g.max_batch = cfg->max_batch;
    g.max_seq_len = cfg->max_seq_len;
    g.dtype = kv_dtype;
    std::string err;
    if (!g.compute(&err)) {
        g_create_error = "kcmm_pool_create: " + err;
        return nullptr;
    }
    const int device = static_cast<int>(cfg->device_ordinal);
    if (!kcmm::dev::set_device(device, &err)) {
        g_create_error = "kcmm_pool_create: " + err;
        return nullptr;
    }
    std::unique_ptr<kcmm::PageBacking> backing = kcmm::dev::make_backing(device, &err);
    if (!backing) {
        g_create_error = "kcmm_pool_create: " + err;
        return nullptr;
    }
    if (!backing->reserve(2 * g.num_layers, g.region_bytes, &err)) {
        g_create_error = "kcmm_pool_create: " + err;
        return nullptr;
    }
    auto* p = new kcmm_pool_t;
    p->core.reset(new kcmm::PoolCore(g, std::move(backing)));
    p->device = device;
    if (cfg->tiering != 0) {
        // ref ffi.rs:480-497 defaults, tiering.rs:723-770 swap sizing (max_blocks
        // blocks of every layer's K and V)
        const size_t max_blocks = cfg->max_blocks ? cfg->max_blocks : 16384;
        const size_t max_batch = cfg->max_batch_blocks ? cfg->max_batch_blocks : 64;
        p->core->enable_tiering(cfg->eviction_policy, max_blocks, max_batch);
        p->swap_slot_bytes = p->core->block_swap_bytes();
    }
    return p;
}

kcmm_pool_t* kcmm_pool_create(const kcmm_config_t* cfg) {
    return kcmm_pool_create_typed(cfg, kcmm::kF16);
}

void kcmm_pool_destroy(kcmm_pool_t* pool) {
    if (pool == nullptr) return;
    std::string err;
    kcmm::dev::synchronize_device(pool->device, &err);  // ref ffi.rs:552-553
    // scratch of host threads that have exited since the last allocation
    kcmm::dev::release_orphaned_workspaces(&err);
    delete pool;
}

size_t kcmm_last_create_error(char* buf, size_t max_len) {
    if (g_create_error.empty()) return 0;
    return write_c_str(buf, max_len, g_create_error);
}

int32_t kcmm_get_kv_dtype(kcmm_pool_t* pool) { return pool ? pool->core->geo().dtype : -1; }

int32_t kcmm_get_backing_kind(kcmm_pool_t* pool) {
    return pool ? pool->core->backing_kind() : -1;
}

// ---- errors ----------------------------------------------------------------

size_t kcmm_get_last_error(kcmm_pool_t* pool, char* buf, size_t max_len) {
    if (pool == nullptr || buf == nullptr || max_len == 0) return 0;
    std::lock_guard<std::mutex> lk(pool->err_mu);
    if (pool->last_error.empty()) return 0;
    return write_c_str(buf, max_len, pool->last_error);
}

void kcmm_clear_error(kcmm_pool_t* pool) {
    if (pool == nullptr) return;
    std::lock_guard<std::mutex> lk(pool->err_mu);
    pool->last_error.clear();
}

// ---- allocation -------------------------------------------------------------

int kcmm_alloc_blocks(kcmm_pool_t* pool, uint32_t n, uint32_t* out) {
    if (pool == nullptr || out == nullptr || n == 0) {
        if (pool) pool->set_error("kcmm_alloc_blocks: null output buffer or zero count");
        return -1;
    }
    std::vector<uint32_t> tmp(n);
    std::string err;
    if (!pool->core->alloc_blocks(n, tmp.data(), &err)) {
        pool->set_error("kcmm_alloc_blocks: " + err);
        return -1;
    }
    std::memcpy(out, tmp.data(), n * sizeof(uint32_t));
    return 0;
}

int kcmm_free_blocks(kcmm_pool_t* pool, const uint32_t* blocks, uint32_t num) {
    if (pool == nullptr || blocks == nullptr || num == 0) return 0;
    pool->core->free_blocks(blocks, num);
    return 0;
}

// ---- sequences ------------------------------------------------------------------

int kcmm_register_sequence(kcmm_pool_t* pool, const uint32_t* table, uint32_t n,
                           uint32_t* out_seq) {
    if (pool == nullptr || table == nullptr || out_seq == nullptr) {
        if (pool) pool->set_error("kcmm_register_sequence: null arguments");
        return -1;
    }
    *out_seq = pool->core->register_sequence(table, n);
    return 0;
}

int kcmm_unregister_sequence(kcmm_pool_t* pool, uint32_t seq) {
    if (pool == nullptr) return -1;
    pool->core->unregister_sequence(seq);
    return 0;
}

void kcmm_touch(kcmm_pool_t* pool, uint32_t seq) {
    if (pool) pool->core->touch(seq);
}

void kcmm_cool(kcmm_pool_t* pool, uint32_t seq) {
    if (pool) pool->core->cool(seq);
}

void kcmm_update_seq_len(kcmm_pool_t* pool, uint32_t seq, uint32_t len) {
    if (pool) pool->core->update_seq_len(seq, len);
}

uint32_t kcmm_get_seq_len(kcmm_pool_t* pool, uint32_t seq) {
    return pool ? pool->core->get_seq_len(seq) : 0;
}

int kcmm_append_block_to_sequence(kcmm_pool_t* pool, uint32_t seq, uint32_t blk) {
    if (pool == nullptr) return -1;
    if (!pool->core->append_block_to_sequence(seq, blk)) {
        pool->set_error(fmtu("kcmm_append_block_to_sequence: seq_idx %llu out of bounds", seq));
        return -1;
    }
    return 0;
}

int kcmm_get_block_table(kcmm_pool_t* pool, uint32_t seq, uint32_t* out, uint32_t max_blocks,
                         uint32_t* count) {
    if (pool == nullptr || out == nullptr || count == nullptr) {
        if (pool) pool->set_error("kcmm_get_block_table: null arguments");
        return -1;
    }
    std::vector<uint32_t> t;
    if (!pool->core->get_block_table(seq, &t)) {
        pool->set_error(fmtu("kcmm_get_block_table: seq_idx %llu not found", seq));
        *count = 0;
        return -1;
    }
    const size_t n = t.size() < max_blocks ? t.size() : max_blocks;
    if (n) std::memcpy(out, t.data(), n * sizeof(uint32_t));
    *count = static_cast<uint32_t>(n);
    return 0;
}

// ---- block queries -------------------------------------------------------------

uint64_t kcmm_get_block_va_offset(kcmm_pool_t* pool, uint32_t blk) {
    if (pool == nullptr) return 0;
    uint64_t v = 0;
    return pool->core->block_va_offset(blk, &v) ? v : 0;
}

int kcmm_get_all_block_offsets_f16(kcmm_pool_t* pool, uint64_t* out, uint32_t max_blocks,
                                   uint32_t* count) {
    if (pool == nullptr || out == nullptr || count == nullptr) {
        if (pool) pool->set_error("kcmm_get_all_block_offsets_f16: null arguments");
        return -1;
    }
    const std::vector<uint64_t> v = pool->core->all_offsets_f16();
    const size_t n = v.size() < max_blocks ? v.size() : max_blocks;
    if (n) std::memcpy(out, v.data(), n * sizeof(uint64_t));
    *count = static_cast<uint32_t>(n);
    return 0;
}

int kcmm_get_all_block_valid(kcmm_pool_t* pool, uint8_t* out, uint32_t max_blocks,
                             uint32_t* count) {
    if (pool == nullptr || out == nullptr || count == nullptr) {
        if (pool) pool->set_error("kcmm_get_all_block_valid: null arguments");
        return -1;
    }
    const std::vector<uint8_t> v = pool->core->all_valid_flags();
    const size_t n = v.size() < max_blocks ? v.size() : max_blocks;
    if (n) std::memcpy(out, v.data(), n);
    *count = static_cast<uint32_t>(n);
    return 0;
}

int kcmm_get_block_location(kcmm_pool_t* pool, uint32_t blk, kcmm_block_location_t* loc) {
    // ref ffi.rs:951-972
    if (pool == nullptr || loc == nullptr) return -1;
    const int l = pool->core->block_location(blk);
    if (l < 0) {
        pool->set_error(fmtu("kcmm_get_block_location: block_idx %llu not found", blk));
        return -1;
    }
    *loc = static_cast<kcmm_block_location_t>(l);
    return 0;
}

int kcmm_get_block_table_va_offsets(kcmm_pool_t* pool, uint32_t seq, uint64_t* out,
                                    uint32_t max_blocks, uint32_t* count) {
    if (pool == nullptr || out == nullptr || count == nullptr) {
        if (pool) pool->set_error("kcmm_get_block_table_va_offsets: null arguments");
        return -1;
    }
    std::vector<uint64_t> v;
    if (!pool->core->table_va_offsets(seq, &v)) {
        pool->set_error(fmtu("kcmm_get_block_table_va_offsets: seq_idx %llu not found", seq));
        *count = 0;
        return -1;
    }
    const size_t n = v.size() < max_blocks ? v.size() : max_blocks;
    if (n) std::memcpy(out, v.data(), n * sizeof(uint64_t));
    *count = static_cast<uint32_t>(n);
    return 0;
}

uint64_t kcmm_get_va_k(kcmm_pool_t* pool, uint32_t layer) {
    if (pool == nullptr || layer >= pool->core->geo().num_layers) return 0;
    return pool->core->va_k(layer);
}

uint64_t kcmm_get_va_v(kcmm_pool_t* pool, uint32_t layer) {
    if (pool == nullptr || layer >= pool->core->geo().num_layers) return 0;
    return pool->core->va_v(layer);
}

// ---- KV write ---------------------------------------------------------------------

int kcmm_append_kv_step(kcmm_pool_t* pool, uint32_t layer_idx, const uint32_t* seqs,
                        const uint32_t* positions, uint32_t batch, uint64_t k_src,
                        uint64_t v_src) {
    // ref ffi.rs:1088-1200
    if (pool == nullptr || seqs == nullptr || positions == nullptr) {
        if (pool) pool->set_error("kcmm_append_kv_step: null arguments");
        return -1;
    }
    if (!layer_ok(pool, layer_idx, "kcmm_append_kv_step")) return -1;
    std::vector<kcmm::RowDst> rows;
    std::string err;
    if (!pool->core->resolve_positions(seqs, positions, batch, &rows, &err)) {
        pool->set_error(err);
        return -1;
    }
    return write_rows(pool, "kcmm_append_kv_step", layer_idx, rows, k_src, v_src, 0);
}

int kcmm_append_kv_slots(kcmm_pool_t* pool, uint32_t layer_idx, const int64_t* slots,
                         uint32_t batch, uint64_t k, uint64_t v) {
    return slots_impl(pool, layer_idx, slots, batch, k, v, 0);
}

int kcmm_append_kv_slots_on_stream(kcmm_pool_t* pool, uint32_t layer_idx, const int64_t* slots,
                                   uint32_t batch, uint64_t k, uint64_t v, uint64_t stream) {
    return slots_impl(pool, layer_idx, slots, batch, k, v, stream);
}

int kcmm_append_kv_device_slots_on_stream(kcmm_pool_t* pool, uint32_t layer_idx,
                                          uint64_t slot_ptr, uint64_t offs_ptr,
                                          uint64_t valid_ptr, uint32_t offs_len,
                                          uint32_t batch, uint64_t k, uint64_t v,
                                          uint64_t status_ptr, uint64_t stream) {
    // ref ffi.rs:1399-1551
    const char* fn = "kcmm_append_kv_device_slots_on_stream";
    if (pool == nullptr || slot_ptr == 0 || offs_ptr == 0 || k == 0 || v == 0) {
        if (pool) pool->set_error(std::string(fn) + ": null pointer argument");
        return -1;
    }
    if (batch == 0 || offs_len == 0) {
        pool->set_error(std::string(fn) +
                        ": batch and offset table length must be positive");
        return -1;
    }
    if (!layer_ok(pool, layer_idx, fn)) return -1;
    const kcmm::PoolGeometry& g = pool->core->geo();
    std::string err;
    if (!kcmm::dev::set_device(pool->device, &err)) {
        pool->set_error(std::string(fn) + ": bind device failed: " + err);
        return -1;
    }
    kcmm::dev::KvDeviceSlotsArgs a{};
    a.dtype = g.dtype;
    a.k_base = pool->core->va_k(layer_idx);
    a.v_base = pool->core->va_v(layer_idx);
    a.k_src = k;
    a.v_src = v;
    a.slot_mapping = slot_ptr;
    a.offsets_f16 = offs_ptr;
    a.valid_blocks = valid_ptr;
    a.status = status_ptr;
    a.offsets_len = offs_len;
    a.batch = batch;
    a.block_size = static_cast<uint32_t>(g.block_size);
    a.kv_heads = static_cast<uint32_t>(g.kv_heads);
    a.head_dim = static_cast<uint32_t>(g.head_dim);
    a.row_bytes = static_cast<uint32_t>(g.row_bytes);
    a.data_bytes = static_cast<uint32_t>(g.data_bytes);
    a.stream = stream;
    if (!kcmm::dev::kv_write_device_slots(a, &err)) {
        pool->set_error(std::string(fn) + ": launch failed: " + err);
        return -1;
    }
    return 0;
}

int kcmm_precompile_vllm_kv_write_f16(kcmm_pool_t* pool) { return pool ? 0 : -1; }

// ---- decode attention -------------------------------------------------------------

#define KCMM_ATTN_ARGS                                                                     \
    kcmm_pool_t *pool, uint32_t layer_idx, uint64_t q, uint64_t out, uint64_t bt,          \
        uint64_t sl, uint64_t offs, uint32_t batch, uint32_t hq, uint32_t hkv, uint32_t d, \
        uint32_t bs, uint32_t mbps, float scale
#define KCMM_ATTN_PASS layer_idx, q, out, bt, sl, offs, batch, hq, hkv, d, bs, mbps, scale

int kcmm_paged_attn_decode_f16(KCMM_ATTN_ARGS) {
    return attn_impl(pool, kcmm::kF16, "kcmm_paged_attn_decode_f16", KCMM_ATTN_PASS, 0, true,
                     true);
}

int kcmm_paged_attn_decode_f16_on_stream(KCMM_ATTN_ARGS, uint64_t stream) {
    return attn_impl(pool, kcmm::kF16, "kcmm_paged_attn_decode_f16", KCMM_ATTN_PASS, stream,
                     false, true);
}

int kcmm_paged_attn_decode_f16_on_current_context_stream(KCMM_ATTN_ARGS, uint64_t stream) {
    return attn_impl(pool, kcmm::kF16, "kcmm_paged_attn_decode_f16", KCMM_ATTN_PASS, stream,
                     false, false);
}

int kcmm_paged_attn_decode_bf16(KCMM_ATTN_ARGS) {
    return attn_impl(pool, kcmm::kBF16, "kcmm_paged_attn_decode_bf16", KCMM_ATTN_PASS, 0, true,
                     true);
}

int kcmm_paged_attn_decode_bf16_on_stream(KCMM_ATTN_ARGS, uint64_t stream) {
    return attn_impl(pool, kcmm::kBF16, "kcmm_paged_attn_decode_bf16", KCMM_ATTN_PASS, stream,
                     false, true);
}

int kcmm_paged_attn_decode_bf16_noalloc_on_stream(KCMM_ATTN_ARGS, uint64_t stream) {
    return attn_impl(pool, kcmm::kBF16, "kcmm_paged_attn_decode_bf16_noalloc_on_stream",
                     KCMM_ATTN_PASS, stream, false, true, true);
}

int kcmm_attn_stream_timing_start(uint32_t max_calls) {
    std::string err;
    if (!kcmm::dev::attn_stream_timing_start(max_calls, &err)) {
        std::fprintf(stderr, "kcmm_attn_stream_timing_start: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

int kcmm_attn_stream_timing_stop(double* avg_us, uint32_t* count) {
    if (avg_us == nullptr || count == nullptr) return -1;
    std::string err;
    if (!kcmm::dev::attn_stream_timing_stop(avg_us, count, &err)) {
        std::fprintf(stderr, "kcmm_attn_stream_timing_stop: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

int kcmm_paged_attn_decode_f32(KCMM_ATTN_ARGS) {
    return attn_impl(pool, kcmm::kF32, "kcmm_paged_attn_decode_f32", KCMM_ATTN_PASS, 0, true,
                     true);
}

int kcmm_paged_attn_decode_f32_on_stream(KCMM_ATTN_ARGS, uint64_t stream) {
    return attn_impl(pool, kcmm::kF32, "kcmm_paged_attn_decode_f32", KCMM_ATTN_PASS, stream,
                     false, true);
}

int kcmm_paged_attn_decode_fp8_on_stream(KCMM_ATTN_ARGS, uint64_t stream) {
    return attn_impl(pool, kcmm::kFP8, "kcmm_paged_attn_decode_fp8", KCMM_ATTN_PASS, stream,
                     false, true);
}

int kcmm_paged_attn_prefill_on_stream(kcmm_pool_t* pool, uint32_t layer_idx, uint64_t q,
                                      uint64_t out, uint64_t bt, uint64_t sl, uint64_t qsl,
                                      uint64_t offs, uint32_t batch, uint32_t total,
                                      uint32_t hq, uint32_t hkv, uint32_t d, uint32_t bs,
                                      uint32_t mbps, float scale, uint64_t stream) {
    const char* fn = "kcmm_paged_attn_prefill_on_stream";
    if (pool == nullptr || q == 0 || out == 0 || bt == 0 || sl == 0 || qsl == 0 || offs == 0) {
        if (pool) pool->set_error(std::string(fn) + ": null pointer argument");
        return -1;
    }
    if (batch == 0 || hq == 0 || hkv == 0 || d == 0 || bs == 0 || mbps == 0) {
        pool->set_error(std::string(fn) + ": shape arguments must be positive");
        return -1;
    }
    if (d > 256 || hq % hkv != 0 || hq > 0xFFFF || mbps > 0xFFFF) {
        pool->set_error(std::string(fn) + ": head_dim <= 256, q heads a multiple of kv heads "
                                          "and packed shapes <= 65535 required");
        return -1;
    }
    if (static_cast<uint64_t>(total) * hq > 0x7fffffffull) {
        pool->set_error(std::string(fn) + ": too many query rows");
        return -1;
    }
    if (!layer_ok(pool, layer_idx, fn)) return -1;
    const kcmm::PoolGeometry& g = pool->core->geo();
    if (hkv != g.kv_heads || d != g.head_dim || bs != g.block_size) {
        pool->set_error(std::string(fn) +
                        ": kv_heads/head_dim/block_size differ from the pool's geometry");
        return -1;
    }
    std::string err;
    if (!kcmm::dev::set_device(pool->device, &err)) {
        pool->set_error(std::string(fn) + ": bind device failed: " + err);
        return -1;
    }
    kcmm::dev::AttnPrefillArgs a{};
    a.dtype = g.dtype;
    a.q = q;
    a.out = out;
    a.k_base = pool->core->va_k(layer_idx);
    a.v_base = pool->core->va_v(layer_idx);
    a.block_tables = bt;
    a.seq_lens = sl;
    a.query_start_loc = qsl;
    a.offsets_f16 = offs;
    a.batch = batch;
    a.total_query_tokens = total;
    a.num_q_heads = hq;
    a.kv_heads = hkv;
    a.head_dim = d;
    a.block_size = bs;
    a.mbps = mbps;
    a.row_bytes = static_cast<uint32_t>(g.row_bytes);
    a.data_bytes = static_cast<uint32_t>(g.data_bytes);
    a.scale = scale;
    a.stream = stream;
    if (!kcmm::dev::attn_prefill(a, &err)) {
        pool->set_error(std::string(fn) + ": launch failed: " + err);
        return -1;
    }
    return 0;
}

int kcmm_precompile_paged_attn_decode_f16(kcmm_pool_t* pool) { return pool ? 0 : -1; }

// ---- tiering: HBM <-> host swap (ref tiering.rs, pool.rs:824-1002) ----------------

namespace {

// every layer's K and V region base, in region order (K0, V0, K1, V1, ...)
std::vector<uint64_t> region_bases(kcmm_pool_t* pool) {
    std::vector<uint64_t> r;
    for (size_t l = 0; l < pool->core->geo().num_layers; ++l) {
        r.push_back(pool->core->va_k(l));
        r.push_back(pool->core->va_v(l));
    }
    return r;
}

// Restores the blocks of ids (begin, copy, end); false with *err on failure.
bool restore_blocks(kcmm_pool_t* pool, const uint32_t* ids, size_t n, std::string* err) {
    std::lock_guard<std::mutex> lk(pool->tier_mu);
    std::vector<kcmm::TierMove> moves;
    bool partial = false;
    if (!pool->core->begin_restore(ids, n, &moves, &partial, err)) return false;
    std::string why = *err;
    if (!moves.empty()) {
        std::vector<uint64_t> pages;
        std::vector<uint8_t*> host;
        std::string cerr;
        bool ok = true;
        for (const auto& m : moves) {
            pages.push_back(m.va_offset);
            host.push_back(pool->swap_slot(m.cpu_offset, &cerr));
            ok = ok && host.back() != nullptr;
        }
        ok = ok && kcmm::dev::set_device(pool->device, &cerr) &&
             kcmm::dev::tier_restore_copy(region_bases(pool), pages.data(), host.data(),
                                          moves.size(),
                                          static_cast<uint32_t>(pool->core->geo().block_bytes),
                                          &cerr);
        pool->core->end_restore(moves, ok);
        if (!ok) {
            *err = "restore copy failed: " + cerr;
            return false;
        }
    }
    if (partial) {
        *err = why;
        return false;
    }
    return true;
}

}  // namespace

uint32_t kcmm_evict_blocks(kcmm_pool_t* pool, uint32_t count) {
    // ref ffi.rs:1900-1945: every in-use GPU-resident block is a candidate
    if (pool == nullptr || count == 0 || !pool->core->tiering_enabled()) return 0;
    std::lock_guard<std::mutex> lk(pool->tier_mu);
    const std::vector<kcmm::TierMove> moves = pool->core->begin_evict(count);
    if (moves.empty()) return 0;
    std::vector<uint64_t> pages;
    std::vector<uint8_t*> host;
    std::string err;
    bool ok = true;
    for (const auto& m : moves) {
        pages.push_back(m.va_offset);
        host.push_back(pool->swap_slot(m.cpu_offset, &err));
        ok = ok && host.back() != nullptr;
    }
    ok = ok && kcmm::dev::set_device(pool->device, &err) &&
         kcmm::dev::tier_evict_copy(region_bases(pool), pages.data(), host.data(), moves.size(),
                                    static_cast<uint32_t>(pool->core->geo().block_bytes), &err);
    pool->core->end_evict(moves, ok);
    if (!ok) {
        pool->set_error("kcmm_evict_blocks: " + err);
        return 0;
    }
    return static_cast<uint32_t>(moves.size());
}

uint64_t kcmm_restore_evicted_block(kcmm_pool_t* pool, uint32_t blk) {
    // ref ffi.rs:1954-1972, pool.rs:833-884: the block's (new) page offset, 0 on error
    if (pool == nullptr) return 0;
    if (!pool->core->tiering_enabled()) {
        pool->set_error("kcmm_restore_evicted_block: tiering is disabled; cannot restore "
                        "evicted block");
        return 0;
    }
    std::string err;
    if (!restore_blocks(pool, &blk, 1, &err)) {
        pool->set_error("kcmm_restore_evicted_block: " + err);
        return 0;
    }
    uint64_t v = 0;
    pool->core->block_va_offset(blk, &v);
    return v;
}

int kcmm_restore_evicted_blocks(kcmm_pool_t* pool, const uint32_t* ids, uint32_t count) {
    // ref ffi.rs:1984-2003
    if (pool == nullptr || ids == nullptr || count == 0) return 0;
    std::string err;
    if (!pool->core->tiering_enabled()) {
        pool->set_error("kcmm_restore_evicted_blocks: tiering is disabled; cannot restore "
                        "evicted blocks");
        return -1;
    }
    if (!restore_blocks(pool, ids, count, &err)) {
        pool->set_error("kcmm_restore_evicted_blocks: " + err);
        return -1;
    }
    return 0;
}

int kcmm_is_gpu_resident(kcmm_pool_t* pool, uint32_t blk) {
    // ref ffi.rs:2010-2022
    if (pool == nullptr) return 0;
    return pool->core->block_location(blk) == kcmm::kLocGpu ? 1 : 0;
}

// ---- metrics ---------------------------------------------------------------------

int kcmm_get_metrics(kcmm_pool_t* pool, kcmm_metrics_t* out) {
    if (pool == nullptr || out == nullptr) return -1;
    const kcmm::Metrics m = pool->core->metrics();
    out->ifr = m.ifr;
    out->pme = m.pme;
    out->bu = m.bu;
    out->rfi = m.rfi;
    out->gpu_blocks = m.gpu_blocks;
    out->cpu_blocks = 0;
    out->nvme_blocks = 0;
    out->eviction_count = 0;
    out->restoration_count = 0;
    return 0;
}

int kcmm_get_pool_stats(kcmm_pool_t* pool, kcmm_pool_stats_t* out) {
    if (pool == nullptr || out == nullptr) return -1;
    const kcmm::Stats s = pool->core->stats();
    out->blocks_in_use = s.blocks_in_use;
    out->total_blocks = s.total_blocks;
    out->total_physical_blocks = s.total_physical_blocks;
    out->free_physical_blocks = s.free_physical_blocks;
    out->active_sequences = s.active_sequences;
    out->num_layers = s.num_layers;
    out->blocks_per_superblock = s.blocks_per_superblock;
    out->superblock_count = s.superblock_count;
    out->block_size = s.block_size;
    out->max_blocks_per_seq = s.max_blocks_per_seq;
    out->block_bytes = s.block_bytes;
    out->tiering_enabled = pool->core->tiering_enabled() ? 1 : 0;
    out->sharing_enabled = 1;
    out->physical_idle_ratio = s.physical_idle_ratio;
    return 0;
}

uint32_t kcmm_blocks_in_use(kcmm_pool_t* pool) { return pool ? pool->core->blocks_in_use() : 0; }
uint32_t kcmm_total_blocks(kcmm_pool_t* pool) { return pool ? pool->core->total_blocks() : 0; }
uint64_t kcmm_block_state_epoch(kcmm_pool_t* pool) { return pool ? pool->core->epoch() : 0; }
uint32_t kcmm_free_physical_blocks(kcmm_pool_t* pool) {
    return pool ? pool->core->free_physical_blocks() : 0;
}
int kcmm_has_free_blocks(kcmm_pool_t* pool) {
    return pool && pool->core->has_free_blocks() ? 1 : 0;
}
uint32_t kcmm_active_sequences(kcmm_pool_t* pool) {
    return pool ? pool->core->active_sequences() : 0;
}

// ---- policy / hints -------------------------------------------------------------------

int kcmm_set_eviction_policy(kcmm_pool_t* pool, const char* policy) {
    // ref ffi.rs:2200-2231, tiering.rs:851-875 (names are case-insensitive)
    if (pool == nullptr || policy == nullptr) return -1;
    if (!pool->core->tiering_enabled()) {
        pool->set_error("kcmm_set_eviction_policy: tiering is disabled");
        return -1;
    }
    std::string name(policy);
    std::transform(name.begin(), name.end(), name.begin(),
                   [](unsigned char c) { return static_cast<char>(std::tolower(c)); });
    if (!pool->core->set_eviction_policy(name)) {
        pool->set_error("kcmm_set_eviction_policy: unknown eviction policy '" + name +
                        "' (expected lru, lfu, fifo, arc, or sink_window)");
        return -1;
    }
    return 0;
}

uint32_t kcmm_get_eviction_policy(kcmm_pool_t* pool, char* out, uint32_t max_len) {
    // ref ffi.rs:2243-2259
    if (pool == nullptr || out == nullptr || max_len == 0) return 0;
    if (!pool->core->tiering_enabled()) return 0;
    return static_cast<uint32_t>(write_c_str(out, max_len, pool->core->eviction_policy_name()));
}

int kcmm_is_tiering_enabled(kcmm_pool_t* pool) {
    return pool != nullptr && pool->core->tiering_enabled() ? 1 : 0;
}

int kcmm_hint(kcmm_pool_t* pool, uint32_t seq, kcmm_hint_t hint) {
    // ref ffi.rs:2296-2379 with tiering off: touch/cool and priority class.
    if (pool == nullptr) return -1;
    if (!pool->core->has_sequence(seq)) {
        pool->set_error(fmtu("kcmm_hint: seq_idx %llu out of bounds", seq));
        return -1;
    }
    switch (hint) {
        case KCMM_HINT_MULTI_TURN:
        case KCMM_HINT_SYSTEM_PROMPT:
        case KCMM_HINT_ATTENTION_SINK:
        case KCMM_HINT_HEAVY_HITTER: {
            pool->core->touch(seq);
            // ref ffi.rs:2326-2336: and an access of every block of the table
            std::vector<uint32_t> table;
            if (pool->core->tiering_enabled() && pool->core->get_block_table(seq, &table))
                for (uint32_t b : table) pool->core->policy_access(b);
            break;
        }
        case KCMM_HINT_HIGH_PRIORITY:
            pool->core->touch(seq);
            pool->core->set_priority(seq, 3);
            break;
        case KCMM_HINT_NEAR_END: pool->core->cool(seq); break;
        case KCMM_HINT_LOW_PRIORITY:
            pool->core->cool(seq);
            pool->core->set_priority(seq, 1);
            break;
        case KCMM_HINT_EVICTABLE:
            pool->core->cool(seq);
            pool->core->set_priority(seq, 0);
            break;
        default: break;
    }
    return 0;
}

int kcmm_protect(kcmm_pool_t* pool, uint32_t, const uint32_t* ids, uint32_t n,
                 kcmm_protection_t level) {
    // ref ffi.rs:2388-2442: with tiering, never-evict / preferred refresh the
    // blocks' access, evict-preferred leaves them; an unknown block is an error
    if (pool == nullptr || ids == nullptr || n == 0) return -1;
    if (!pool->core->tiering_enabled()) return 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (pool->core->block_location(ids[i]) < 0) {
            pool->set_error(fmtu("kcmm_protect: block_idx %llu not found", ids[i]));
            return -1;
        }
        if (level != KCMM_EVICT_PREFERRED) pool->core->policy_access(ids[i]);
    }
    return 0;
}

// ---- prefix sharing / copy-on-write ---------------------------------------------------

int kcmm_share_prefix(kcmm_pool_t* pool, uint32_t src, uint32_t dst, uint32_t n,
                      uint32_t* out) {
    if (pool == nullptr || out == nullptr || n == 0) return -1;  // ref ffi.rs:2458-2460
    std::string err;
    if (!pool->core->share_prefix(src, dst, n, out, &err)) {
        pool->set_error(err);
        return -1;
    }
    return 0;
}

int kcmm_prefix_hash_blocks(const int32_t* tokens, uint32_t n_tokens, uint32_t block_size,
                            uint64_t seed, uint64_t* out, uint32_t max_out, uint32_t* count) {
    if ((tokens == nullptr && n_tokens > 0) || out == nullptr || count == nullptr ||
        block_size == 0)
        return -1;
    *count = static_cast<uint32_t>(
        kcmm::prefix_hash_blocks(tokens, n_tokens, block_size, seed, out, max_out));
    return 0;
}

int kcmm_prefix_register(kcmm_pool_t* pool, uint32_t seq, const uint64_t* hashes, uint32_t n,
                         uint32_t* out_added) {
    if (pool == nullptr || (hashes == nullptr && n > 0) || out_added == nullptr) {
        if (pool) pool->set_error("kcmm_prefix_register: null arguments");
        return -1;
    }
    std::string err;
    if (!pool->core->prefix_register(seq, hashes, n, out_added, &err)) {
        pool->set_error(err);
        return -1;
    }
    return 0;
}

int kcmm_prefix_match(kcmm_pool_t* pool, const uint64_t* hashes, uint32_t n, uint32_t* out_blocks,
                      uint32_t* out_matched) {
    if (pool == nullptr || (hashes == nullptr && n > 0) || out_matched == nullptr) {
        if (pool) pool->set_error("kcmm_prefix_match: null arguments");
        return -1;
    }
    *out_matched = pool->core->prefix_match(hashes, n, out_blocks);
    return 0;
}

int kcmm_prefix_attach(kcmm_pool_t* pool, uint32_t dst, const uint64_t* hashes, uint32_t n,
                       uint32_t* out_blocks, uint32_t* out_matched) {
    if (pool == nullptr || (hashes == nullptr && n > 0) || out_matched == nullptr) {
        if (pool) pool->set_error("kcmm_prefix_attach: null arguments");
        return -1;
    }
    std::string err;
    if (!pool->core->prefix_attach(dst, hashes, n, out_blocks, out_matched, &err)) {
        pool->set_error(err);
        return -1;
    }
    return 0;
}

int kcmm_prefix_evict(kcmm_pool_t* pool, uint32_t max_entries, uint32_t* out_evicted) {
    if (pool == nullptr || out_evicted == nullptr) {
        if (pool) pool->set_error("kcmm_prefix_evict: null arguments");
        return -1;
    }
    *out_evicted = pool->core->prefix_evict(max_entries);
    return 0;
}

uint32_t kcmm_prefix_cached_blocks(kcmm_pool_t* pool) {
    return pool ? pool->core->prefix_entries() : 0;
}

int kcmm_fork_sequence(kcmm_pool_t* pool, uint32_t src, uint32_t* out_seq) {
    if (pool == nullptr || out_seq == nullptr) {
        if (pool) pool->set_error("kcmm_fork_sequence: null arguments");
        return -1;
    }
    std::string err;
    if (!pool->core->fork_sequence(src, out_seq, &err)) {
        pool->set_error(err);
        return -1;
    }
    return 0;
}

uint32_t kcmm_get_block_refcount(kcmm_pool_t* pool, uint32_t blk) {
    return pool ? pool->core->refcount(blk) : 0;
}

int kcmm_cow_block_for_append(kcmm_pool_t* pool, uint32_t seq, uint32_t logical,
                              uint32_t* out_src, uint32_t* out_dst) {
    if (pool == nullptr || out_src == nullptr || out_dst == nullptr) {
        if (pool) pool->set_error("kcmm_cow_block_for_append: null arguments");
        return -1;
    }
    std::string err;
    const int rc = pool->core->cow_block_for_append(seq, logical, out_src, out_dst, &err);
    if (rc < 0) pool->set_error(err);
    return rc;
}


int kcmm_copy_blocks_on_stream(kcmm_pool_t* pool, const uint32_t* pairs, uint32_t n,
                               uint64_t stream) {
    if (pool == nullptr || (pairs == nullptr && n > 0)) {
        if (pool) pool->set_error("kcmm_copy_blocks_on_stream: null arguments");
        return -1;
    }
    if (n == 0) return 0;
    std::vector<uint64_t> offs;
    std::string err;
    if (!pool->core->resolve_pairs(pairs, n, &offs, &err)) {
        pool->set_error(err);
        return -1;
    }
    if (!kcmm::dev::set_device(pool->device, &err) ||
        !kcmm::dev::copy_pages(region_bases(pool), offs.data(), n,
                               static_cast<uint32_t>(pool->core->geo().block_bytes), stream,
                               &err)) {
        pool->set_error("kcmm_copy_blocks_on_stream: " + err);
        return -1;
    }
    return 0;
}

int kcmm_fork_beams_on_stream(kcmm_pool_t* pool, const uint32_t* parents, uint32_t n_parents,
                              uint32_t beam_width, uint32_t* children_out, uint64_t stream) {
    if (pool == nullptr || ((parents == nullptr || children_out == nullptr) && n_parents > 0)) {
        if (pool) pool->set_error("kcmm_fork_beams_on_stream: null arguments");
        return -1;
    }
    std::vector<uint32_t> pairs;
    std::string err;
    if (!pool->core->fork_beams(parents, n_parents, beam_width, children_out, &pairs, &err)) {
        pool->set_error(err);
        return -1;
    }
    const uint32_t n = static_cast<uint32_t>(pairs.size() / 2);
    if (n == 0) return 0;
    std::vector<uint64_t> offs;
    if (!pool->core->resolve_pairs(pairs.data(), n, &offs, &err) ||
        !kcmm::dev::set_device(pool->device, &err) ||
        !kcmm::dev::copy_pages(region_bases(pool), offs.data(), n,
                               static_cast<uint32_t>(pool->core->geo().block_bytes), stream,
                               &err)) {
        pool->set_error("kcmm_fork_beams_on_stream: " + err);
        return -1;
    }
    return static_cast<int>(n);
}

int kcmm_copy_blocks_device_on_stream(kcmm_pool_t* pool, uint64_t pairs_ptr, uint64_t offs_ptr,
                                      uint32_t n, uint64_t stream) {
    if (pool == nullptr || pairs_ptr == 0 || offs_ptr == 0) {
        if (pool) pool->set_error("kcmm_copy_blocks_device_on_stream: null pointer argument");
        return -1;
    }
    if (n == 0) return 0;
    std::string err;
    if (!kcmm::dev::set_device(pool->device, &err) ||
        !kcmm::dev::copy_pages_device(region_bases(pool), pairs_ptr, offs_ptr, n,
                                      pool->core->total_blocks(),
                                      static_cast<uint32_t>(pool->core->geo().block_bytes),
                                      stream, &err)) {
        pool->set_error("kcmm_copy_blocks_device_on_stream: " + err);
        return -1;
    }
    return 0;
}

// ---- GEMM ---------------------------------------------------------------------------------

int kcmm_gemm_bf16_on_stream(uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t n,
                             uint32_t k, uint64_t stream) {
    if (x == 0 || w == 0 || y == 0 || m == 0 || n == 0 || k == 0) return -1;
    std::string err;
    if (!kcmm::dev::gemm_bf16(x, w, y, m, n, k, stream, &err)) {
        std::fprintf(stderr, "kcmm_gemm_bf16_on_stream: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

int kcmm_gemm_plan(uint32_t m, uint32_t n, uint32_t k, uint32_t fp8_weights, int64_t* out) {
    if (out == nullptr) return -1;
    std::string err;
    kcmm::dev::GemmPlan plan;
    if (!kcmm::dev::gemm_plan(m, n, k, fp8_weights != 0, &plan, &err)) {
        std::fprintf(stderr, "kcmm_gemm_plan: %s\n", err.c_str());
        return -1;
    }
    out[0] = plan.kernel;
    out[1] = plan.splits;
    out[2] = plan.tile;
    out[3] = static_cast<int64_t>(plan.partial_bytes);
    return 0;
}

int kcmm_gemm_fp8w_bf16_on_stream(uint64_t x, uint64_t w8, uint64_t wscale, uint64_t y, uint32_t m,
                                  uint32_t n, uint32_t k, uint64_t stream) {
    if (x == 0 || w8 == 0 || wscale == 0 || y == 0) return -1;
    std::string err;
    if (!kcmm::dev::gemm_fp8w_bf16(x, w8, wscale, y, m, n, k, stream, &err)) {
        std::fprintf(stderr, "kcmm_gemm_fp8w_bf16_on_stream: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

int kcmm_gemm_bf16_add_on_stream(uint64_t x, uint64_t w, uint64_t residual, uint64_t y,
                                 uint32_t m, uint32_t n, uint32_t k, uint64_t stream) {
    if (x == 0 || w == 0 || residual == 0 || y == 0 || m == 0 || n == 0 || k == 0) return -1;
    std::string err;
    if (!kcmm::dev::gemm_bf16(x, w, y, m, n, k, stream, &err, residual)) {
        std::fprintf(stderr, "kcmm_gemm_bf16_add_on_stream: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

// ---- decode-step glue and the layer step ------------------------------------------------------

int kcmm_gemm_bf16_swiglu_on_stream(uint64_t x, uint64_t w_gate_up, uint64_t act, uint32_t m,
                                    uint32_t intermediate, uint32_t k, uint64_t stream) {
    if (x == 0 || w_gate_up == 0 || act == 0 || m == 0 || intermediate == 0 || k == 0) return -1;
    std::string err;
    if (!kcmm::dev::gemm_bf16_swiglu(x, w_gate_up, act, m, intermediate, k, stream, &err)) {
        std::fprintf(stderr, "kcmm_gemm_bf16_swiglu_on_stream: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

int kcmm_gemm_bf16_add_rmsnorm_on_stream(uint64_t x, uint64_t w, uint64_t hidden, uint64_t norm_w,
                                         uint64_t normed, uint32_t m, uint32_t n, uint32_t k,
                                         float eps, uint64_t stream) {
    if (x == 0 || w == 0 || hidden == 0 || norm_w == 0 || normed == 0 || m == 0 || n == 0 ||
        k == 0 || n % 8 != 0 || !(eps >= 0.0f))
        return -1;
    std::string err;
    float* part = nullptr;
    int splits = 1;
    if (!kcmm::dev::gemm_bf16_partials(x, w, m, n, k, stream, &part, &splits, &err) ||
        !kcmm::dev::residual_rmsnorm_from_partials(part, splits, hidden, norm_w, normed, m, n, eps,
                                                   stream, &err)) {
        std::fprintf(stderr, "kcmm_gemm_bf16_add_rmsnorm_on_stream: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

int kcmm_rmsnorm_bf16_on_stream(uint64_t x, uint64_t w, uint64_t y, uint32_t rows,
                                uint32_t hidden, float eps, uint64_t stream) {
    if (x == 0 || w == 0 || y == 0 || rows == 0 || hidden == 0 || hidden % 8 != 0 ||
        !(eps >= 0.0f))
        return -1;
    std::string err;
    if (!kcmm::dev::rmsnorm_bf16(x, w, y, rows, hidden, eps, stream, &err)) {
        std::fprintf(stderr, "kcmm_rmsnorm_bf16_on_stream: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

int kcmm_embed_tokens_bf16_on_stream(uint64_t embed, uint64_t token_ids, uint64_t hidden,
                                     uint32_t batch, uint32_t hidden_size, uint32_t vocab,
                                     uint64_t stream) {
    if (embed == 0 || token_ids == 0 || hidden == 0 || batch == 0 || hidden_size == 0 ||
        hidden_size % 8 != 0 || vocab == 0)
        return -1;
    std::string err;
    if (!kcmm::dev::embed_bf16(embed, token_ids, hidden, batch, hidden_size, vocab, stream, &err)) {
        std::fprintf(stderr, "kcmm_embed_tokens_bf16_on_stream: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

int kcmm_silu_mul_bf16_on_stream(uint64_t gate_up, uint64_t act, uint32_t rows,
                                 uint32_t intermediate, uint64_t stream) {
    if (gate_up == 0 || act == 0 || rows == 0 || intermediate == 0 || intermediate % 8 != 0)
        return -1;
    std::string err;
    if (!kcmm::dev::silu_mul_bf16(gate_up, act, rows, intermediate, stream, &err)) {
        std::fprintf(stderr, "kcmm_silu_mul_bf16_on_stream: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

namespace {

// Shape checks shared by the RoPE/append and layer-step entry points; the
// kv geometry is the pool's.
bool step_shapes_ok(kcmm_pool_t* pool, const char* fn, uint32_t layer_idx, uint32_t batch,
                    uint32_t hq, uint32_t mbps) {
    if (!layer_ok(pool, layer_idx, fn)) return false;
    const kcmm::PoolGeometry& g = pool->core->geo();
    if (g.dtype != kcmm::kBF16 && g.dtype != kcmm::kFP8) {
        pool->set_error(std::string(fn) + ": needs a bf16 or fp8 pool (bf16 activations)");
        return false;
    }
    if (batch == 0 || hq == 0 || mbps == 0 || hq % g.kv_heads != 0 || hq > 0xFFFF ||
        mbps > 0xFFFF) {
        pool->set_error(std::string(fn) +
                        ": batch, q heads (a multiple of kv heads) and max_blocks_per_seq must "
                        "be positive (q heads and max_blocks_per_seq <= 65535)");
        return false;
    }
    if (g.head_dim % 8 != 0 || g.head_dim > 256) {
        pool->set_error(std::string(fn) + ": head_dim must be a multiple of 8, <= 256");
        return false;
    }
    return true;
}

kcmm::dev::RopeAppendArgs rope_args(kcmm_pool_t* pool, uint32_t layer_idx, uint64_t qkv,
                                    uint64_t q_out, uint64_t bt, uint64_t sl, uint64_t offs,
                                    uint64_t inv_freq, uint32_t batch, uint32_t hq,
                                    uint32_t mbps, uint64_t stream) {
    const kcmm::PoolGeometry& g = pool->core->geo();
    kcmm::dev::RopeAppendArgs a{};
    a.qkv = qkv;
    a.q_out = q_out;
    a.k_base = pool->core->va_k(layer_idx);
    a.v_base = pool->core->va_v(layer_idx);
    a.block_tables = bt;
    a.seq_lens = sl;
    a.offsets_f16 = offs;
    a.inv_freq = inv_freq;
    a.batch = batch;
    a.num_q_heads = hq;
    a.kv_heads = static_cast<uint32_t>(g.kv_heads);
    a.head_dim = static_cast<uint32_t>(g.head_dim);
    a.block_size = static_cast<uint32_t>(g.block_size);
    a.mbps = mbps;
    a.row_bytes = static_cast<uint32_t>(g.row_bytes);
    a.stream = stream;
    a.dtype = g.dtype;
    a.data_bytes = static_cast<uint32_t>(g.data_bytes);
    a.n_ids = pool->core->total_blocks();
    return a;
}

}  // namespace

int kcmm_rope_append_bf16_on_stream(kcmm_pool_t* pool, uint32_t layer_idx, uint64_t qkv,
                                    uint64_t q_out, uint64_t block_tables, uint64_t seq_lens,
                                    uint64_t offsets_f16, uint64_t inv_freq, uint32_t batch,
                                    uint32_t num_q_heads, uint32_t max_blocks_per_seq,
                                    uint64_t stream) {
    const char* fn = "kcmm_rope_append_bf16_on_stream";
    if (pool == nullptr || qkv == 0 || q_out == 0 || block_tables == 0 || seq_lens == 0 ||
        offsets_f16 == 0 || inv_freq == 0) {
        if (pool) pool->set_error(std::string(fn) + ": null pointer argument");
        return -1;
    }
    if (!step_shapes_ok(pool, fn, layer_idx, batch, num_q_heads, max_blocks_per_seq)) return -1;
    std::string err;
    if (!kcmm::dev::set_device(pool->device, &err) ||
        !kcmm::dev::rope_append_bf16(rope_args(pool, layer_idx, qkv, q_out, block_tables, seq_lens,
                                               offsets_f16, inv_freq, batch, num_q_heads,
                                               max_blocks_per_seq, stream),
                                     &err)) {
        pool->set_error(std::string(fn) + ": " + err);
        return -1;
    }
    return 0;
}

int kcmm_qkv_rope_append_bf16_on_stream(kcmm_pool_t* pool, uint32_t layer_idx, uint64_t x,
                                        uint64_t w_qkv, uint64_t q_out, uint64_t block_tables,
                                        uint64_t seq_lens, uint64_t offsets_f16, uint64_t inv_freq,
                                        uint32_t batch, uint32_t hidden_size, uint32_t num_q_heads,
                                        uint32_t max_blocks_per_seq, uint64_t stream) {
    const char* fn = "kcmm_qkv_rope_append_bf16_on_stream";
    if (pool == nullptr || x == 0 || w_qkv == 0 || q_out == 0 || block_tables == 0 ||
        seq_lens == 0 || offsets_f16 == 0 || inv_freq == 0) {
        if (pool) pool->set_error(std::string(fn) + ": null pointer argument");
        return -1;
    }
    if (!step_shapes_ok(pool, fn, layer_idx, batch, num_q_heads, max_blocks_per_seq)) return -1;
    std::string err;
    if (!kcmm::dev::set_device(pool->device, &err) ||
        !kcmm::dev::gemm_bf16_rope_append(x, w_qkv, batch, hidden_size,
                                          rope_args(pool, layer_idx, 0, q_out, block_tables,
                                                    seq_lens, offsets_f16, inv_freq, batch,
                                                    num_q_heads, max_blocks_per_seq, stream),
                                          &err)) {
        pool->set_error(std::string(fn) + ": " + err);
        return -1;
    }
    return 0;
}

extern "C++" {
namespace {

// One layer's weights as the layer driver takes them: bf16 projections (every
// *_scale 0), or fp8-e4m3 projections with an fp32 scale per output row.
struct LayerView {
    uint64_t attn_norm, qkv, qkv_scale, o, o_scale, mlp_norm, gate_up, gate_up_scale, down,
        down_scale;
};

LayerView layer_view(const kcmm_layer_weights_t& l) {
    return {l.attn_norm, l.qkv, 0, l.o, 0, l.mlp_norm, l.gate_up, 0, l.down, 0};
}

LayerView layer_view(const kcmm_layer_weights_fp8_t& l) {
    return {l.attn_norm, l.qkv, l.qkv_scale, l.o, l.o_scale, l.mlp_norm, l.gate_up,
            l.gate_up_scale, l.down, l.down_scale};
}

// Layers first .. first + n - 1 of a decode step, in place on hidden.  Per
// layer: RMSNorm -> QKV projection with RoPE + KV append -> paged attention
// -> O projection (fp32 partials) -> residual add + RMSNorm -> gate/up with
// SwiGLU -> down projection.  Between layers the down projection also leaves
// partials, and the next layer's first RMSNorm finishes its residual add;
// the last layer's down projection adds its residual itself.  W is
// kcmm_layer_weights_t (bf16 projections) or kcmm_layer_weights_fp8_t.
template <typename W>
int run_decode_layers(kcmm_pool_t* pool, const char* fn, uint32_t first, uint32_t n,
                      const W* weights, uint64_t hidden, uint64_t block_tables,
                      uint64_t seq_lens, uint64_t offsets_f16, uint64_t inv_freq, uint32_t batch,
                      uint32_t hidden_size, uint32_t num_q_heads, uint32_t intermediate_size,
                      uint32_t max_blocks_per_seq, float rms_eps, uint64_t stream) {
    if (pool == nullptr || weights == nullptr || n == 0 || hidden == 0 || block_tables == 0 ||
        seq_lens == 0 || offsets_f16 == 0 || inv_freq == 0) {
        if (pool) pool->set_error(std::string(fn) + ": null pointer argument or no layers");
        return -1;
    }
    constexpr bool kFp8 = std::is_same<W, kcmm_layer_weights_fp8_t>::value;
    std::vector<LayerView> w(n);
    for (uint32_t i = 0; i < n; ++i) {
        const LayerView& l = w[i] = layer_view(weights[i]);
        if (l.attn_norm == 0 || l.qkv == 0 || l.o == 0 || l.mlp_norm == 0 || l.gate_up == 0 ||
            l.down == 0 ||
            (kFp8 && (l.qkv_scale == 0 || l.o_scale == 0 || l.gate_up_scale == 0 ||
                      l.down_scale == 0))) {
            pool->set_error(std::string(fn) + ": null weight pointer at layer " +
                            std::to_string(first + i));
            return -1;
        }
    }
    if (first + static_cast<uint64_t>(n) - 1 > 0xFFFFFFFFull ||
        !step_shapes_ok(pool, fn, first, batch, num_q_heads, max_blocks_per_seq) ||
        !step_shapes_ok(pool, fn, first + n - 1, batch, num_q_heads, max_blocks_per_seq))
        return -1;
    const kcmm::PoolGeometry& g = pool->core->geo();
    const uint64_t D = g.head_dim, hkv = g.kv_heads, hq = num_q_heads;
    const uint64_t H = hidden_size, I = intermediate_size;
    const uint64_t qkv_n = (hq + 2 * hkv) * D, attn_k = hq * D;
    // the projection GEMMs take n % 64 == 0 and k % 256 == 0
    if (H == 0 || I == 0 || H % 256 != 0 || I % 256 != 0 || attn_k % 256 != 0 ||
        qkv_n % 64 != 0 || !(rms_eps >= 0.0f)) {
        pool->set_error(std::string(fn) +
                        ": hidden, intermediate and q_heads*head_dim must be multiples of 256, "
                        "(q_heads + 2 kv_heads)*head_dim a multiple of 64, eps >= 0");
        return -1;
    }
    std::string err;
    if (!kcmm::dev::set_device(pool->device, &err)) {
        pool->set_error(std::string(fn) + ": bind device failed: " + err);
        return -1;
    }
    // activations: normed [B][H], qkv [B][qkv_n] (only when RoPE is not fused),
    // q [B][Hq D], attn [B][Hq D], act [B][I] (bf16), each 256-byte aligned
    auto al = [](uint64_t bytes) { return (bytes + 255) & ~255ull; };
    const uint64_t sz_norm = al(batch * H * 2), sz_qkv = D % 16 == 0 ? 0 : al(batch * qkv_n * 2),
                   sz_q = al(batch * attn_k * 2), sz_act = al(batch * I * 2);
    void* ws = nullptr;
    if (!kcmm::dev::stream_workspace(stream, 3, sz_norm + sz_qkv + 2 * sz_q + sz_act, &ws, false,
                                     &err)) {
        pool->set_error(std::string(fn) + ": workspace: " + err);
        return -1;
    }
    const uint64_t base = reinterpret_cast<uint64_t>(ws);
    const uint64_t normed = base, qkv = normed + sz_norm, q = qkv + sz_qkv, attn = q + sz_q,
                   act = attn + sz_q;
    const uint32_t B = batch;

    float* down_part = nullptr;   // previous layer's down-projection partials
    int down_splits = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t layer = first + i;
        const LayerView& l = w[i];
        kcmm::dev::AttnDecodeArgs at{};
        at.dtype = g.dtype;
        at.q = q;
        at.out = attn;
        at.k_base = pool->core->va_k(layer);
        at.v_base = pool->core->va_v(layer);
        at.block_tables = block_tables;
        at.seq_lens = seq_lens;
        at.offsets_f16 = offsets_f16;
        at.batch = batch;
        at.num_q_heads = num_q_heads;
        at.kv_heads = static_cast<uint32_t>(hkv);
        at.head_dim = static_cast<uint32_t>(D);
        at.block_size = static_cast<uint32_t>(g.block_size);
        at.mbps = max_blocks_per_seq;
        at.row_bytes = static_cast<uint32_t>(g.row_bytes);
        at.data_bytes = static_cast<uint32_t>(g.data_bytes);
        at.scale = 1.0f / std::sqrt(static_cast<float>(D));
        at.stream = stream;
        const auto ra = rope_args(pool, layer, qkv, q, block_tables, seq_lens, offsets_f16,
                                  inv_freq, B, num_q_heads, max_blocks_per_seq, stream);
        auto norm1 = [&]() {
            if (down_part == nullptr)
                return kcmm::dev::rmsnorm_bf16(hidden, l.attn_norm, normed, B, hidden_size, rms_eps,
                                               stream, &err);
            return kcmm::dev::residual_rmsnorm_from_partials(down_part, down_splits, hidden,
                                                             l.attn_norm, normed, B, hidden_size,
                                                             rms_eps, stream, &err);
        };
        // QKV projection with RoPE + KV append in its store (head_dim % 16 ==
        // 0), else the projection then the standalone RoPE/append kernel
        auto qkv_step = [&]() {
            if (D % 16 == 0)
                return kcmm::dev::gemm_bf16_rope_append(normed, l.qkv, B, hidden_size, ra, &err,
                                                        l.qkv_scale);
            const bool proj =
                kFp8 ? kcmm::dev::gemm_fp8w_bf16(normed, l.qkv, l.qkv_scale, qkv, B,
                                                 static_cast<uint32_t>(qkv_n), hidden_size,
                                                 stream, &err)
                     : kcmm::dev::gemm_bf16(normed, l.qkv, qkv, B, static_cast<uint32_t>(qkv_n),
                                            hidden_size, stream, &err);
            return proj && kcmm::dev::rope_append_bf16(ra, &err);
        };
        // O projection as partials; the residual add is finished by the
        // RMSNorm kernel that reads them
        auto o_step = [&]() {
            float* part = nullptr;
            int splits = 1;
            return kcmm::dev::gemm_bf16_partials(attn, l.o, B, hidden_size,
                                                 static_cast<uint32_t>(attn_k), stream, &part,
                                                 &splits, &err, l.o_scale) &&
                   kcmm::dev::residual_rmsnorm_from_partials(part, splits, hidden, l.mlp_norm,
                                                             normed, B, hidden_size, rms_eps,
                                                             stream, &err);
        };
        auto down_step = [&]() {
            if (i + 1 == n) {
                down_part = nullptr;
                if (kFp8)
                    return kcmm::dev::gemm_fp8w_bf16(act, l.down, l.down_scale, hidden, B,
                                                     hidden_size, intermediate_size, stream, &err,
                                                     hidden);
                return kcmm::dev::gemm_bf16(act, l.down, hidden, B, hidden_size,
                                            intermediate_size, stream, &err, hidden);
            }
            return kcmm::dev::gemm_bf16_partials(act, l.down, B, hidden_size, intermediate_size,
                                                 stream, &down_part, &down_splits, &err,
                                                 l.down_scale);
        };
        const bool ok = norm1() && qkv_step() && kcmm::dev::attn_decode(at, &err) && o_step() &&
                        kcmm::dev::gemm_bf16_swiglu(normed, l.gate_up, act, B, intermediate_size,
                                                    hidden_size, stream, &err, l.gate_up_scale) &&
                        down_step();
        if (!ok) {
            pool->set_error(std::string(fn) + ": launch failed at layer " + std::to_string(layer) +
                            ": " + err);
            return -1;
        }
    }
    return 0;
}

}  // namespace
}  // extern "C++"

int kcmm_decode_layer_step_on_stream(kcmm_pool_t* pool, uint32_t layer_idx,
                                     const kcmm_layer_weights_t* w, uint64_t hidden,
                                     uint64_t block_tables, uint64_t seq_lens,
                                     uint64_t offsets_f16, uint64_t inv_freq, uint32_t batch,
                                     uint32_t hidden_size, uint32_t num_q_heads,
                                     uint32_t intermediate_size, uint32_t max_blocks_per_seq,
                                     float rms_eps, uint64_t stream) {
    return run_decode_layers(pool, "kcmm_decode_layer_step_on_stream", layer_idx, 1, w, hidden,
                             block_tables, seq_lens, offsets_f16, inv_freq, batch, hidden_size,
                             num_q_heads, intermediate_size, max_blocks_per_seq, rms_eps, stream);
}

int kcmm_decode_layers_on_stream(kcmm_pool_t* pool, uint32_t first_layer, uint32_t num_layers,
                                 const kcmm_layer_weights_t* weights, uint64_t hidden,
                                 uint64_t block_tables, uint64_t seq_lens, uint64_t offsets_f16,
                                 uint64_t inv_freq, uint32_t batch, uint32_t hidden_size,
                                 uint32_t num_q_heads, uint32_t intermediate_size,
                                 uint32_t max_blocks_per_seq, float rms_eps, uint64_t stream) {
    return run_decode_layers(pool, "kcmm_decode_layers_on_stream", first_layer, num_layers,
                             weights, hidden, block_tables, seq_lens, offsets_f16, inv_freq, batch,
                             hidden_size, num_q_heads, intermediate_size, max_blocks_per_seq,
                             rms_eps, stream);
}

int kcmm_decode_layers_fp8w_on_stream(kcmm_pool_t* pool, uint32_t first_layer, uint32_t num_layers,
                                      const kcmm_layer_weights_fp8_t* weights, uint64_t hidden,
                                      uint64_t block_tables, uint64_t seq_lens,
                                      uint64_t offsets_f16, uint64_t inv_freq, uint32_t batch,
                                      uint32_t hidden_size, uint32_t num_q_heads,
                                      uint32_t intermediate_size, uint32_t max_blocks_per_seq,
                                      float rms_eps, uint64_t stream) {
    return run_decode_layers(pool, "kcmm_decode_layers_fp8w_on_stream", first_layer, num_layers,
                             weights, hidden, block_tables, seq_lens, offsets_f16, inv_freq, batch,
                             hidden_size, num_q_heads, intermediate_size, max_blocks_per_seq,
                             rms_eps, stream);
}

int kcmm_decode_logits_bf16_on_stream(uint64_t hidden, uint64_t norm_w, uint64_t lm_head,
                                      uint64_t logits, uint32_t batch, uint32_t hidden_size,
                                      uint32_t vocab_size, float rms_eps, uint64_t stream) {
    if (hidden == 0 || norm_w == 0 || lm_head == 0 || logits == 0 || batch == 0 ||
        hidden_size == 0 || hidden_size % 256 != 0 || vocab_size == 0 || vocab_size % 64 != 0 ||
        !(rms_eps >= 0.0f))
        return -1;
    std::string err;
    void* ws = nullptr;
    if (!kcmm::dev::stream_workspace(stream, 4, static_cast<size_t>(batch) * hidden_size * 2, &ws,
                                     false, &err) ||
        !kcmm::dev::rmsnorm_bf16(hidden, norm_w, reinterpret_cast<uint64_t>(ws), batch,
                                 hidden_size, rms_eps, stream, &err) ||
        !kcmm::dev::gemm_bf16(reinterpret_cast<uint64_t>(ws), lm_head, logits, batch, vocab_size,
                              hidden_size, stream, &err)) {
        std::fprintf(stderr, "kcmm_decode_logits_bf16_on_stream: %s\n", err.c_str());
        return -1;
    }
    return 0;
}

// ---- utilities ---------------------------------------------------------------------------------

int kcmm_below_low_watermark(kcmm_pool_t* pool, float threshold) {
    return pool && pool->core->below_low_watermark(threshold) ? 1 : 0;
}

int kcmm_synchronize(kcmm_pool_t* pool) {
    if (pool == nullptr) return -1;
    std::string err;
    if (!kcmm::dev::synchronize_device(pool->device, &err)) {
        pool->set_error("kcmm_synchronize: " + err);
        return -1;
    }
    return 0;
}

uint32_t kcmm_get_block_size(kcmm_pool_t* p) {
    return p ? static_cast<uint32_t>(p->core->geo().block_size) : 0;
}
uint32_t kcmm_get_max_blocks_per_seq(kcmm_pool_t* p) {
    return p ? static_cast<uint32_t>(p->core->geo().max_blocks_per_seq) : 0;
}
uint32_t kcmm_get_block_bytes(kcmm_pool_t* p) {
    return p ? static_cast<uint32_t>(p->core->geo().block_bytes) : 0;
}
uint32_t kcmm_get_num_layers(kcmm_pool_t* p) {
    return p ? static_cast<uint32_t>(p->core->geo().num_layers) : 0;
}
uint32_t kcmm_get_max_batch(kcmm_pool_t* p) {
    return p ? static_cast<uint32_t>(p->core->geo().max_batch) : 0;
}
uint32_t kcmm_get_max_seq_len(kcmm_pool_t* p) {
    return p ? static_cast<uint32_t>(p->core->geo().max_seq_len) : 0;
}

}  // extern "C"
