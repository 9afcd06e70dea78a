// KV append (reshape-and-cache) kernels for gfx950.
//
// Reference semantics: a source row b of [batch][kv_heads*head_dim] lands at
// region + page_offset + slot*row_bytes for both K and V (ref pool.rs:1036-1098,
// ffi.rs:1088-1383), or -- with device slot ids -- at
// region + offsets_f16[slot/bs]*2 + (slot%bs)*row_bytes with the status word
// of ref kcmm_vllm_kv_write.cu:8-66 (1 = id past the table, 2 = inactive id).
// The reference issues two driver memcpys per row (host paths) or one thread
// per 16-bit element (device path); here one launch moves every row with
// 16-byte vector copies.
//
// fp8-e4m3 pools take bf16 source rows and quantize per (page, kv head): the
// row written at slot 0 sets the page scale to amax/448 (1 for an all-zero
// row); a later row whose amax exceeds 448*scale raises the scale to
// amax/448 and re-encodes the rows already in the page, so no value is ever
// clipped.  Encoding is round-to-nearest-even with saturation to +-448.
#include <algorithm>
#include <cmath>
#include <vector>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

constexpr int kRowsPerLaunch = 64;

struct RowBatch {
    uint64_t dst[kRowsPerLaunch];  // byte offset of the destination row in a region
    uint32_t src[kRowsPerLaunch];  // source row index
};

// 16-bit pools: plain row copies.
__global__ __launch_bounds__(256) void kv_rows_copy(RowBatch rb, uint8_t* k_base, uint8_t* v_base,
                                                     const uint8_t* k_src, const uint8_t* v_src,
                                                     uint32_t row_bytes) {
    const int r = blockIdx.x;
    const uint64_t d = rb.dst[r];
    const uint64_t s = static_cast<uint64_t>(rb.src[r]) * row_bytes;
    if ((row_bytes & 15u) == 0) {
        for (uint32_t i = threadIdx.x * 16; i < row_bytes; i += 256 * 16) {
            *reinterpret_cast<u32x4*>(k_base + d + i) = *reinterpret_cast<const u32x4*>(k_src + s + i);
            *reinterpret_cast<u32x4*>(v_base + d + i) = *reinterpret_cast<const u32x4*>(v_src + s + i);
        }
    } else {
        for (uint32_t i = threadIdx.x * 2; i < row_bytes; i += 256 * 2) {
            *reinterpret_cast<uint16_t*>(k_base + d + i) = *reinterpret_cast<const uint16_t*>(k_src + s + i);
            *reinterpret_cast<uint16_t*>(v_base + d + i) = *reinterpret_cast<const uint16_t*>(v_src + s + i);
        }
    }
}

// fp32 -> OCP e4m3fn, round to nearest even, saturating to +-448.
__device__ __forceinline__ uint32_t f32_to_fp8e4m3(float x) {
    const uint32_t bits = __float_as_uint(x);
    const uint32_t sign = (bits >> 24) & 0x80u;
    const float a = fabsf(x);
    if (a != a) return sign | 0x7fu;
    if (a >= 448.0f) return sign | 0x7eu;
    if (a < 0.015625f) {  // below 2^-6: subnormal grid of 2^-9
        return sign | static_cast<uint32_t>(rintf(a * 512.0f));
    }
    const uint32_t ab = __float_as_uint(a);
    int e = static_cast<int>(ab >> 23) - 127;
    const uint32_t mant = ab & 0x7fffffu;
    uint32_t q = mant >> 20;
    const uint32_t rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ++q;
    if (q == 8) {
        q = 0;
        ++e;
    }
    uint32_t code = (static_cast<uint32_t>(e + 7) << 3) | q;
    if (code > 0x7eu) code = 0x7eu;
    return sign | code;
}

// Writes the bf16 head row `src` at token row `slot` of an fp8 page (kv head
// kvh) with one wavefront.  `scale` is the page scale before this row (unused
// when slot == 0); returns the scale after it, which the caller stores in the
// footer once its last row is written.  Rows of one page must go through one
// wavefront in call order: each may raise the scale and re-encode the rows
// before it.
__device__ float fp8_put_row(uint8_t* page, uint32_t slot, uint32_t kvh, const uint16_t* src,
                             uint32_t head_dim, uint32_t row_bytes, float scale) {
    const int lane = threadIdx.x & 63;
    float x[4];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = lane + 64 * i;
        x[i] = d < head_dim ? bf16_bits_to_f32(src[d]) : 0.0f;
        amax = fmaxf(amax, fabsf(x[i]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if (slot == 0) {
        scale = amax > 0.0f ? amax / 448.0f : 1.0f;
    } else if (amax > 448.0f * scale) {
        const float old = scale;
        scale = amax / 448.0f;
        // re-encode the rows already in this page with the larger scale
        for (uint32_t u = 0; u < slot; ++u) {
            uint8_t* row = page + static_cast<uint64_t>(u) * row_bytes + kvh * head_dim;
            for (uint32_t d = lane; d < head_dim; d += 64) {
                const float y = fp8e4m3_to_f32(row[d]) * old;
                row[d] = static_cast<uint8_t>(f32_to_fp8e4m3(y / scale));
            }
        }
    }
    uint8_t* row = page + static_cast<uint64_t>(slot) * row_bytes + kvh * head_dim;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = lane + 64 * i;
        if (d < head_dim) row[d] = static_cast<uint8_t>(f32_to_fp8e4m3(x[i] / scale));
    }
    return scale;
}

__device__ __forceinline__ float* fp8_scale_ptr(uint8_t* page, uint32_t data_bytes, uint32_t kvh) {
    return reinterpret_cast<float*>(page + data_bytes) + kvh;
}

// Host-resolved fp8 rows grouped by page: rows start[g] .. start[g+1]-1 of the
// batch target one page, in call order.  A page's rows may continue in the
// next launch of the same call (launches on one stream run in order).
struct Fp8RowBatch {
    uint64_t page[kRowsPerLaunch];
    uint32_t slot[kRowsPerLaunch];
    uint32_t src[kRowsPerLaunch];
    uint16_t start[kRowsPerLaunch + 1];
};

// Waves per fp8 writer workgroup: one per (kv head, K|V) pair, at most 16.
constexpr int kFp8MaxWaves = 16;

// grid (groups); wave w takes the (kv head, K|V) pairs w, w + waves, ...
__global__ __launch_bounds__(64 * kFp8MaxWaves) void kv_rows_fp8(
    Fp8RowBatch rb, uint8_t* k_base, uint8_t* v_base, const uint16_t* k_src,
    const uint16_t* v_src, uint32_t kv_heads, uint32_t head_dim, uint32_t row_bytes,
    uint32_t data_bytes) {
    const uint32_t g = blockIdx.x;
    const uint32_t r0 = rb.start[g], r1 = rb.start[g + 1];
    const uint32_t waves = blockDim.x >> 6;
    for (uint32_t j = threadIdx.x >> 6; j < 2 * kv_heads; j += waves) {
        const uint32_t kvh = j >> 1;
        const bool is_v = j & 1;
        uint8_t* page = (is_v ? v_base : k_base) + rb.page[r0];
        float* sp = fp8_scale_ptr(page, data_bytes, kvh);
        float scale = rb.slot[r0] == 0 ? 1.0f : *sp;
        for (uint32_t r = r0; r < r1; ++r) {
            const uint16_t* src = (is_v ? v_src : k_src) +
                                  (static_cast<uint64_t>(rb.src[r]) * kv_heads + kvh) * head_dim;
            scale = fp8_put_row(page, rb.slot[r], kvh, src, head_dim, row_bytes, scale);
        }
        if ((threadIdx.x & 63) == 0) *sp = scale;
    }
}

struct SlotArgs {
    const int64_t* slots;
    const uint64_t* offsets_f16;
    const uint8_t* valid;
    int32_t* status;
    uint8_t* k_base;
    uint8_t* v_base;
    const uint8_t* k_src;
    const uint8_t* v_src;
    uint32_t offsets_len, block_size, row_bytes, src_row_bytes, kv_heads, head_dim, data_bytes;
};

// Resolves row r's slot; returns false (after recording the status) when the
// row is padding or invalid.
__device__ __forceinline__ bool resolve_slot(const SlotArgs& a, uint32_t r, uint64_t* page,
                                             uint32_t* slot_in_page) {
    const int64_t slot = a.slots[r];
    if (slot < 0) return false;
    const int64_t id = slot / a.block_size;
    if (id >= static_cast<int64_t>(a.offsets_len)) {
        if (a.status && threadIdx.x == 0) atomicCAS(a.status, 0, 1);
        return false;
    }
    if (a.valid && a.valid[id] == 0) {
        if (a.status && threadIdx.x == 0) atomicCAS(a.status, 0, 2);
        return false;
    }
    *page = a.offsets_f16[id] * 2ull;
    *slot_in_page = static_cast<uint32_t>(slot % a.block_size);
    return true;
}

__global__ __launch_bounds__(256) void kv_slots_copy(SlotArgs a) {
    const uint32_t r = blockIdx.x;
    uint64_t page;
    uint32_t sl;
    if (!resolve_slot(a, r, &page, &sl)) return;
    const uint64_t d = page + static_cast<uint64_t>(sl) * a.row_bytes;
    const uint64_t s = static_cast<uint64_t>(r) * a.row_bytes;
    if ((a.row_bytes & 15u) == 0) {
        for (uint32_t i = threadIdx.x * 16; i < a.row_bytes; i += 256 * 16) {
            *reinterpret_cast<u32x4*>(a.k_base + d + i) = *reinterpret_cast<const u32x4*>(a.k_src + s + i);
            *reinterpret_cast<u32x4*>(a.v_base + d + i) = *reinterpret_cast<const u32x4*>(a.v_src + s + i);
        }
    } else {
        for (uint32_t i = threadIdx.x * 2; i < a.row_bytes; i += 256 * 2) {
            *reinterpret_cast<uint16_t*>(a.k_base + d + i) = *reinterpret_cast<const uint16_t*>(a.k_src + s + i);
            *reinterpret_cast<uint16_t*>(a.v_base + d + i) = *reinterpret_cast<const uint16_t*>(a.v_src + s + i);
        }
    }
}

// fp8 pages through device slot ids, in two kernels so that the rows of one
// page are applied in call order by one wavefront per (kv head, K|V), as a
// sequential writer would.  `lead` / `cnt` (int32 per block id, zero between
// calls) collect, per page, batch - (first row) and the number of rows.
// Pass 1: one thread per row resolves the slot (status as above) and enters
// the row; pass 2: the workgroup of a page's first row writes all its rows,
// then restores both entries to zero.
__global__ __launch_bounds__(256) void kv_slots_fp8_collect(SlotArgs a, uint32_t batch,
                                                            int32_t* lead, int32_t* cnt) {
    const uint32_t r = blockIdx.x * 256 + threadIdx.x;
    if (r >= batch) return;
    const int64_t slot = a.slots[r];
    if (slot < 0) return;
    const int64_t id = slot / a.block_size;
    if (id >= static_cast<int64_t>(a.offsets_len)) {
        if (a.status) atomicCAS(a.status, 0, 1);
        return;
    }
    if (a.valid && a.valid[id] == 0) {
        if (a.status) atomicCAS(a.status, 0, 2);
        return;
    }
    atomicMax(lead + id, static_cast<int32_t>(batch - r));
    atomicAdd(cnt + id, 1);
}

// grid (batch); 64 * min(2 kv_heads, 16) threads.
__global__ __launch_bounds__(64 * kFp8MaxWaves) void kv_slots_fp8_write(SlotArgs a,
                                                                         uint32_t batch,
                                                                         int32_t* lead,
                                                                         int32_t* cnt) {
    __shared__ int32_t s_rows;
    const uint32_t r = blockIdx.x;
    const int64_t slot = a.slots[r];
    // Rows that pass 1 skipped never lead; neither does a row whose page has
    // an earlier row (its entry holds another row, or zero once restored).
    if (slot < 0) return;
    const int64_t id = slot / a.block_size;
    if (id >= static_cast<int64_t>(a.offsets_len) || (a.valid && a.valid[id] == 0)) return;
    if (threadIdx.x == 0)
        s_rows = __atomic_load_n(lead + id, __ATOMIC_RELAXED) == static_cast<int32_t>(batch - r)
                     ? __atomic_load_n(cnt + id, __ATOMIC_RELAXED)
                     : 0;
    __syncthreads();
    const int32_t rows = s_rows;
    if (rows == 0) return;
    const uint64_t page_off = a.offsets_f16[id] * 2ull;
    const uint32_t waves = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    for (uint32_t j = threadIdx.x >> 6; j < 2 * a.kv_heads; j += waves) {
        const uint32_t kvh = j >> 1;
        const bool is_v = j & 1;
        uint8_t* page = (is_v ? a.v_base : a.k_base) + page_off;
        const uint16_t* src_base = reinterpret_cast<const uint16_t*>(is_v ? a.v_src : a.k_src);
        float* sp = fp8_scale_ptr(page, a.data_bytes, kvh);
        float scale = 1.0f;
        bool have_scale = false;
        int32_t done = 0;
        // rows of this page, in call order, from this one on
        for (uint32_t base = r; done < rows && base < batch; base += 64) {
            const uint32_t rr = base + lane;
            const int64_t s2 = rr < batch ? a.slots[rr] : -1;
            const bool mine = s2 >= 0 && s2 / a.block_size == id;
            uint64_t mask = __ballot(mine);
            while (mask != 0 && done < rows) {
                const int i = __builtin_ctzll(mask);
                mask &= mask - 1;
                const uint32_t row = base + i;
                const uint32_t in_page = static_cast<uint32_t>(a.slots[row] % a.block_size);
                if (!have_scale) {
                    scale = in_page == 0 ? 1.0f : *sp;
                    have_scale = true;
                }
                scale = fp8_put_row(page, in_page, kvh,
                                    src_base + (static_cast<uint64_t>(row) * a.kv_heads + kvh) *
                                                   a.head_dim,
                                    a.head_dim, a.row_bytes, scale);
                ++done;
            }
        }
        if (lane == 0) *sp = scale;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        lead[id] = 0;
        cnt[id] = 0;
    }
}

}  // namespace

namespace dev {

bool kv_write_rows(const KvRowsArgs& a, std::string* err) {
    hipStream_t s = reinterpret_cast<hipStream_t>(a.stream);
    auto* kb = reinterpret_cast<uint8_t*>(a.k_base);
    auto* vb = reinterpret_cast<uint8_t*>(a.v_base);
    if (a.dtype == kDtFP8) {
        if (a.head_dim > 256) {
            *err = "fp8 KV write supports head_dim <= 256";
            return false;
        }
        // Rows grouped by page, call order kept inside a page (pages are
        // independent, so groups may run in any order).
        std::vector<uint32_t> order(a.num_rows);
        for (size_t i = 0; i < a.num_rows; ++i) order[i] = static_cast<uint32_t>(i);
        std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) {
            return a.rows[x].page_offset < a.rows[y].page_offset;
        });
        const int waves = static_cast<int>(std::min<uint32_t>(2 * a.kv_heads, kFp8MaxWaves));
        for (size_t base = 0; base < a.num_rows; base += kRowsPerLaunch) {
            const size_t n = std::min<size_t>(kRowsPerLaunch, a.num_rows - base);
            Fp8RowBatch rb{};
            uint32_t groups = 0;
            for (size_t i = 0; i < n; ++i) {
                const RowDst& r = a.rows[order[base + i]];
                if (i == 0 || r.page_offset != rb.page[i - 1]) rb.start[groups++] = static_cast<uint16_t>(i);
                rb.page[i] = r.page_offset;
                rb.slot[i] = r.slot;
                rb.src[i] = r.src_row;
            }
            rb.start[groups] = static_cast<uint16_t>(n);
            hipLaunchKernelGGL(kv_rows_fp8, dim3(groups), dim3(64 * waves), 0, s, rb, kb, vb,
                               reinterpret_cast<const uint16_t*>(a.k_src),
                               reinterpret_cast<const uint16_t*>(a.v_src), a.kv_heads, a.head_dim,
                               a.row_bytes, a.data_bytes);
            KCMM_HIP_CHECK(hipGetLastError(), err);
        }
        return true;
    }
    for (size_t base = 0; base < a.num_rows; base += kRowsPerLaunch) {
        const size_t n = std::min<size_t>(kRowsPerLaunch, a.num_rows - base);
        RowBatch rb{};
        for (size_t i = 0; i < n; ++i) {
            const RowDst& r = a.rows[base + i];
            rb.dst[i] = r.page_offset + static_cast<uint64_t>(r.slot) * a.row_bytes;
            rb.src[i] = r.src_row;
        }
        hipLaunchKernelGGL(kv_rows_copy, dim3(n), dim3(256), 0, s, rb, kb, vb,
                           reinterpret_cast<const uint8_t*>(a.k_src),
                           reinterpret_cast<const uint8_t*>(a.v_src), a.row_bytes);
        KCMM_HIP_CHECK(hipGetLastError(), err);
    }
    return true;
}

bool kv_write_device_slots(const KvDeviceSlotsArgs& a, std::string* err) {
    hipStream_t s = reinterpret_cast<hipStream_t>(a.stream);
    SlotArgs sa{};
    sa.slots = reinterpret_cast<const int64_t*>(a.slot_mapping);
    sa.offsets_f16 = reinterpret_cast<const uint64_t*>(a.offsets_f16);
    sa.valid = reinterpret_cast<const uint8_t*>(a.valid_blocks);
    sa.status = reinterpret_cast<int32_t*>(a.status);
    sa.k_base = reinterpret_cast<uint8_t*>(a.k_base);
    sa.v_base = reinterpret_cast<uint8_t*>(a.v_base);
    sa.k_src = reinterpret_cast<const uint8_t*>(a.k_src);
    sa.v_src = reinterpret_cast<const uint8_t*>(a.v_src);
    sa.offsets_len = a.offsets_len;
    sa.block_size = a.block_size;
    sa.row_bytes = a.row_bytes;
    sa.kv_heads = a.kv_heads;
    sa.head_dim = a.head_dim;
    sa.data_bytes = a.data_bytes;
    if (a.dtype == kDtFP8) {
        if (a.head_dim > 256) {
            *err = "fp8 KV write supports head_dim <= 256";
            return false;
        }
        if (a.batch > 0x7FFFFFFFu || a.offsets_len > (1u << 28)) {
            *err = "fp8 KV write: batch or offset table too large";
            return false;
        }
        // per block id: batch - first row, row count (zero between calls)
        void* ws = nullptr;
        if (!stream_workspace(a.stream, 8, static_cast<size_t>(a.offsets_len) * 8, &ws, true, err))
            return false;
        int32_t* lead = static_cast<int32_t*>(ws);
        int32_t* cnt = lead + a.offsets_len;
        hipLaunchKernelGGL(kv_slots_fp8_collect, dim3((a.batch + 255) / 256), dim3(256), 0, s, sa,
                           a.batch, lead, cnt);
        KCMM_HIP_CHECK(hipGetLastError(), err);
        const int waves = static_cast<int>(std::min<uint32_t>(2 * a.kv_heads, kFp8MaxWaves));
        hipLaunchKernelGGL(kv_slots_fp8_write, dim3(a.batch), dim3(64 * waves), 0, s, sa, a.batch,
                           lead, cnt);
    } else {
        hipLaunchKernelGGL(kv_slots_copy, dim3(a.batch), dim3(256), 0, s, sa);
    }
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

}  // namespace dev
}  // namespace kcmm
