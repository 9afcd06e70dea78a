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
#include <cmath>

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

// One wavefront per (row, kv head, K|V): quantize a bf16 head row into an fp8
// page, maintaining the page's scale.  `page` points at the page start.
__device__ void fp8_write_head(uint8_t* page, uint32_t slot, uint32_t kvh, const uint16_t* src,
                               uint32_t head_dim, uint32_t row_bytes, uint32_t data_bytes) {
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
    float* scale_p = reinterpret_cast<float*>(page + data_bytes) + kvh;
    float scale;
    if (slot == 0) {
        scale = amax > 0.0f ? amax / 448.0f : 1.0f;
    } else {
        const float old = *scale_p;
        scale = old;
        if (amax > 448.0f * old) {
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
    }
    uint8_t* row = page + static_cast<uint64_t>(slot) * row_bytes + kvh * head_dim;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t d = lane + 64 * i;
        if (d < head_dim) row[d] = static_cast<uint8_t>(f32_to_fp8e4m3(x[i] / scale));
    }
    if (lane == 0) *scale_p = scale;
}

struct Fp8RowBatch {
    uint64_t page[kRowsPerLaunch];
    uint32_t slot[kRowsPerLaunch];
    uint32_t src[kRowsPerLaunch];
};

// grid (rows, kv_heads, 2); one wavefront each.
__global__ __launch_bounds__(64) void kv_rows_fp8(Fp8RowBatch rb, uint8_t* k_base, uint8_t* v_base,
                                                   const uint16_t* k_src, const uint16_t* v_src,
                                                   uint32_t kv_heads, uint32_t head_dim,
                                                   uint32_t row_bytes, uint32_t data_bytes) {
    const uint32_t r = blockIdx.x, kvh = blockIdx.y;
    const bool is_v = blockIdx.z == 1;
    uint8_t* page = (is_v ? v_base : k_base) + rb.page[r];
    const uint16_t* src = (is_v ? v_src : k_src) +
                          (static_cast<uint64_t>(rb.src[r]) * kv_heads + kvh) * head_dim;
    fp8_write_head(page, rb.slot[r], kvh, src, head_dim, row_bytes, data_bytes);
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

// grid (batch, kv_heads, 2); one wavefront each.
__global__ __launch_bounds__(64) void kv_slots_fp8(SlotArgs a) {
    const uint32_t r = blockIdx.x, kvh = blockIdx.y;
    const bool is_v = blockIdx.z == 1;
    uint64_t page;
    uint32_t sl;
    // Only the (kvh 0, K) wavefront reports status, so the word is set once.
    SlotArgs aa = a;
    if (kvh != 0 || is_v) aa.status = nullptr;
    if (!resolve_slot(aa, r, &page, &sl)) return;
    const uint16_t* src = reinterpret_cast<const uint16_t*>(is_v ? a.v_src : a.k_src) +
                          (static_cast<uint64_t>(r) * a.kv_heads + kvh) * a.head_dim;
    fp8_write_head((is_v ? a.v_base : a.k_base) + page, sl, kvh, src, a.head_dim, a.row_bytes,
                   a.data_bytes);
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
        // Rows of one launch must not share a page (they would race on its scale).
        for (size_t i = 0; i < a.num_rows; ++i)
            for (size_t j = 0; j < i; ++j)
                if (a.rows[i].page_offset == a.rows[j].page_offset) {
                    *err = "fp8 KV write: two rows of one call target the same page";
                    return false;
                }
        for (size_t base = 0; base < a.num_rows; base += kRowsPerLaunch) {
            const size_t n = std::min<size_t>(kRowsPerLaunch, a.num_rows - base);
            Fp8RowBatch rb{};
            for (size_t i = 0; i < n; ++i) {
                rb.page[i] = a.rows[base + i].page_offset;
                rb.slot[i] = a.rows[base + i].slot;
                rb.src[i] = a.rows[base + i].src_row;
            }
            hipLaunchKernelGGL(kv_rows_fp8, dim3(n, a.kv_heads, 2), dim3(64), 0, s, rb, kb, vb,
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
        hipLaunchKernelGGL(kv_slots_fp8, dim3(a.batch, a.kv_heads, 2), dim3(64), 0, s, sa);
    } else {
        hipLaunchKernelGGL(kv_slots_copy, dim3(a.batch), dim3(256), 0, s, sa);
    }
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

}  // namespace dev
}  // namespace kcmm
