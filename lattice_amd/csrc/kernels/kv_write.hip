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
// fp8-e4m3 pools take bf16 source rows and quantize per (page, kv head) with
// one fp32 scale in the page footer.  The rows one call writes into a page
// are applied as a set (the call's last row for each slot), so the result
// does not depend on their order: a call that writes slot 0 starts the page
// with scale amax/448 over its rows (1 if all zero); a later call raises the
// scale to amax/448 when its rows exceed 448*scale and re-encodes every slot
// it does not write, so no value is ever clipped (fp8_write_page_head).
// Encoding is round-to-nearest-even with saturation to +-448.
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

// fp8 page write of one (page, kv head) for one call.  `row_of` (bs entries,
// LDS) gives, for each token slot, the source row this call writes there (the
// call's last row for that slot), or -1.  The rows a call writes into a page
// are applied as one set, so the bytes do not depend on their order:
//   amax  = max |x| over the written rows of this kv head;
//   fresh = the call writes slot 0, or the footer scale is not a finite
//           positive number (a page never started);
//   fresh:  scale = amax / 448 (1 for amax 0); the slots the call does not
//           write are left as they are and are undefined from then on;
//   else:   scale = old, raised to amax / 448 when amax > 448 * old, and then
//           every slot the call does not write is re-encoded from old to the
//           new scale (e4m3(decode(code) * old / scale));
// and each written row is stored as e4m3(x / scale).  One wavefront.
__device__ void fp8_write_page_head(uint8_t* page, uint32_t kvh, const uint16_t* src_base,
                                    const int32_t* row_of, uint32_t bs, uint32_t kv_heads,
                                    uint32_t head_dim, uint32_t row_bytes, uint32_t data_bytes) {
    const int lane = threadIdx.x & 63;
    float* sp = reinterpret_cast<float*>(page + data_bytes) + kvh;
    const float old = *sp;
    float amax = 0.0f;
    for (uint32_t u = 0; u < bs; ++u) {
        const int32_t r = row_of[u];
        if (r < 0) continue;
        const uint16_t* src = src_base + (static_cast<uint64_t>(r) * kv_heads + kvh) * head_dim;
#pragma unroll
        for (int i = 0; i < 4; ++i) {   // head_dim <= 256
            const uint32_t d = lane + 64 * i;
            if (d < head_dim) amax = fmaxf(amax, fabsf(bf16_bits_to_f32(src[d])));
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const bool fresh = row_of[0] >= 0 || !(old > 0.0f && old <= 3.40282347e38f);
    float scale;
    if (fresh) {
        scale = amax > 0.0f ? amax / 448.0f : 1.0f;
    } else {
        scale = old;
        if (amax > 448.0f * old) {
            scale = amax / 448.0f;
            if ((head_dim & 15) == 0 && (row_bytes & 15) == 0) {
                // 16-byte pieces of all unwritten slots at once: one memory
                // round trip for the page instead of one per slot
                const uint32_t pieces = head_dim / 16;
                for (uint32_t c = lane; c < bs * pieces; c += 64) {
                    const uint32_t u = c / pieces;
                    if (row_of[u] >= 0) continue;
                    u32x4* q = reinterpret_cast<u32x4*>(page + static_cast<uint64_t>(u) * row_bytes +
                                                        kvh * head_dim + (c - u * pieces) * 16);
                    u32x4 v = *q;
#pragma unroll
                    for (int w = 0; w < 4; ++w) {
                        uint32_t o = 0;
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const float y = fp8e4m3_to_f32((v[w] >> (8 * b)) & 0xffu) * old;
                            o |= f32_to_fp8e4m3(y / scale) << (8 * b);
                        }
                        v[w] = o;
                    }
                    *q = v;
                }
            } else {
                for (uint32_t u = 0; u < bs; ++u) {
                    if (row_of[u] >= 0) continue;
                    uint8_t* row = page + static_cast<uint64_t>(u) * row_bytes + kvh * head_dim;
                    for (uint32_t d = lane; d < head_dim; d += 64) {
                        const float y = fp8e4m3_to_f32(row[d]) * old;
                        row[d] = static_cast<uint8_t>(f32_to_fp8e4m3(y / scale));
                    }
                }
            }
        }
    }
    for (uint32_t u = 0; u < bs; ++u) {
        const int32_t r = row_of[u];
        if (r < 0) continue;
        const uint16_t* src = src_base + (static_cast<uint64_t>(r) * kv_heads + kvh) * head_dim;
        uint8_t* row = page + static_cast<uint64_t>(u) * row_bytes + kvh * head_dim;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t d = lane + 64 * i;
            if (d < head_dim)
                row[d] = static_cast<uint8_t>(f32_to_fp8e4m3(bf16_bits_to_f32(src[d]) / scale));
        }
    }
    if (lane == 0) *sp = scale;
}

// Host-resolved fp8 rows grouped by page: rows start[g] .. start[g+1]-1 of the
// batch target one page, in call order.  A page's rows never span launches.
struct Fp8RowBatch {
    uint64_t page[kRowsPerLaunch];
    uint32_t slot[kRowsPerLaunch];
    uint32_t src[kRowsPerLaunch];
    uint16_t start[kRowsPerLaunch + 1];
};

// Waves per fp8 writer workgroup: one per (kv head, K|V) pair, at most 16.
constexpr int kFp8MaxWaves = 16;
// Token slots per page the fp8 writer handles (its slot table lives in LDS).
constexpr uint32_t kFp8MaxBlockSize = 4096;

// grid (groups), dynamic LDS bs * 4 bytes; wave w takes the (kv head, K|V)
// pairs w, w + waves, ...
__global__ __launch_bounds__(64 * kFp8MaxWaves) void kv_rows_fp8(
    Fp8RowBatch rb, uint8_t* k_base, uint8_t* v_base, const uint16_t* k_src,
    const uint16_t* v_src, uint32_t bs, uint32_t kv_heads, uint32_t head_dim, uint32_t row_bytes,
    uint32_t data_bytes) {
    extern __shared__ int32_t row_of[];
    const uint32_t g = blockIdx.x;
    const uint32_t r0 = rb.start[g], r1 = rb.start[g + 1];
    for (uint32_t u = threadIdx.x; u < bs; u += blockDim.x) row_of[u] = -1;
    __syncthreads();
    if (threadIdx.x == 0)
        for (uint32_t r = r0; r < r1; ++r) row_of[rb.slot[r]] = static_cast<int32_t>(rb.src[r]);
    __syncthreads();
    const uint32_t waves = blockDim.x >> 6;
    for (uint32_t j = threadIdx.x >> 6; j < 2 * kv_heads; j += waves) {
        const bool is_v = j & 1;
        fp8_write_page_head((is_v ? v_base : k_base) + rb.page[r0], j >> 1, is_v ? v_src : k_src,
                            row_of, bs, kv_heads, head_dim, row_bytes, data_bytes);
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

// fp8 pages through device slot ids, in two kernels so that all rows of a
// page are applied as one set by one workgroup (fp8_write_page_head).
// `lead` / `cnt` (int32 per block id, zero between calls) collect, per page,
// batch - (first row) and the number of rows.  Pass 1: one thread per row
// resolves the slot (status as above) and enters the row; pass 2: the
// workgroup of a page's first row builds the page's slot table in LDS (rows
// in call order, so the last row for a slot wins), writes the page, then
// restores both entries to zero.
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

// grid (batch); 64 * min(2 kv_heads, 16) threads; dynamic LDS block_size * 4.
__global__ __launch_bounds__(64 * kFp8MaxWaves) void kv_slots_fp8_write(SlotArgs a,
                                                                         uint32_t batch,
                                                                         int32_t* lead,
                                                                         int32_t* cnt) {
    extern __shared__ int32_t row_of[];
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
    for (uint32_t u = threadIdx.x; u < a.block_size; u += blockDim.x) row_of[u] = -1;
    __syncthreads();
    const int32_t rows = s_rows;
    if (rows == 0) return;
    const int lane = threadIdx.x & 63;
    if (rows == 1) {
        // the page's only row is this one (the common decode append)
        if (threadIdx.x == 0)
            row_of[static_cast<uint32_t>(slot % a.block_size)] = static_cast<int32_t>(r);
    } else if (threadIdx.x < 64) {
        // rows of this page, in call order, from this one on
        int32_t done = 0;
        for (uint32_t base = r; done < rows && base < batch; base += 64) {
            const uint32_t rr = base + lane;
            const int64_t s2 = rr < batch ? a.slots[rr] : -1;
            uint64_t mask = __ballot(s2 >= 0 && s2 / a.block_size == id);
            while (mask != 0 && done < rows) {
                const int i = __builtin_ctzll(mask);
                mask &= mask - 1;
                const uint32_t row = base + i;
                if (lane == 0)
                    row_of[static_cast<uint32_t>(a.slots[row] % a.block_size)] =
                        static_cast<int32_t>(row);
                ++done;
            }
        }
    }
    __syncthreads();
    const uint64_t page_off = a.offsets_f16[id] * 2ull;
    const uint32_t waves = blockDim.x >> 6;
    for (uint32_t j = threadIdx.x >> 6; j < 2 * a.kv_heads; j += waves) {
        const bool is_v = j & 1;
        fp8_write_page_head((is_v ? a.v_base : a.k_base) + page_off, j >> 1,
                            reinterpret_cast<const uint16_t*>(is_v ? a.v_src : a.k_src), row_of,
                            a.block_size, a.kv_heads, a.head_dim, a.row_bytes, a.data_bytes);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        lead[id] = 0;
        cnt[id] = 0;
    }
}

}  // namespace

namespace dev {

// Row indices sorted by (page, slot), keeping only the last row of the call
// for each (page, slot): a call that names a slot twice stores its last row
// there, as the reference's sequential row copies do (ref pool.rs:1084-1091).
static std::vector<uint32_t> last_row_per_slot(const RowDst* rows, size_t n) {
    std::vector<uint32_t> order(n);
    for (size_t i = 0; i < n; ++i) order[i] = static_cast<uint32_t>(i);
    std::sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) {
        if (rows[x].page_offset != rows[y].page_offset)
            return rows[x].page_offset < rows[y].page_offset;
        if (rows[x].slot != rows[y].slot) return rows[x].slot < rows[y].slot;
        return x < y;
    });
    size_t m = 0;
    for (size_t i = 0; i < n; ++i) {
        const bool superseded = i + 1 < n && rows[order[i]].page_offset == rows[order[i + 1]].page_offset &&
                                rows[order[i]].slot == rows[order[i + 1]].slot;
        if (!superseded) order[m++] = order[i];
    }
    order.resize(m);
    return order;
}

bool kv_write_rows(const KvRowsArgs& a, std::string* err) {
    hipStream_t s = reinterpret_cast<hipStream_t>(a.stream);
    auto* kb = reinterpret_cast<uint8_t*>(a.k_base);
    auto* vb = reinterpret_cast<uint8_t*>(a.v_base);
    const std::vector<uint32_t> order = last_row_per_slot(a.rows, a.num_rows);
    const size_t num = order.size();
    if (a.dtype == kDtFP8) {
        if (a.head_dim > 256) {
            *err = "fp8 KV write supports head_dim <= 256";
            return false;
        }
        if (a.block_size == 0 || a.block_size > kFp8MaxBlockSize) {
            *err = "fp8 KV write supports block_size <= 4096";
            return false;
        }
        // One workgroup per page; a page's rows (distinct slots) go to one
        // launch, whole groups packed kRowsPerLaunch rows at a time.
        const int waves = static_cast<int>(std::min<uint32_t>(2 * a.kv_heads, kFp8MaxWaves));
        const size_t lds = static_cast<size_t>(a.block_size) * 4;
        size_t i = 0;
        while (i < num) {
            Fp8RowBatch rb{};
            uint32_t groups = 0, n = 0;
            while (i < num) {
                size_t j = i;
                while (j < num && a.rows[order[j]].page_offset == a.rows[order[i]].page_offset) ++j;
                if (j - i > static_cast<size_t>(kRowsPerLaunch)) {
                    *err = "fp8 KV write: more than 64 rows into one page in one call";
                    return false;
                }
                if (n + (j - i) > static_cast<size_t>(kRowsPerLaunch)) break;
                rb.start[groups++] = static_cast<uint16_t>(n);
                for (; i < j; ++i, ++n) {
                    const RowDst& r = a.rows[order[i]];
                    rb.page[n] = r.page_offset;
                    rb.slot[n] = r.slot;
                    rb.src[n] = r.src_row;
                }
            }
            rb.start[groups] = static_cast<uint16_t>(n);
            hipLaunchKernelGGL(kv_rows_fp8, dim3(groups), dim3(64 * waves), lds, s, rb, kb, vb,
                               reinterpret_cast<const uint16_t*>(a.k_src),
                               reinterpret_cast<const uint16_t*>(a.v_src), a.block_size,
                               a.kv_heads, a.head_dim, a.row_bytes, a.data_bytes);
            KCMM_HIP_CHECK(hipGetLastError(), err);
        }
        return true;
    }
    for (size_t base = 0; base < num; base += kRowsPerLaunch) {
        const size_t n = std::min<size_t>(kRowsPerLaunch, num - base);
        RowBatch rb{};
        for (size_t i = 0; i < n; ++i) {
            const RowDst& r = a.rows[order[base + i]];
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
        if (a.block_size == 0 || a.block_size > kFp8MaxBlockSize) {
            *err = "fp8 KV write supports block_size <= 4096";
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
        hipLaunchKernelGGL(kv_slots_fp8_write, dim3(a.batch), dim3(64 * waves),
                           static_cast<size_t>(a.block_size) * 4, s, sa, a.batch, lead, cnt);
    } else {
        hipLaunchKernelGGL(kv_slots_copy, dim3(a.batch), dim3(256), 0, s, sa);
    }
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

}  // namespace dev
}  // namespace kcmm
