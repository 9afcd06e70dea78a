// Decode-step glue kernels for gfx950: the element-wise and row-wise steps of
// one Llama decoder layer around the GEMMs and the paged attention (ref
// src/model/llama_transformer.rs:262-391, whose CUDA helpers are
// rms_norm.cu, rope.cu, silu_mul.cu and add.cu; the semantics here are the
// Hugging Face Llama ones, because the reference's RoPE pairs and theta are
// not HF's).  bf16 in and out, fp32 arithmetic.
//
//  * rmsnorm: y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), one workgroup
//    per row (HF LlamaRMSNorm rounds the normalised row to the input type
//    before the weight multiply);
//  * rope_append: one workgroup per sequence's new token.  q of the fused
//    QKV row is rotated into the contiguous q buffer the attention reads; k
//    is rotated and written with v straight into the token's page row
//    (reshape-and-cache fused with RoPE: the rotated k never makes a round
//    trip through HBM).  HF rotate_half pairing (i, i + D/2), angle =
//    pos * inv_freq[i], inv_freq supplied by the caller so that any HF
//    rope_type is served;
//  * silu_mul: act = bf16(bf16(silu(gate)) * up) over the fused [gate | up]
//    row (F.silu on a bf16 tensor rounds before the multiply).
#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

// 8 bf16 <-> 8 floats
__device__ __forceinline__ void unpack8(const u32x4& v, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(v[i] << 16);
        f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = f32_to_bf16_bits(f[2 * i]) | (f32_to_bf16_bits(f[2 * i + 1]) << 16);
    return v;
}

// Sum over the NT threads of the workgroup, waves added in order (the same
// order for every row and kernel variant).
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) s += red[w];
    return s;
}

// Sum of the `splits` fp32 partials at pp, pp + MN, ... in split order; up
// to W splits' loads are in flight together (indices past the last split
// re-read it and are not added: no branch around a load).
template <int W>
__device__ __forceinline__ f32x4 sum_partials_w(const float* pp, size_t MN, int splits) {
    f32x4 s = f32x4{0, 0, 0, 0};
    for (int k0 = 0; k0 < splits; k0 += W) {
        f32x4 v[W];
#pragma unroll
        for (int k = 0; k < W; ++k)
            v[k] = *reinterpret_cast<const f32x4*>(pp + static_cast<size_t>(min(k0 + k, splits - 1)) * MN);
#pragma unroll
        for (int k = 0; k < W; ++k)
            if (k0 + k < splits) s += v[k];
    }
    return s;
}
// Four-wide when every split fits in one round (the GEMM plans at most 4 at
// the decode shapes), so no load is spent re-reading the last split.
__device__ __forceinline__ f32x4 sum_partials(const float* pp, size_t MN, int splits) {
    return splits <= 4 ? sum_partials_w<4>(pp, MN, splits) : sum_partials_w<8>(pp, MN, splits);
}

// One row per workgroup; H % 8 == 0.  FROM_PARTIALS: the row is first
// finished as the O projection's residual add -- x = bf16(x + bf16(sum of
// the `splits` fp32 partials [s][rows][H])) -- and written back to x (the
// hidden state), exactly what the GEMM's residual store would have written.
template <bool FROM_PARTIALS, int NT>
__global__ __launch_bounds__(NT) void rmsnorm_rows(uint16_t* __restrict__ x,
                                                   const uint16_t* __restrict__ w,
                                                   uint16_t* __restrict__ y, int H, float eps,
                                                   const float* __restrict__ part, int splits) {
    __shared__ float red[NT / 64];
    uint16_t* xr = x + static_cast<size_t>(blockIdx.x) * H;
    uint16_t* yr = y + static_cast<size_t>(blockIdx.x) * H;
    if (H <= NT * 8) {
        // one 8-element piece per thread (the launcher's choice up to H =
        // 8192): the weights are loaded with the row, and the finished row
        // stays in registers across the reduction, so the kernel makes one
        // memory round trip instead of two
        const int i = threadIdx.x * 8;
        const bool mine = i < H;
        const int ic = mine ? i : 0;   // idle threads read piece 0 and store nothing
        float f[8], g[8];
        unpack8(*reinterpret_cast<const u32x4*>(xr + ic), f);
        unpack8(*reinterpret_cast<const u32x4*>(w + ic), g);
        if constexpr (FROM_PARTIALS) {
            const size_t MN = static_cast<size_t>(gridDim.x) * H;
            const float* pp = part + static_cast<size_t>(blockIdx.x) * H + ic;
            const f32x4 s0 = sum_partials(pp, MN, splits);
            const f32x4 s1 = sum_partials(pp + 4, MN, splits);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f[j] = bf16_round_f32(bf16_round_f32(s0[j]) + f[j]);
                f[4 + j] = bf16_round_f32(bf16_round_f32(s1[j]) + f[4 + j]);
            }
            if (mine) *reinterpret_cast<u32x4*>(xr + i) = pack8(f);
        }
        float ss = 0.0f;
        if (mine) {
#pragma unroll
            for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
        }
        const float r = 1.0f / sqrtf(block_sum<NT>(ss, red) / static_cast<float>(H) + eps);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = g[j] * bf16_round_f32(f[j] * r);
        if (mine) *reinterpret_cast<u32x4*>(yr + i) = pack8(f);
        return;
    }
    float ss = 0.0f;
    for (int i = threadIdx.x * 8; i < H; i += NT * 8) {
        float f[8];
        unpack8(*reinterpret_cast<const u32x4*>(xr + i), f);
        if constexpr (FROM_PARTIALS) {
            const size_t MN = static_cast<size_t>(gridDim.x) * H;
            const float* pp = part + static_cast<size_t>(blockIdx.x) * H + i;
            const f32x4 s0 = sum_partials(pp, MN, splits);
            const f32x4 s1 = sum_partials(pp + 4, MN, splits);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f[j] = bf16_round_f32(bf16_round_f32(s0[j]) + f[j]);
                f[4 + j] = bf16_round_f32(bf16_round_f32(s1[j]) + f[4 + j]);
            }
            *reinterpret_cast<u32x4*>(xr + i) = pack8(f);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
    }
    const float r = 1.0f / sqrtf(block_sum<NT>(ss, red) / static_cast<float>(H) + eps);
    for (int i = threadIdx.x * 8; i < H; i += NT * 8) {
        float f[8], g[8];
        unpack8(*reinterpret_cast<const u32x4*>(xr + i), f);   // (this thread's own writes)
        unpack8(*reinterpret_cast<const u32x4*>(w + i), g);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = g[j] * bf16_round_f32(f[j] * r);
        *reinterpret_cast<u32x4*>(yr + i) = pack8(f);
    }
}

struct RopeAppendParams {
    const uint16_t* qkv;      // [B][(Hq + 2 Hkv) D] (bf16 source)
    const float* part;        // [splits][B][(Hq + 2 Hkv) D] (fp32 partials source)
    int splits;
    uint16_t* q_out;          // [B][Hq][D]
    uint8_t* k_base;
    uint8_t* v_base;
    const int32_t* block_tables;
    const int32_t* seq_lens;  // cached tokens including this step's (position = len - 1)
    const uint64_t* offsets_f16;
    const float* inv_freq;    // [D/2]
    int num_q_heads, kv_heads, head_dim, block_size, mbps, row_bytes;
    // fp8 pages: k / v rows go to bf16 staging [B][Hkv D] and each
    // sequence's slot id (page * block_size + offset, -1 when skipped) to
    // slots, for the fp8 page writer (null: rows go straight into the pages)
    uint16_t* k_stage;
    uint16_t* v_stage;
    int64_t* slots;
};

// Workgroup (b, y) handles heads [y*hs, (y+1)*hs) of sequence b's qkv row,
// hs = 256 / (D/8): thread t takes quad iq = t % (D/8) of the D/2 rotation
// pairs (elements 4iq..4iq+3 and D/2 + 4iq..+3) of head y*hs + t / (D/8).
// q and k heads are rotated (into q_out / the token's K page row), v heads
// copied into the V page row.  FROM_PARTIALS: the qkv row is the split-order
// sum of the QKV projection's fp32 partials, rounded to bf16 (what the
// projection's own store writes).
template <bool FROM_PARTIALS>
__global__ __launch_bounds__(256) void rope_append_rows(RopeAppendParams p) {
    const int b = blockIdx.x;
    const int D = p.head_dim;
    const int quads = D / 8;
    const int hs = 256 / quads;
    const int iq = threadIdx.x % quads;
    const int hl = threadIdx.x / quads;
    const int heads = p.num_q_heads + 2 * p.kv_heads;
    // threads past whole heads load head 0's elements and store nothing
    const bool live = hl < hs && blockIdx.y * hs + hl < heads;
    const int h = live ? blockIdx.y * hs + hl : 0;
    const int stride = heads * D;
    const int e1 = h * D + 4 * iq, e2 = e1 + D / 2;
    // The row's elements and the rotation frequencies do not depend on the
    // sequence length: they are loaded before it, so only the K / V page
    // lookup (block table, then page offset) waits for seq_lens.
    float fr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) fr[j] = p.inv_freq[4 * iq + j];
    // elements e..e+3 of the row (as bf16 values)
    float x1[4], x2[4];
    if constexpr (FROM_PARTIALS) {
        const size_t MN = static_cast<size_t>(gridDim.x) * stride;
        const float* row = p.part + static_cast<size_t>(b) * stride;
        const f32x4 s1 = sum_partials(row + e1, MN, p.splits);
        const f32x4 s2 = sum_partials(row + e2, MN, p.splits);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x1[j] = bf16_round_f32(s1[j]);
            x2[j] = bf16_round_f32(s2[j]);
        }
    } else {
        const uint16_t* row = p.qkv + static_cast<size_t>(b) * stride;
        const u32x2 a = *reinterpret_cast<const u32x2*>(row + e1);
        const u32x2 c = *reinterpret_cast<const u32x2*>(row + e2);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            x1[2 * j] = __uint_as_float(a[j] << 16);
            x1[2 * j + 1] = __uint_as_float(a[j] & 0xffff0000u);
            x2[2 * j] = __uint_as_float(c[j] << 16);
            x2[2 * j + 1] = __uint_as_float(c[j] & 0xffff0000u);
        }
    }
    const int L = p.seq_lens[b];
    const int pos = L - 1;
    const bool has_row = pos >= 0 && pos < p.mbps * p.block_size;   // no token / past the table
    if (p.slots != nullptr && blockIdx.y == 0 && threadIdx.x == 0)
        p.slots[b] = has_row ? static_cast<int64_t>(p.block_tables[static_cast<size_t>(b) * p.mbps +
                                                                   pos / p.block_size]) *
                                       p.block_size +
                                   pos % p.block_size
                             : -1;
    if (!has_row || !live) return;
    float y1[4], y2[4];
    if (h < p.num_q_heads + p.kv_heads) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float cs, sn;
            rope_cos_sin(pos, fr[j], &cs, &sn);
            y1[j] = rope_first(x1[j], x2[j], cs, sn);
            y2[j] = rope_second(x1[j], x2[j], cs, sn);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            y1[j] = x1[j];
            y2[j] = x2[j];
        }
    }
    uint16_t* dst;
    if (h < p.num_q_heads) {
        dst = p.q_out + (static_cast<size_t>(b) * p.num_q_heads + h) * D;
    } else if (p.k_stage != nullptr) {
        const bool is_k = h < p.num_q_heads + p.kv_heads;
        const int kvh = is_k ? h - p.num_q_heads : h - p.num_q_heads - p.kv_heads;
        dst = (is_k ? p.k_stage : p.v_stage) + (static_cast<size_t>(b) * p.kv_heads + kvh) * D;
    } else {
        const int lb = pos / p.block_size;
        const uint64_t page = p.offsets_f16[p.block_tables[static_cast<size_t>(b) * p.mbps + lb]] * 2ull +
                              static_cast<uint64_t>(pos - lb * p.block_size) * p.row_bytes;
        const bool is_k = h < p.num_q_heads + p.kv_heads;
        const int kvh = is_k ? h - p.num_q_heads : h - p.num_q_heads - p.kv_heads;
        dst = reinterpret_cast<uint16_t*>((is_k ? p.k_base : p.v_base) + page +
                                          static_cast<uint64_t>(kvh) * D * 2);
    }
    u32x2 o1, o2;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        o1[j] = f32_to_bf16_bits(y1[2 * j]) | (f32_to_bf16_bits(y1[2 * j + 1]) << 16);
        o2[j] = f32_to_bf16_bits(y2[2 * j]) | (f32_to_bf16_bits(y2[2 * j + 1]) << 16);
    }
    *reinterpret_cast<u32x2*>(dst + 4 * iq) = o1;
    *reinterpret_cast<u32x2*>(dst + D / 2 + 4 * iq) = o2;
}

// act[m][j] = bf16(bf16(silu(gu[m][j])) * gu[m][I + j]); 8 elements per thread.
__global__ __launch_bounds__(256) void silu_mul_rows(const uint16_t* __restrict__ gu,
                                                     uint16_t* __restrict__ act, int M, int I) {
    const size_t idx = (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
    if (idx >= static_cast<size_t>(M) * I) return;
    const size_t m = idx / I, j = idx - m * I;
    const uint16_t* row = gu + m * 2 * I;
    float g[8], u[8];
    unpack8(*reinterpret_cast<const u32x4*>(row + j), g);
    unpack8(*reinterpret_cast<const u32x4*>(row + I + j), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = swiglu_bf16(g[e], u[e]);
    *reinterpret_cast<u32x4*>(act + idx) = pack8(g);
}

// Workgroup size by row length: one 8-element piece per thread when H <=
// 8192 (every load of a row in flight at once); the same choice for both
// variants, so they reduce in the same order.
template <bool FROM_PARTIALS>
void launch_rmsnorm(uint16_t* x, const uint16_t* w, uint16_t* y, uint32_t rows, uint32_t H,
                    float eps, const float* part, int splits, uint64_t stream) {
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int h = static_cast<int>(H);
    if (H > 4096)
        hipLaunchKernelGGL((rmsnorm_rows<FROM_PARTIALS, 1024>), dim3(rows), dim3(1024), 0, s, x, w, y,
                           h, eps, part, splits);
    else if (H > 2048)
        hipLaunchKernelGGL((rmsnorm_rows<FROM_PARTIALS, 512>), dim3(rows), dim3(512), 0, s, x, w, y,
                           h, eps, part, splits);
    else
        hipLaunchKernelGGL((rmsnorm_rows<FROM_PARTIALS, 256>), dim3(rows), dim3(256), 0, s, x, w, y,
                           h, eps, part, splits);
}

// hidden[b] = embed[ids[b]] (ref llama_transformer.rs:264-275 copies each
// token's row with its own driver memcpy); one workgroup per row, 16-byte
// pieces; an id outside [0, vocab) gives a zero row.
__global__ __launch_bounds__(256) void embed_rows(const uint8_t* __restrict__ embed,
                                                  const int32_t* __restrict__ ids,
                                                  uint8_t* __restrict__ hidden, uint32_t row_bytes,
                                                  uint32_t vocab) {
    const int b = blockIdx.x;
    const int32_t id = ids[b];
    const bool ok = id >= 0 && static_cast<uint32_t>(id) < vocab;
    const uint8_t* src = embed + static_cast<size_t>(ok ? id : 0) * row_bytes;
    uint8_t* dst = hidden + static_cast<size_t>(b) * row_bytes;
    for (uint32_t o = threadIdx.x * 16; o < row_bytes; o += 256 * 16)
        *reinterpret_cast<u32x4*>(dst + o) = ok ? *reinterpret_cast<const u32x4*>(src + o)
                                                : u32x4{0, 0, 0, 0};
}

}  // namespace

namespace dev {

bool rmsnorm_bf16(uint64_t x, uint64_t w, uint64_t y, uint32_t rows, uint32_t hidden, float eps,
                  uint64_t stream, std::string* err) {
    if (rows == 0) return true;
    if (hidden == 0 || hidden % 8 != 0) {
        *err = "rmsnorm: hidden size must be a positive multiple of 8";
        return false;
    }
    launch_rmsnorm<false>(reinterpret_cast<uint16_t*>(x), reinterpret_cast<const uint16_t*>(w),
                          reinterpret_cast<uint16_t*>(y), rows, hidden, eps, nullptr, 0, stream);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

bool residual_rmsnorm_from_partials(const float* part, int splits, uint64_t hidden, uint64_t w,
                                    uint64_t y, uint32_t rows, uint32_t H, float eps,
                                    uint64_t stream, std::string* err) {
    if (rows == 0) return true;
    if (H == 0 || H % 8 != 0 || splits < 1) {
        *err = "residual_rmsnorm: hidden size must be a positive multiple of 8";
        return false;
    }
    launch_rmsnorm<true>(reinterpret_cast<uint16_t*>(hidden), reinterpret_cast<const uint16_t*>(w),
                         reinterpret_cast<uint16_t*>(y), rows, H, eps, part, splits, stream);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

namespace {
bool launch_rope(const RopeAppendArgs& a, const float* part, int splits, std::string* err) {
    if (a.batch == 0) return true;
    if (a.head_dim % 8 != 0 || a.head_dim > 2048) {
        *err = "rope_append: head_dim must be a multiple of 8 (<= 2048)";
        return false;
    }
    RopeAppendParams p{};
    p.qkv = reinterpret_cast<const uint16_t*>(a.qkv);
    p.part = part;
    p.splits = splits;
    p.q_out = reinterpret_cast<uint16_t*>(a.q_out);
    p.k_base = reinterpret_cast<uint8_t*>(a.k_base);
    p.v_base = reinterpret_cast<uint8_t*>(a.v_base);
    p.block_tables = reinterpret_cast<const int32_t*>(a.block_tables);
    p.seq_lens = reinterpret_cast<const int32_t*>(a.seq_lens);
    p.offsets_f16 = reinterpret_cast<const uint64_t*>(a.offsets_f16);
    p.inv_freq = reinterpret_cast<const float*>(a.inv_freq);
    p.num_q_heads = static_cast<int>(a.num_q_heads);
    p.kv_heads = static_cast<int>(a.kv_heads);
    p.head_dim = static_cast<int>(a.head_dim);
    p.block_size = static_cast<int>(a.block_size);
    p.mbps = static_cast<int>(a.mbps);
    p.row_bytes = static_cast<int>(a.row_bytes);
    const bool fp8 = a.dtype == kDtFP8;
    uint64_t stage = 0;
    const size_t rows_bytes = static_cast<size_t>(a.batch) * a.kv_heads * a.head_dim * 2;
    if (fp8) {
        // fp8 pages: rotated k and v rows are staged in bf16, then written by
        // the fp8 page writer (per-page scales), which reads the slot ids
        void* ws = nullptr;
        if (!stream_workspace(a.stream, 7, 2 * rows_bytes + a.batch * sizeof(int64_t), &ws, false,
                              err))
            return false;
        stage = reinterpret_cast<uint64_t>(ws);
        p.k_stage = reinterpret_cast<uint16_t*>(stage);
        p.v_stage = reinterpret_cast<uint16_t*>(stage + rows_bytes);
        p.slots = reinterpret_cast<int64_t*>(stage + 2 * rows_bytes);
    }
    const uint32_t hs = 256 / (a.head_dim / 8);
    const dim3 grid(a.batch, (a.num_q_heads + 2 * a.kv_heads + hs - 1) / hs);
    if (part != nullptr)
        hipLaunchKernelGGL(rope_append_rows<true>, grid, dim3(256), 0,
                           reinterpret_cast<hipStream_t>(a.stream), p);
    else
        hipLaunchKernelGGL(rope_append_rows<false>, grid, dim3(256), 0,
                           reinterpret_cast<hipStream_t>(a.stream), p);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    if (fp8) {
        KvDeviceSlotsArgs w{};
        w.dtype = kDtFP8;
        w.k_base = a.k_base;
        w.v_base = a.v_base;
        w.k_src = stage;
        w.v_src = stage + rows_bytes;
        w.slot_mapping = stage + 2 * rows_bytes;
        w.offsets_f16 = a.offsets_f16;
        w.valid_blocks = 0;   // slots come from the block table
        w.status = 0;
        w.offsets_len = a.n_ids;
        w.batch = a.batch;
        w.block_size = a.block_size;
        w.kv_heads = a.kv_heads;
        w.head_dim = a.head_dim;
        w.row_bytes = a.row_bytes;
        w.data_bytes = a.data_bytes;
        w.stream = a.stream;
        if (!kv_write_device_slots(w, err)) return false;
    }
    return true;
}
}  // namespace

bool rope_append_bf16(const RopeAppendArgs& a, std::string* err) {
    return launch_rope(a, nullptr, 1, err);
}

bool rope_append_from_partials(const RopeAppendArgs& a, const float* part, int splits,
                               std::string* err) {
    return launch_rope(a, part, splits, err);
}

bool embed_bf16(uint64_t embed, uint64_t ids, uint64_t hidden, uint32_t batch, uint32_t hidden_size,
                uint32_t vocab, uint64_t stream, std::string* err) {
    if (batch == 0) return true;
    hipLaunchKernelGGL(embed_rows, dim3(batch), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       reinterpret_cast<const uint8_t*>(embed), reinterpret_cast<const int32_t*>(ids),
                       reinterpret_cast<uint8_t*>(hidden), hidden_size * 2u, vocab);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

bool silu_mul_bf16(uint64_t gate_up, uint64_t act, uint32_t rows, uint32_t inter,
                   uint64_t stream, std::string* err) {
    if (rows == 0) return true;
    if (inter == 0 || inter % 8 != 0) {
        *err = "silu_mul: intermediate size must be a positive multiple of 8";
        return false;
    }
    const size_t n = static_cast<size_t>(rows) * inter / 8;
    hipLaunchKernelGGL(silu_mul_rows, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream),
                       reinterpret_cast<const uint16_t*>(gate_up), reinterpret_cast<uint16_t*>(act),
                       static_cast<int>(rows), static_cast<int>(inter));
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

}  // namespace dev
}  // namespace kcmm
