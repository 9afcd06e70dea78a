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
//  * silu_mul: act = bf16(silu(gate) * up) over the fused [gate | up] row.
#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

__device__ __forceinline__ float bf16_round(float f) {
    return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

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

__device__ __forceinline__ float block_sum_256(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

// One row per workgroup; H % 8 == 0.
__global__ __launch_bounds__(256) void rmsnorm_rows(const uint16_t* __restrict__ x,
                                                    const uint16_t* __restrict__ w,
                                                    uint16_t* __restrict__ y, int H, float eps) {
    __shared__ float red[4];
    const uint16_t* xr = x + static_cast<size_t>(blockIdx.x) * H;
    uint16_t* yr = y + static_cast<size_t>(blockIdx.x) * H;
    float ss = 0.0f;
    for (int i = threadIdx.x * 8; i < H; i += 256 * 8) {
        float f[8];
        unpack8(*reinterpret_cast<const u32x4*>(xr + i), f);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
    }
    const float r = 1.0f / sqrtf(block_sum_256(ss, red) / static_cast<float>(H) + eps);
    for (int i = threadIdx.x * 8; i < H; i += 256 * 8) {
        float f[8], g[8];
        unpack8(*reinterpret_cast<const u32x4*>(xr + i), f);
        unpack8(*reinterpret_cast<const u32x4*>(w + i), g);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = g[j] * bf16_round(f[j] * r);
        *reinterpret_cast<u32x4*>(yr + i) = pack8(f);
    }
}

struct RopeAppendParams {
    const uint16_t* qkv;      // [B][(Hq + 2 Hkv) D]
    uint16_t* q_out;          // [B][Hq][D]
    uint8_t* k_base;
    uint8_t* v_base;
    const int32_t* block_tables;
    const int32_t* seq_lens;  // cached tokens including this step's (position = len - 1)
    const uint64_t* offsets_f16;
    const float* inv_freq;    // [D/2]
    int num_q_heads, kv_heads, head_dim, block_size, mbps, row_bytes;
};

// One workgroup per sequence.  Thread t takes quad iq = t % (D/8) of the
// D/2 rotation pairs (elements 4iq..4iq+3 and D/2 + 4iq..+3) of heads
// t / (D/8), + 256/(D/8), ...; its four (cos, sin) pairs serve every head.
__global__ __launch_bounds__(256) void rope_append_rows(RopeAppendParams p) {
    const int b = blockIdx.x;
    const int L = p.seq_lens[b];
    const int D = p.head_dim;
    const int pos = L - 1;
    if (pos < 0 || pos >= p.mbps * p.block_size) return;   // no token / past the table
    const int quads = D / 8;
    const int iq = threadIdx.x % quads;
    const int h0 = threadIdx.x / quads;
    const int hstep = 256 / quads;
    float cs[4], sn[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float ang = static_cast<float>(pos) * p.inv_freq[4 * iq + j];
        cs[j] = cosf(ang);
        sn[j] = sinf(ang);
    }
    const int lb = pos / p.block_size;
    const uint64_t page = p.offsets_f16[p.block_tables[static_cast<size_t>(b) * p.mbps + lb]] * 2ull +
                          static_cast<uint64_t>(pos - lb * p.block_size) * p.row_bytes;
    const int stride = (p.num_q_heads + 2 * p.kv_heads) * D;
    const uint16_t* row = p.qkv + static_cast<size_t>(b) * stride;
    auto rotate = [&](const uint16_t* src, uint16_t* dst) {
        const u32x2 a = *reinterpret_cast<const u32x2*>(src + 4 * iq);
        const u32x2 c = *reinterpret_cast<const u32x2*>(src + D / 2 + 4 * iq);
        float x1[4], x2[4];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            x1[2 * j] = __uint_as_float(a[j] << 16);
            x1[2 * j + 1] = __uint_as_float(a[j] & 0xffff0000u);
            x2[2 * j] = __uint_as_float(c[j] << 16);
            x2[2 * j + 1] = __uint_as_float(c[j] & 0xffff0000u);
        }
        u32x2 o1, o2;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float y0 = x1[2 * j] * cs[2 * j] - x2[2 * j] * sn[2 * j];
            const float y1 = x1[2 * j + 1] * cs[2 * j + 1] - x2[2 * j + 1] * sn[2 * j + 1];
            const float z0 = x2[2 * j] * cs[2 * j] + x1[2 * j] * sn[2 * j];
            const float z1 = x2[2 * j + 1] * cs[2 * j + 1] + x1[2 * j + 1] * sn[2 * j + 1];
            o1[j] = f32_to_bf16_bits(y0) | (f32_to_bf16_bits(y1) << 16);
            o2[j] = f32_to_bf16_bits(z0) | (f32_to_bf16_bits(z1) << 16);
        }
        *reinterpret_cast<u32x2*>(dst + 4 * iq) = o1;
        *reinterpret_cast<u32x2*>(dst + D / 2 + 4 * iq) = o2;
    };
    const int hq_end = h0 < hstep ? p.num_q_heads : 0;   // (threads past whole head groups idle)
    const int hk_end = h0 < hstep ? p.kv_heads : 0;
    for (int h = h0; h < hq_end; h += hstep)
        rotate(row + h * D, p.q_out + (static_cast<size_t>(b) * p.num_q_heads + h) * D);
    for (int h = h0; h < hk_end; h += hstep)
        rotate(row + (p.num_q_heads + h) * D,
               reinterpret_cast<uint16_t*>(p.k_base + page + static_cast<uint64_t>(h) * D * 2));
    // v: plain copy of the kv_heads x D row (8 bytes per thread and step)
    const uint16_t* vsrc = row + (p.num_q_heads + p.kv_heads) * D;
    uint16_t* vdst = reinterpret_cast<uint16_t*>(p.v_base + page);
    for (int e = threadIdx.x * 4; e < p.kv_heads * D; e += 256 * 4)
        *reinterpret_cast<u32x2*>(vdst + e) = *reinterpret_cast<const u32x2*>(vsrc + e);
}

// act[m][j] = bf16(silu(gu[m][j]) * gu[m][I + j]); 8 elements per thread.
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
    for (int e = 0; e < 8; ++e) g[e] = g[e] / (1.0f + __expf(-g[e])) * u[e];
    *reinterpret_cast<u32x4*>(act + idx) = pack8(g);
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
    hipLaunchKernelGGL(rmsnorm_rows, dim3(rows), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       reinterpret_cast<const uint16_t*>(x), reinterpret_cast<const uint16_t*>(w),
                       reinterpret_cast<uint16_t*>(y), static_cast<int>(hidden), eps);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

bool rope_append_bf16(const RopeAppendArgs& a, std::string* err) {
    if (a.batch == 0) return true;
    if (a.head_dim % 8 != 0 || a.head_dim > 2048) {
        *err = "rope_append: head_dim must be a multiple of 8 (<= 2048)";
        return false;
    }
    RopeAppendParams p{};
    p.qkv = reinterpret_cast<const uint16_t*>(a.qkv);
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
    hipLaunchKernelGGL(rope_append_rows, dim3(a.batch), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(a.stream), p);
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
