// Shared device helpers for the gfx950 kernels: vector types, element
// conversions, HIP error plumbing.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace kcmm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Element codes shared with PoolGeometry::dtype.
constexpr int kDtF16 = 0;
constexpr int kDtBF16 = 1;
constexpr int kDtFP8 = 2;
constexpr int kDtF32 = 3;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// fp32 -> IEEE half, round to nearest even (hardware conversion).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT>
__device__ __forceinline__ float elem_to_f32(uint32_t bits) {
    if constexpr (DT == kDtF16) return f16_bits_to_f32(bits);
    else return bf16_bits_to_f32(bits);
}

template <int DT>
__device__ __forceinline__ uint32_t f32_to_elem(float f) {
    if constexpr (DT == kDtF16) return f32_to_f16_bits(f);
    else return f32_to_bf16_bits(f);
}

// OCP e4m3fn decode: 1 sign, 4 exponent (bias 7), 3 mantissa bits; the only
// NaN codes are S.1111.111; no infinities.
__device__ __forceinline__ float fp8e4m3_to_f32(uint32_t b) {
    const uint32_t s = (b & 0x80u) << 24;
    const uint32_t e = (b >> 3) & 0xFu;
    const uint32_t m = b & 0x7u;
    if (e == 0xFu && m == 0x7u) return __uint_as_float(s | 0x7fc00000u);
    if (e == 0) {
        // subnormal: m * 2^-9
        return __uint_as_float(s) + (s ? -1.0f : 1.0f) * static_cast<float>(m) * 0.001953125f;
    }
    return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

// q / out rows of the attention kernels: f16 for f16 pools, fp32 for fp32
// pools, bf16 otherwise (bf16 and fp8 pools).  Element i of a row at `row`.
template <int DT>
__device__ __forceinline__ float io_load(const uint8_t* row, int i) {
    if constexpr (DT == kDtF32) return reinterpret_cast<const float*>(row)[i];
    else if constexpr (DT == kDtF16) return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(row)[i]);
    else return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(row)[i]);
}
template <int DT>
__device__ __forceinline__ void io_store(uint8_t* row, int i, float v) {
    if constexpr (DT == kDtF32) reinterpret_cast<float*>(row)[i] = v;
    else if constexpr (DT == kDtF16) reinterpret_cast<uint16_t*>(row)[i] = static_cast<uint16_t>(f32_to_f16_bits(v));
    else reinterpret_cast<uint16_t*>(row)[i] = static_cast<uint16_t>(f32_to_bf16_bits(v));
}
template <int DT>
constexpr int io_bytes() { return DT == kDtF32 ? 4 : 2; }
// Bytes of one K/V element in a page of type DT.
template <int DT>
constexpr int kv_elem_bytes() { return DT == kDtFP8 ? 1 : (DT == kDtF32 ? 4 : 2); }
// exp for the any-shape kernels: correctly rounded-ish expf for fp32 pools
// (their tolerance is 1e-5), the hardware exp2 path otherwise.
template <int DT>
__device__ __forceinline__ float kexp(float x) {
    if constexpr (DT == kDtF32) return expf(x);
    else return __expf(x);
}

__device__ __forceinline__ float bf16_round_f32(float f) {
    return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

// Decoder-layer element arithmetic shared by the standalone glue kernels and
// the GEMM epilogues that fuse them, so both give identical bits.
//  * RoPE of one rotate-half pair (x1 = element i, x2 = element i + D/2):
//    x1' = x1 c - x2 s, x2' = x2 c + x1 s, with c, s of pos * inv_freq[i];
//  * SwiGLU: bf16(bf16(silu(g)) * u), the roundings of a bf16 model.
__device__ __forceinline__ void rope_cos_sin(int pos, float inv_freq, float* c, float* s) {
    const float ang = static_cast<float>(pos) * inv_freq;
    *c = cosf(ang);
    *s = sinf(ang);
}
__device__ __forceinline__ float rope_first(float x1, float x2, float c, float s) {
    return __builtin_fmaf(x1, c, -(x2 * s));
}
__device__ __forceinline__ float rope_second(float x1, float x2, float c, float s) {
    return __builtin_fmaf(x2, c, x1 * s);
}
__device__ __forceinline__ float swiglu_bf16(float g, float u) {
    const float sg = bf16_round_f32(g / (1.0f + __expf(-g)));
    return bf16_round_f32(sg * u);
}

}  // namespace kcmm

#define KCMM_HIP_CHECK(expr, errp)                                              \
    do {                                                                        \
        hipError_t e_ = (expr);                                                 \
        if (e_ != hipSuccess) {                                                 \
            (void)hipGetLastError(); /* do not leave the error for the caller */ \
            if (errp) *(errp) = std::string(#expr) + ": " + hipGetErrorString(e_); \
            return false;                                                       \
        }                                                                       \
    } while (0)
