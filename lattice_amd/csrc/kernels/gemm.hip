// Decode-step projection GEMM for gfx950: Y[M][N] = X[M][K] * W[N][K]^T,
// bf16 operands, fp32 accumulation, bf16 result (the HF Linear layout the
// reference's weights use, ref llama_transformer.rs:115-120; the reference
// hands this to cuBLAS, ref runtime.rs:17-41).
//
// At decode the token count M is small (64..256) and the weights dominate
// the bytes: at M = 64 the arithmetic intensity is ~62 flop/B, far below the
// MFMA ridge, so the kernel is a weight stream.  Layout:
//  * workgroup = 4 wavefronts = 64 weight rows (n) x 64 tokens (m) x one
//    K split; every wave owns 16 weight rows;
//  * weights go from HBM straight into MFMA A-operand registers (each lane a
//    16-byte run along k), never through LDS -- every weight byte is used by
//    exactly one wave;
//  * the activation tile (64 x 256 k) is staged in LDS once per k block and
//    shared by the four waves as the B operand of v_mfma_f32_16x16x32_bf16;
//  * K is split so the grid has enough workgroups to keep HBM busy; split
//    partials (fp32) are summed by a second small kernel.
#include <algorithm>
#include <cstdlib>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

constexpr int kBM = 64;    // tokens per workgroup
constexpr int kBN = 64;    // weight rows per workgroup
constexpr int kKB = 256;   // k block staged in LDS
constexpr int kXRow = kKB + 8;

__global__ __launch_bounds__(256) void gemm_bf16_skinny(const uint16_t* __restrict__ X,
                                                        const uint16_t* __restrict__ W,
                                                        uint16_t* __restrict__ Y,
                                                        float* __restrict__ part, int M, int N,
                                                        int K, int KR) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[kBM * kXRow];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 15, lg = lane >> 4;
    const int n0 = blockIdx.x * kBN + wave * 16;
    const int m0 = blockIdx.y * kBM;
    const int ks = blockIdx.z;
    const int kbeg = ks * KR;

    f32x4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = f32x4{0, 0, 0, 0};

    const uint16_t* wrow = W + static_cast<size_t>(n0 + ln) * K + kbeg + lg * 8;

    for (int kb = 0; kb < KR; kb += kKB) {
        // weight fragments of this k block: issued first so they are in flight
        // while the activation tile is staged
        u32x4 wa[kKB / 32];
#pragma unroll
        for (int s = 0; s < kKB / 32; ++s)
            wa[s] = *reinterpret_cast<const u32x4*>(wrow + kb + s * 32);

        __syncthreads();
#pragma unroll
        for (int i = tid; i < kBM * (kKB / 8); i += 256) {
            const int row = i / (kKB / 8);
            const int c = i - row * (kKB / 8);
            const int m = m0 + row;
            u32x4 v = u32x4{0, 0, 0, 0};
            if (m < M) v = *reinterpret_cast<const u32x4*>(X + static_cast<size_t>(m) * K + kbeg + kb + c * 8);
            *reinterpret_cast<u32x4*>(xs + row * kXRow + c * 8) = v;
        }
        __syncthreads();

#pragma unroll
        for (int s = 0; s < kKB / 32; ++s) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 b = *reinterpret_cast<const u32x4*>(xs + (16 * j + ln) * kXRow + s * 32 + lg * 8);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wa[s]),
                                                                 __builtin_bit_cast(bf16x8, b),
                                                                 acc[j], 0, 0, 0);
            }
        }
    }

    // acc[j][r] = Y[m0 + 16j + ln][n0 + 4lg + r]
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = m0 + 16 * j + ln;
        if (m >= M) continue;
        const int n = n0 + 4 * lg;
        if (part == nullptr) {
            u32x2 o;
            o[0] = f32_to_bf16_bits(acc[j][0]) | (f32_to_bf16_bits(acc[j][1]) << 16);
            o[1] = f32_to_bf16_bits(acc[j][2]) | (f32_to_bf16_bits(acc[j][3]) << 16);
            *reinterpret_cast<u32x2*>(Y + static_cast<size_t>(m) * N + n) = o;
        } else {
            *reinterpret_cast<f32x4*>(part + (static_cast<size_t>(ks) * M + m) * N + n) = acc[j];
        }
    }
}

// Y = bf16(sum over splits of the fp32 partials); 4 outputs per thread.
__global__ __launch_bounds__(256) void gemm_split_reduce(const float* __restrict__ part,
                                                         uint16_t* __restrict__ Y, int MN,
                                                         int splits) {
    const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= MN) return;
    f32x4 s = *reinterpret_cast<const f32x4*>(part + i);
    for (int k = 1; k < splits; ++k) s += *reinterpret_cast<const f32x4*>(part + static_cast<size_t>(k) * MN + i);
    u32x2 o;
    o[0] = f32_to_bf16_bits(s[0]) | (f32_to_bf16_bits(s[1]) << 16);
    o[1] = f32_to_bf16_bits(s[2]) | (f32_to_bf16_bits(s[3]) << 16);
    *reinterpret_cast<u32x2*>(Y + i) = o;
}

// Split count: the smallest divisor of K/kKB giving >= ~2 workgroups per CU.
int choose_splits(int M, int N, int K) {
    const char* e = std::getenv("KCMM_GEMM_SPLITS");
    const int kblocks = K / kKB;
    if (e) {
        const int s = std::atoi(e);
        if (s >= 1 && kblocks % s == 0) return s;
    }
    const int tiles = (N / kBN) * ((M + kBM - 1) / kBM);
    int best = 1;
    for (int s = 1; s <= kblocks; ++s) {
        if (kblocks % s) continue;
        best = s;
        if (tiles * s >= 512) break;
    }
    return best;
}

}  // namespace

namespace dev {

bool gemm_bf16(uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t n, uint32_t k,
               uint64_t stream, std::string* err) {
    if (n % kBN != 0 || k % kKB != 0) {
        *err = "gemm_bf16 needs n % 64 == 0 and k % 256 == 0";
        return false;
    }
    if (static_cast<uint64_t>(m) * k >= (1ull << 31) || static_cast<uint64_t>(n) * k >= (1ull << 31)) {
        *err = "gemm_bf16 operand too large";
        return false;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
    const int splits = choose_splits(M, N, K);
    float* part = nullptr;
    if (splits > 1) {
        void* ws = nullptr;
        if (!stream_workspace(stream, 1, static_cast<size_t>(splits) * M * N * sizeof(float), &ws,
                              false, err))
            return false;
        part = static_cast<float*>(ws);
    }
    const dim3 grid(N / kBN, (M + kBM - 1) / kBM, splits);
    hipLaunchKernelGGL(gemm_bf16_skinny, grid, dim3(256), 0, s,
                       reinterpret_cast<const uint16_t*>(x), reinterpret_cast<const uint16_t*>(w),
                       reinterpret_cast<uint16_t*>(y), part, M, N, K, K / splits);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    if (splits > 1) {
        const int MN = M * N;
        hipLaunchKernelGGL(gemm_split_reduce, dim3((MN / 4 + 255) / 256), dim3(256), 0, s, part,
                           reinterpret_cast<uint16_t*>(y), MN, splits);
        KCMM_HIP_CHECK(hipGetLastError(), err);
    }
    return true;
}

}  // namespace dev
}  // namespace kcmm
