// Decode-step projection GEMM for gfx950: Y[M][N] = X[M][K] * W[N][K]^T,
// bf16 operands, fp32 accumulation, bf16 result (the HF Linear layout the
// reference's weights use, ref llama_transformer.rs:115-120; the reference
// hands this to cuBLAS, ref runtime.rs:17-41).
//
// At decode the token count M is small (64..256) and the weights dominate the
// bytes: at M = 64 the arithmetic intensity is ~62 flop/B, far below the MFMA
// ridge, so the kernel is a weight stream (see gemm_bf16_stream).  K is split
// when N alone gives too few workgroups; fp32 split partials are summed by a
// second small kernel.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

// Row rotation by 8 inside each 16-lane row (DPP row_ror:8; its own inverse).
__device__ __forceinline__ uint32_t ror8(uint32_t x) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x128, 0xF, 0xF, false));
}

// x was loaded as lane (r, lg) <- row (r & 7), bytes (4*(r >> 3) + lg)*16 of a
// 128-byte line; y the same for rows 8..15.  Afterwards x holds bytes 0..63
// and y bytes 64..127 of rows 0..15, lane r = row r (MFMA A layout).
__device__ __forceinline__ void fix_lines(u32x4& x, u32x4& y, bool low8) {
    u32x4 nx, ny;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t rx = ror8(x[c]);
        const uint32_t ry = ror8(y[c]);
        nx[c] = low8 ? x[c] : ry;
        ny[c] = low8 ? rx : y[c];
    }
    x = nx;
    y = ny;
}

__device__ __forceinline__ u32x4 load_stream(const uint8_t* a) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a));
}

// Weight-streaming GEMM.  Workgroup = 4 waves = 64 weight rows (16 per wave)
// x up to 16*MB tokens x one K split of `klen`, walked in chunks of KCH:
//  * each wave's weight chunk (16 rows x KCH) goes HBM -> registers with
//    whole-line nontemporal loads (8 rows x 128 B per instruction) and is put
//    into MFMA A layout by fix_lines; chunk c+1 is in flight while chunk c is
//    consumed, so every weight byte is read once and never touches LDS;
//  * the activation chunk (M x KCH) is staged in LDS, double-buffered, 16-byte
//    pieces XOR-swizzled by row so that B-operand reads are conflict-free; one
//    barrier per chunk;
//  * rows of X past M are clamped (their output columns are never stored).
// (Measured alternatives that were slower at the Llama-3-8B decode shapes: a
// persistent grid over (row block, k chunk) tiles with a 6-deep ring, and
// direct-to-LDS activation loads with a 3-deep weight ring.)
// v (4 consecutive outputs) rounded to bf16, then + the residual row piece r,
// in fp32 (the result is rounded once more by the store): the order of a bf16
// model's "residual + o_proj(x)".
__device__ __forceinline__ f32x4 add_residual(f32x4 v, const uint16_t* r) {
    const u32x2 rr = *reinterpret_cast<const u32x2*>(r);
    f32x4 o;
    o[0] = bf16_bits_to_f32(f32_to_bf16_bits(v[0])) + __uint_as_float(rr[0] << 16);
    o[1] = bf16_bits_to_f32(f32_to_bf16_bits(v[1])) + __uint_as_float(rr[0] & 0xffff0000u);
    o[2] = bf16_bits_to_f32(f32_to_bf16_bits(v[2])) + __uint_as_float(rr[1] << 16);
    o[3] = bf16_bits_to_f32(f32_to_bf16_bits(v[3])) + __uint_as_float(rr[1] & 0xffff0000u);
    return o;
}

template <int MB, int KCH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void gemm_bf16_stream(const uint16_t* __restrict__ X, const uint16_t* __restrict__ W,
                      uint16_t* Y, float* __restrict__ part, const uint16_t* R, int M, int N, int K,
                      int klen) {
    constexpr int LINES = KCH / 64;          // 128-byte lines per weight row per chunk
    constexpr int KC = KCH / 32;             // MFMA k-steps per chunk
    constexpr int PIECES = KCH / 8;          // 16-byte pieces per activation row
    constexpr int MROWS = 16 * MB;
    constexpr int XLOADS = MROWS * PIECES / 256;
    static_assert(XLOADS * 256 == MROWS * PIECES, "activation chunk must split over 256 threads");
    __shared__ u32x4 xs[2][MROWS * PIECES];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 15, lg = lane >> 4;
    const bool low8 = ln < 8;
    const int n0 = blockIdx.x * 64 + wave * 16;
    const int m_base = blockIdx.z * MROWS;
    const int kbeg = blockIdx.y * klen;
    const int nchunks = klen / KCH;

    const uint8_t* wx = reinterpret_cast<const uint8_t*>(W + static_cast<size_t>(n0 + (ln & 7)) * K + kbeg) +
                        ((ln >> 3) * 4 + lg) * 16;
    const size_t row8 = static_cast<size_t>(8) * K * 2;
    auto load_w = [&](u32x4* dst, int c) {
        const uint8_t* q = wx + static_cast<size_t>(c) * KCH * 2;
#pragma unroll
        for (int c2 = 0; c2 < LINES; ++c2) {
            dst[2 * c2] = load_stream(q + c2 * 128);
            dst[2 * c2 + 1] = load_stream(q + row8 + c2 * 128);
        }
    };
    u32x4 xr[XLOADS];
    auto load_x = [&](int c) {
#pragma unroll
        for (int i = 0; i < XLOADS; ++i) {
            const int idx = tid + 256 * i;
            const int m = min(m_base + idx / PIECES, M - 1);
            xr[i] = *reinterpret_cast<const u32x4*>(X + static_cast<size_t>(m) * K + kbeg + c * KCH +
                                                    (idx % PIECES) * 8);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XLOADS; ++i) {
            const int idx = tid + 256 * i;
            const int r = idx / PIECES, pc = idx % PIECES;
            xs[buf][r * PIECES + (pc ^ (r & (PIECES - 1)))] = xr[i];
        }
    };

    f32x4 acc[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[j] = f32x4{0, 0, 0, 0};

    auto compute = [&](u32x4* wa, int buf) {
#pragma unroll
        for (int c2 = 0; c2 < LINES; ++c2) fix_lines(wa[2 * c2], wa[2 * c2 + 1], low8);
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            const int pc = 4 * kc + lg;
#pragma unroll
            for (int j = 0; j < MB; ++j) {
                const int r = 16 * j + ln;
                const u32x4 b = xs[buf][r * PIECES + (pc ^ (r & (PIECES - 1)))];
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wa[kc]),
                                                                 __builtin_bit_cast(bf16x8, b),
                                                                 acc[j], 0, 0, 0);
            }
        }
    };

    u32x4 wa0[2 * LINES], wa1[2 * LINES];
    load_x(0);
    load_w(wa0, 0);
    __builtin_amdgcn_sched_barrier(0);
    store_x(0);
    __syncthreads();
    // one chunk: loads of chunk c+1 (when MORE) are issued before chunk c is consumed
    auto step = [&](u32x4* now, u32x4* later, int buf, int c, auto more_tag) {
        constexpr bool MORE = decltype(more_tag)::value;
        if constexpr (MORE) {
            load_x(c + 1);
            load_w(later, c + 1);
        }
        // keep the compiler from sinking these loads below the chunk's math
        __builtin_amdgcn_sched_barrier(0);
        compute(now, buf);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (MORE) {
            store_x(buf ^ 1);
            __syncthreads();
        }
    };
    using More = std::integral_constant<bool, true>;
    using Last = std::integral_constant<bool, false>;
    int c = 0;
    for (; c + 2 < nchunks; c += 2) {
        step(wa0, wa1, 0, c, More{});
        step(wa1, wa0, 1, c + 1, More{});
    }
    if (c + 1 < nchunks) {
        step(wa0, wa1, 0, c, More{});
        step(wa1, wa0, 1, c + 1, Last{});
    } else {
        step(wa0, wa1, 0, c, Last{});
    }

    // acc[j][r] = Y[m_base + 16j + ln][n0 + 4lg + r]
#pragma unroll
    for (int j = 0; j < MB; ++j) {
        const int m = m_base + 16 * j + ln;
        if (m >= M) continue;
        const int n = n0 + 4 * lg;
        if (part == nullptr) {
            f32x4 v = acc[j];
            if (R != nullptr) v = add_residual(v, R + static_cast<size_t>(m) * N + n);
            u32x2 o;
            o[0] = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
            o[1] = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
            *reinterpret_cast<u32x2*>(Y + static_cast<size_t>(m) * N + n) = o;
        } else {
            *reinterpret_cast<f32x4*>(part + (static_cast<size_t>(blockIdx.y) * M + m) * N + n) = acc[j];
        }
    }
}

// Y = bf16(sum over splits of the fp32 partials) (+ R); 4 outputs per thread.
__global__ __launch_bounds__(256) void gemm_split_reduce(const float* __restrict__ part,
                                                         uint16_t* Y, const uint16_t* R, int MN,
                                                         int splits) {
    const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= MN) return;
    f32x4 s = *reinterpret_cast<const f32x4*>(part + i);
    for (int k = 1; k < splits; ++k) s += *reinterpret_cast<const f32x4*>(part + static_cast<size_t>(k) * MN + i);
    if (R != nullptr) s = add_residual(s, R + i);
    u32x2 o;
    o[0] = f32_to_bf16_bits(s[0]) | (f32_to_bf16_bits(s[1]) << 16);
    o[1] = f32_to_bf16_bits(s[2]) | (f32_to_bf16_bits(s[3]) << 16);
    *reinterpret_cast<u32x2*>(Y + i) = o;
}

int env_int(const char* name, int dflt) {
    const char* e = std::getenv(name);
    return e ? std::atoi(e) : dflt;
}

// K splits: the smallest divisor of K/kch giving at least `target` workgroups
// (KCMM_GEMM_WGS, default 256: fewer, longer splits measured faster than
// 512-1024 at the Llama-3-8B decode shapes) with each split at least two
// chunks long.
int choose_splits(int N, int K, int kch, int mgroups) {
    const int chunks = K / kch;
    const int forced = env_int("KCMM_GEMM_SPLITS", 0);
    if (forced >= 1 && chunks % forced == 0) return forced;
    const int target = env_int("KCMM_GEMM_WGS", 256);
    const int tiles = (N / 64) * mgroups;
    int best = 1;
    for (int s = 1; s <= chunks; ++s) {
        if (chunks % s) continue;
        if (chunks / s < 2 && s > 1) break;
        best = s;
        if (tiles * s >= target) break;
    }
    return best;
}

template <int MB, int KCH>
bool launch_gemm(const uint16_t* X, const uint16_t* W, uint16_t* Y, const uint16_t* R, int M,
                 int N, int K, uint64_t stream, std::string* err) {
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int mgroups = (M + 16 * MB - 1) / (16 * MB);
    const int splits = choose_splits(N, K, KCH, mgroups);
    float* part = nullptr;
    if (splits > 1) {
        void* ws = nullptr;
        if (!dev::stream_workspace(stream, 1, static_cast<size_t>(splits) * M * N * sizeof(float),
                                   &ws, false, err))
            return false;
        part = static_cast<float*>(ws);
    }
    const dim3 grid(N / 64, splits, mgroups);
    hipLaunchKernelGGL((gemm_bf16_stream<MB, KCH>), grid, dim3(256), 0, s, X, W, Y, part, R, M, N, K,
                       K / splits);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    if (splits > 1) {
        const int MN = M * N;
        hipLaunchKernelGGL(gemm_split_reduce, dim3((MN / 4 + 255) / 256), dim3(256), 0, s, part, Y,
                           R, MN, splits);
        KCMM_HIP_CHECK(hipGetLastError(), err);
    }
    return true;
}

}  // namespace

namespace dev {

bool gemm_bf16(uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t n, uint32_t k,
               uint64_t stream, std::string* err, uint64_t residual) {
    if (m == 0 || n % 64 != 0 || k % 256 != 0 || n == 0 || k == 0) {
        *err = "gemm_bf16 needs m > 0, n % 64 == 0 and k % 256 == 0";
        return false;
    }
    if (static_cast<uint64_t>(m) * k >= (1ull << 31) || static_cast<uint64_t>(n) * k >= (1ull << 31) ||
        static_cast<uint64_t>(m) * n >= (1ull << 29)) {
        *err = "gemm_bf16 operand too large";
        return false;
    }
    const auto* X = reinterpret_cast<const uint16_t*>(x);
    const auto* W = reinterpret_cast<const uint16_t*>(w);
    auto* Y = reinterpret_cast<uint16_t*>(y);
    const auto* R = reinterpret_cast<const uint16_t*>(residual);
    const int M = static_cast<int>(m), N = static_cast<int>(n), K = static_cast<int>(k);
    // token blocks per pass: the activation chunk (M x KCH bf16) is 32 KiB
    if (M <= 16) return launch_gemm<1, 256>(X, W, Y, R, M, N, K, stream, err);
    if (M <= 32) return launch_gemm<2, 256>(X, W, Y, R, M, N, K, stream, err);
    if (M <= 64) return launch_gemm<4, 256>(X, W, Y, R, M, N, K, stream, err);
    if (M <= 128) return launch_gemm<8, 128>(X, W, Y, R, M, N, K, stream, err);
    return launch_gemm<16, 64>(X, W, Y, R, M, N, K, stream, err);
}

}  // namespace dev
}  // namespace kcmm
