// Projection GEMM for many tokens (M > 128) on gfx950:
// Y[M][N] = X[M][K] * W[N][K]^T (+ R), bf16 operands, fp32 accumulation on
// v_mfma_f32_16x16x32_bf16 -- the product the reference hands to cuBLAS
// (ref runtime.rs:17-41, called at llama_transformer.rs:115-120).
//
// With a few hundred tokens the MFMA work per weight byte is 4x that of a
// decode batch of 64, so both operands are staged through LDS and reused
// from there (the decode-sized kernel streams weights straight into
// registers instead):
//  * workgroup = 4 waves on a BN (weight rows) x BM (tokens) tile, waves in a
//    2 x 2 grid, each accumulating (BN/2) x (BM/2) in registers;
//  * K is walked in 64-element chunks through an NS-stage ring of LDS
//    buffers filled by direct-to-LDS loads (global_load_lds_dwordx4: 16 bytes
//    per lane, lane-contiguous in LDS), NS - 1 chunks in flight while one is
//    consumed, one barrier per chunk;
//  * LDS rows are 128 bytes of 16-byte pieces, piece p of row r stored at
//    slot p ^ (r & 7): the MFMA operand reads (16 rows x one piece per
//    16 lanes) hit distinct banks; the permutation is applied on the global
//    side, since the LDS side of a direct load is fixed;
//  * tiles are numbered so that the M tiles of one weight tile run on the
//    same XCD at the same time (workgroup i runs on XCD i % 8): the weight
//    tile then comes from HBM once and from that XCD's L2 for the rest;
//  * optional K split: each split writes fp32 partials, summed in split
//    order by gemm_split_reduce (the same partial layout as the streaming
//    kernel);
//  * fp8-e4m3 weights (WF8): the weight tile is staged as codes, 64-byte
//    LDS rows of four 16-byte pieces (piece p of row r at slot
//    p ^ ((r >> 2) & 3)), each MFMA operand read as 8 codes and converted
//    exactly to bf16 in registers; the fp32 row scale multiplies the
//    accumulator before the store.
#include <algorithm>
#include <cstdlib>
#include <string>
#include <type_traits>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

typedef __attribute__((address_space(3))) void* lds_ptr;

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (lds is wave-uniform).  A plain function: inside a template the host
// compilation pass rejects the LDS address-space cast.
__device__ __forceinline__ void load_lds16(const uint8_t* g, uint8_t* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr)lds, 16, 0, 0);
}
// The same, nontemporal (streamed data: weights are read once).
__device__ __forceinline__ void load_lds16_nt(const uint8_t* g, uint8_t* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr)lds, 16, 0, 2);
}

// s_waitcnt vmcnt(N), leaving the other counters alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt lgkmcnt(0): this wave's LDS reads and writes are done.
__device__ __forceinline__ void wait_lgkm0() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));
}

struct TiledParams {
    const uint8_t* X;    // [M][K] bf16
    const uint8_t* W;    // [N][K] bf16, or e4m3 codes with WF8
    const float* wscale; // WF8: fp32 scale per weight row [N]
    uint16_t* Y;         // [M][N]
    const uint16_t* R;   // residual [M][N] or null (may equal Y)
    float* part;         // non-null: fp32 partials [split][M][N]
    int M, N, K, klen;   // klen: K per split
    int tiles_m;         // M tiles per weight tile
    int xcd_order;       // tiles % 8 == 0: XCD-grouped numbering
};

__device__ __forceinline__ u32x2 pack4(f32x4 v) {
    u32x2 o;
    o[0] = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
    o[1] = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
    return o;
}

// Eight e4m3 codes (two dwords) -> eight bf16, exactly.
__device__ __forceinline__ u32x4 fp8x8_bf16(u32x2 d) {
    u32x4 r;
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d[0], 1.0f, false));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d[0], 1.0f, true));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d[1], 1.0f, false));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d[1], 1.0f, true));
    return r;
}

// WN x WM waves, each accumulating (BN/WN) x (BM/WM) of the tile.
template <int BN, int BM, int WN, int WM, int NS, bool WNT, bool WF8 = false>
__global__ __launch_bounds__(64 * WN * WM) void gemm_tiled_kernel(TiledParams p) {
    constexpr int NWAVES = WN * WM;
    constexpr int KT = 64;                  // k per chunk: 128-byte LDS rows (fp8 weights: 64)
    constexpr int WROW = WF8 ? 64 : 128;    // LDS bytes per weight row per chunk
    constexpr int WRI = 1024 / WROW;        // weight rows per load instruction
    constexpr int WB = BN * WROW, XB = BM * 128, SB = WB + XB;
    constexpr int WL = BN / (WRI * NWAVES), XL = BM / (8 * NWAVES);   // loads per wave per chunk
    constexpr int TN = BN / WN, TM = BM / WM;                     // wave tile
    constexpr int FA = TN / 16, FB = TM / 16;                     // MFMA fragments per k-step
    static_assert(WL * WRI * NWAVES == BN && XL * 8 * NWAVES == BM, "tile rows split over the waves");
    static_assert(TN % 16 == 0 && TM % 16 == 0, "wave tile");
    static_assert(NS * SB <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * SB];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ln = lane & 15, lg = lane >> 4;

    // tile of this workgroup
    const int ntiles = gridDim.x;
    int t = blockIdx.x;
    if (p.xcd_order) t = (t & 7) * (ntiles >> 3) + (t >> 3);
    const int tn = t / p.tiles_m, tm = t - tn * p.tiles_m;
    const int n0 = tn * BN, m0 = tm * BM;
    const int kbeg = blockIdx.y * p.klen;
    const int nchunks = p.klen / KT;
    const size_t rowb = static_cast<size_t>(p.K) * 2;
    const size_t wrowb = static_cast<size_t>(p.K) * (WF8 ? 1 : 2);

    // Direct loads: instruction i of wave w fills LDS rows 8*(NWAVES*i + w)
    // .. +8 of the W (then X) tile; lane l writes slot l & 7 of row
    // 8*(NWAVES*i + w) + (l >> 3), i.e. piece (l & 7) ^ (row & 7).
    const int lrow = lane >> 3;
    const int lpiece = (lane & 7) ^ lrow;   // rows of one instruction start at a multiple of 8
    const uint8_t* wsrc[WL];
    const uint8_t* xsrc[XL];
#pragma unroll
    for (int i = 0; i < WL; ++i) {
        if constexpr (WF8) {
            // 16 rows x 64 bytes per instruction: lane l fills slot l & 3 of
            // row 16*(NWAVES*i + w) + (l >> 2) with piece (l & 3) ^ ((row >> 2) & 3)
            const int r = 16 * (NWAVES * i + wave) + (lane >> 2);
            const int pc = (lane & 3) ^ ((lane >> 4) & 3);
            wsrc[i] = p.W + (n0 + r) * wrowb + static_cast<size_t>(kbeg) + pc * 16;
        } else {
            const int r = 8 * (NWAVES * i + wave) + lrow;
            wsrc[i] = p.W + (n0 + r) * wrowb + static_cast<size_t>(kbeg) * 2 + lpiece * 16;
        }
    }
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        const int r = min(m0 + 8 * (NWAVES * i + wave) + lrow, p.M - 1);   // rows past M: clamped, unused
        xsrc[i] = p.X + r * rowb + static_cast<size_t>(kbeg) * 2 + lpiece * 16;
    }
    auto issue = [&](int c) {
        uint8_t* st = lds + (c % NS) * SB;
        const size_t ko = static_cast<size_t>(c) * KT * 2;
        const size_t kw = static_cast<size_t>(c) * KT * (WF8 ? 1 : 2);
#pragma unroll
        for (int i = 0; i < WL; ++i) {
            if constexpr (WNT) load_lds16_nt(wsrc[i] + kw, st + (NWAVES * i + wave) * 1024);
            else load_lds16(wsrc[i] + kw, st + (NWAVES * i + wave) * 1024);
        }
#pragma unroll
        for (int i = 0; i < XL; ++i) load_lds16(xsrc[i] + ko, st + WB + (NWAVES * i + wave) * 1024);
    };

    // wave (wn, wm): weight rows wn*TN .., tokens wm*TM ..
    const int wn = wave % WN, wm = wave / WN;
    f32x4 acc[FA][FB];
#pragma unroll
    for (int i = 0; i < FA; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    // Fragments of one k-step (32 k) of chunk c: weight rows and tokens of
    // this wave, from LDS stage c % NS.
    auto read_frags = [&](u32x4* a, u32x4* b, int c, int ks) {
        const uint8_t* st = lds + (c % NS) * SB;
        const int pc = ks * 4 + lg;
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            const int r = wn * TN + 16 * i + ln;
            if constexpr (WF8) {
                // codes k = ks*32 + 8*lg .. +8: piece 2 ks + lg/2, half lg & 1
                const int pp = 2 * ks + (lg >> 1);
                a[i] = fp8x8_bf16(*reinterpret_cast<const u32x2*>(
                    st + r * 64 + ((pp ^ ((r >> 2) & 3)) * 16) + (lg & 1) * 8));
            } else {
                a[i] = *reinterpret_cast<const u32x4*>(st + r * 128 + ((pc ^ (r & 7)) * 16));
            }
        }
#pragma unroll
        for (int j = 0; j < FB; ++j) {
            const int r = wm * TM + 16 * j + ln;
            b[j] = *reinterpret_cast<const u32x4*>(st + WB + r * 128 + ((pc ^ (r & 7)) * 16));
        }
    };
    auto mfmas = [&](const u32x4* a, const u32x4* b) {
#pragma unroll
        for (int i = 0; i < FA; ++i)
#pragma unroll
            for (int j = 0; j < FB; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8, a[i]), __builtin_bit_cast(bf16x8, b[j]), acc[i][j],
                    0, 0, 0);
    };
    // chunk c landed in LDS for every wave (this wave waits for its own
    // loads, the barrier for the others'), and every wave's earlier LDS
    // reads are done; bare barrier: a fenced one would also wait for the
    // chunks still in flight
    constexpr int PER = WL + XL;
    auto chunk_ready = [&](int c) {
        if (c + NS - 2 < nchunks) wait_vmcnt<(NS - 2) * PER>();
        else wait_vmcnt<0>();
        wait_lgkm0();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // Software pipeline: the reads of one k-step are in flight while the
    // MFMAs of the previous one run.  Per chunk c:
    //   refill the stage chunk c-1 used, read k-step 1 of c, MFMAs of
    //   k-step 0 of c, wait for chunk c+1 + barrier, read k-step 0 of c+1,
    //   MFMAs of k-step 1 of c.
    // The stage refilled at chunk c (chunk c+NS-1's, = c-1's stage) was last
    // read by k-step 1 of c-1, complete in every wave at the barrier of
    // iteration c-1.
#pragma unroll
    for (int c = 0; c < NS - 1; ++c)
        if (c < nchunks) issue(c);
    // (the last chunk's "next" reads re-read it, unused: the LDS reads in
    // flight are the same on every path, so the compiler's waits stay exact)
    const int last = nchunks - 1;
    u32x4 a0[FA], b0[FB], a1[FA], b1[FB];
    chunk_ready(0);
    read_frags(a0, b0, 0, 0);
    for (int c = 0; c < nchunks; ++c) {
        if (c + NS - 1 < nchunks) issue(c + NS - 1);
        read_frags(a1, b1, c, 1);
        mfmas(a0, b0);
        const int nx = min(c + 1, last);
        chunk_ready(nx);
        read_frags(a0, b0, nx, 0);
        mfmas(a1, b1);
    }

    // store: acc[i][j][r] = (token m0 + wm*TM + 16j + ln, row n0 + wn*TN + 16i + 4lg + r)
#pragma unroll
    for (int j = 0; j < FB; ++j) {
        const int m = m0 + wm * TM + 16 * j + ln;
        if (m >= p.M) continue;
#pragma unroll
        for (int i = 0; i < FA; ++i) {
            const int n = n0 + wn * TN + 16 * i + 4 * lg;
            if constexpr (WF8) {
                const f32x4 s4 = {p.wscale[n], p.wscale[n + 1], p.wscale[n + 2], p.wscale[n + 3]};
                acc[i][j] *= s4;
            }
            if (p.part != nullptr) {
                *reinterpret_cast<f32x4*>(p.part + (static_cast<size_t>(blockIdx.y) * p.M + m) * p.N + n) =
                    acc[i][j];
                continue;
            }
            f32x4 v = acc[i][j];
            if (p.R != nullptr) {
                const u32x2 rr = *reinterpret_cast<const u32x2*>(p.R + static_cast<size_t>(m) * p.N + n);
                v[0] = bf16_round_f32(v[0]) + __uint_as_float(rr[0] << 16);
                v[1] = bf16_round_f32(v[1]) + __uint_as_float(rr[0] & 0xffff0000u);
                v[2] = bf16_round_f32(v[2]) + __uint_as_float(rr[1] << 16);
                v[3] = bf16_round_f32(v[3]) + __uint_as_float(rr[1] & 0xffff0000u);
            }
            *reinterpret_cast<u32x2*>(p.Y + static_cast<size_t>(m) * p.N + n) = pack4(v);
        }
    }
}

// Kernel configurations: tile (BN weight rows x BM tokens), wave grid and
// LDS stages; every one keeps two waves on each SIMD (8-wave workgroups, or
// 4-wave workgroups small enough for two per CU).
struct TiledConfig {
    int id, bn, bm, splits;
};
constexpr int kCfgs = 11;
constexpr int kCfgBN[kCfgs] = {128, 128, 128, 64, 64, 128, 256, 128, 128, 128, 64};
constexpr int kCfgBM[kCfgs] = {256, 128, 64, 128, 64, 256, 128, 256, 256, 128, 64};

template <int V>
using ic = std::integral_constant<int, V>;

// f(BN, BM, WN, WM, NS, weights nontemporal).  Nontemporal weights keep the
// activation tile in L2 when every weight tile is used once (BM covers M);
// smaller token tiles reuse the weight tile from L2 instead (measured
// slower with it).
template <typename F>
void by_config(int id, F&& f) {
    using T = std::true_type;
    using F0 = std::false_type;
    switch (id) {
        case 0: f(ic<128>{}, ic<256>{}, ic<2>{}, ic<4>{}, ic<3>{}, T{}); break;
        case 1: f(ic<128>{}, ic<128>{}, ic<2>{}, ic<4>{}, ic<4>{}, F0{}); break;
        case 2: f(ic<128>{}, ic<64>{}, ic<2>{}, ic<2>{}, ic<3>{}, F0{}); break;
        case 3: f(ic<64>{}, ic<128>{}, ic<2>{}, ic<2>{}, ic<3>{}, F0{}); break;
        case 4: f(ic<64>{}, ic<64>{}, ic<2>{}, ic<2>{}, ic<4>{}, F0{}); break;
        case 5: f(ic<128>{}, ic<256>{}, ic<2>{}, ic<2>{}, ic<3>{}, F0{}); break;
        case 6: f(ic<256>{}, ic<128>{}, ic<4>{}, ic<2>{}, ic<3>{}, F0{}); break;
        case 7: f(ic<128>{}, ic<256>{}, ic<2>{}, ic<4>{}, ic<2>{}, F0{}); break;
        case 8: f(ic<128>{}, ic<256>{}, ic<2>{}, ic<4>{}, ic<3>{}, F0{}); break;
        case 9: f(ic<128>{}, ic<128>{}, ic<2>{}, ic<4>{}, ic<4>{}, T{}); break;
        default: f(ic<64>{}, ic<64>{}, ic<2>{}, ic<2>{}, ic<4>{}, T{}); break;
    }
}

// Tile and K split by a cost model fitted to cold-cache timings (weights
// not resident in the Infinity Cache, as in a model's layer loop): among
// the nontemporal-weight configurations 0 (128 x 256), 9 (128 x 128) and
// 10 (64 x 64), and splits whose parts are at least 8 chunks long, the one
// that minimises
//   (weight bytes + 3 x fp32 partial bytes + L2->LDS bytes / 2) / efficiency
// where L2->LDS bytes = 2 N M K (1/BM + 1/BN) (each tile loads its weight
// rows and tokens) and efficiency = the fraction of workgroup slots the grid
// fills in its last round (one workgroup per CU for configurations 0 and 9,
// two for 10) times the fraction of each token tile that is real tokens
// (partials count three times: written, read back, and the reduction's own
// launch).
// At the Llama-3-8B shapes this picks 9 x 2 / 9 x 4 for QKV / O at M = 256
// (32.5 / 24.7 us against 46.8 / 30.2 for 64 x 64 unsplit, caches flushed),
// 9 x 1 / 9 x 2 at M = 512, and keeps 0 for gate/up and 0 x 8 (M = 256) /
// 0 x 4 (M = 512) for down.  KCMM_GEMM_TILE
// (configuration index) and KCMM_GEMM_SPLITS override.
TiledConfig choose(int M, int N, int K) {
    const int chunks = K / 64;
    const int forced_tile = dev::tunable_or(dev::Tun::kGemmTile, -1);
    auto ok_split = [&](int s) { return chunks % s == 0 && chunks / s >= 8; };
    TiledConfig best{-1, 0, 0, 1};
    if (forced_tile >= 0 && forced_tile < kCfgs && N % kCfgBN[forced_tile] == 0) {
        best = TiledConfig{forced_tile, kCfgBN[forced_tile], kCfgBM[forced_tile], 1};
    } else {
        double best_cost = 0.0;
        const double wbytes = 2.0 * N * K;
        for (int cand : {0, 9, 10}) {
            const int bn = kCfgBN[cand], bm = kCfgBM[cand];
            if (N % bn) continue;
            const int tiles_m = (M + bm - 1) / bm;
            const int tiles = (N / bn) * tiles_m;
            const int slots = cand == 10 ? 512 : 256;
            const double real = static_cast<double>(M) / (tiles_m * bm);
            const double l2 = 2.0 * N * M * K * (1.0 / bm + 1.0 / bn);
            for (int s = 1; s <= 16; s *= 2) {
                if (!ok_split(s)) break;
                const int wgs = tiles * s;
                const int rounds = (wgs + slots - 1) / slots;
                const double eff = static_cast<double>(wgs) / (rounds * slots) * real;
                const double part = s > 1 ? 4.0 * s * M * N : 0.0;
                const double cost = (wbytes + 3.0 * part + 0.5 * l2) / eff;
                if (best.id < 0 || cost < best_cost) {
                    best = TiledConfig{cand, bn, bm, s};
                    best_cost = cost;
                }
            }
        }
        if (best.id < 0) best = TiledConfig{3, kCfgBN[3], kCfgBM[3], 1};   // N % 64 == 0 only
    }
    const int forced = dev::tunable_or(dev::Tun::kGemmSplits, 0);
    if (forced >= 1 && forced <= 16 && chunks % forced == 0) best.splits = forced;
    return best;
}

}  // namespace

namespace dev {

void gemm_tiled_plan(uint32_t m, uint32_t n, uint32_t k, int* splits, int* tile) {
    const TiledConfig c = choose(static_cast<int>(m), static_cast<int>(n), static_cast<int>(k));
    *splits = c.splits;
    *tile = c.id;
}

bool gemm_tiled(uint64_t x, uint64_t w, uint64_t wscale, uint64_t y, uint32_t m, uint32_t n,
                uint32_t k, uint64_t stream, uint64_t residual, std::string* err) {
    if (m == 0 || n % 64 != 0 || k % 64 != 0) {
        *err = "tiled gemm needs m > 0, n % 64 == 0 and k % 64 == 0";
        return false;
    }
    const TiledConfig c = choose(static_cast<int>(m), static_cast<int>(n), static_cast<int>(k));
    TiledParams p{};
    p.X = reinterpret_cast<const uint8_t*>(x);
    p.W = reinterpret_cast<const uint8_t*>(w);
    p.wscale = reinterpret_cast<const float*>(wscale);
    p.Y = reinterpret_cast<uint16_t*>(y);
    p.R = reinterpret_cast<const uint16_t*>(residual);
    p.M = static_cast<int>(m);
    p.N = static_cast<int>(n);
    p.K = static_cast<int>(k);
    p.klen = p.K / c.splits;
    p.tiles_m = (p.M + c.bm - 1) / c.bm;
    const int tiles = (p.N / c.bn) * p.tiles_m;
    p.xcd_order = tiles % 8 == 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (c.splits > 1) {
        void* ws = nullptr;
        if (!stream_workspace(stream, 1, static_cast<size_t>(c.splits) * p.M * p.N * sizeof(float),
                              &ws, false, err))
            return false;
        p.part = static_cast<float*>(ws);
    }
    by_config(c.id, [&](auto bn, auto bm, auto wn, auto wm, auto ns, auto nt) {
        constexpr int BN = decltype(bn)::value, BM = decltype(bm)::value;
        constexpr int WN = decltype(wn)::value, WM = decltype(wm)::value, NS = decltype(ns)::value;
        constexpr bool NT = decltype(nt)::value;
        if (wscale != 0)
            hipLaunchKernelGGL((gemm_tiled_kernel<BN, BM, WN, WM, NS, NT, true>),
                               dim3(tiles, c.splits), dim3(64 * WN * WM), 0, s, p);
        else
            hipLaunchKernelGGL((gemm_tiled_kernel<BN, BM, WN, WM, NS, NT>), dim3(tiles, c.splits),
                               dim3(64 * WN * WM), 0, s, p);
    });
    KCMM_HIP_CHECK(hipGetLastError(), err);
    if (c.splits > 1)
        return gemm_split_reduce_launch(p.part, p.Y, p.R, p.M * p.N, c.splits, stream, err);
    return true;
}

bool gemm_bf16_tiled(uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t n, uint32_t k,
                     uint64_t stream, uint64_t residual, std::string* err) {
    return gemm_tiled(x, w, 0, y, m, n, k, stream, residual, err);
}

}  // namespace dev
}  // namespace kcmm
