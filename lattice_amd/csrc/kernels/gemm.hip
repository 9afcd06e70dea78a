// Decode-step projection GEMM for gfx950: Y[M][N] = X[M][K] * W[N][K]^T,
// bf16 operands, fp32 accumulation, bf16 result (the HF Linear layout the
// reference's weights use, ref llama_transformer.rs:115-120; the reference
// hands this to cuBLAS, ref runtime.rs:17-41).
//
// At decode the token count M is small (64..256) and the weights dominate the
// bytes: at M = 64 the arithmetic intensity is ~62 flop/B, far below the MFMA
// ridge, so the kernel is a weight stream (see gemm_bf16_stream).  K is split
// when N alone gives too few workgroups: each split then writes fp32
// partials and the kernel that consumes the product sums them (in split
// order) as its first step -- a plain reduce, the SwiGLU finish here, or the
// RoPE/append and residual/RMSNorm kernels of glue.hip -- so no workgroup
// waits on another and no extra kernel is spent on the sum.
//
// Without a split, three epilogues run in the GEMM's own store:
//  * plain: Y = bf16(acc), or Y = bf16(R + bf16(acc)) with a residual R;
//  * rope_append (the fused QKV projection of a decode step): q heads are
//    rotated into q_out, k heads rotated and v heads copied straight into the
//    token's page row, so qkv never makes a round trip through HBM;
//  * swiglu (the fused gate/up projection): act = bf16(bf16(silu(g)) * u).
// The paired epilogues choose which weight rows a wave streams so that both
// members of a pair (RoPE i and i + D/2; gate j and up I + j) land in the
// same wave, 32 lanes apart.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "../device_api.hpp"
#include "common.hpp"


namespace kcmm {
namespace {

constexpr int kEpiPlain = 0;
constexpr int kEpiRope = 1;
constexpr int kEpiSwiglu = 2;

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

// Eight e4m3 values (two dwords) -> eight bf16, exactly (every e4m3 value is
// a bf16 value).
__device__ __forceinline__ u32x4 fp8x8_to_bf16(uint32_t d0, uint32_t d1) {
    u32x4 r;
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, false));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, true));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, false));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, true));
    return r;
}

__device__ __forceinline__ u32x4 load_stream(const uint8_t* a) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a));
}

__device__ __forceinline__ u32x2 pack4_bf16(f32x4 v) {
    u32x2 o;
    o[0] = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
    o[1] = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
    return o;
}

// 4 consecutive outputs rounded to bf16, then + the residual piece r in fp32
// (rounded once more by the store): the order of a bf16 model's
// "residual + o_proj(x)".
__device__ __forceinline__ f32x4 add_residual(f32x4 v, const uint16_t* r) {
    const u32x2 rr = *reinterpret_cast<const u32x2*>(r);
    f32x4 o;
    o[0] = bf16_round_f32(v[0]) + __uint_as_float(rr[0] << 16);
    o[1] = bf16_round_f32(v[1]) + __uint_as_float(rr[0] & 0xffff0000u);
    o[2] = bf16_round_f32(v[2]) + __uint_as_float(rr[1] << 16);
    o[3] = bf16_round_f32(v[3]) + __uint_as_float(rr[1] & 0xffff0000u);
    return o;
}

struct GemmParams {
    const uint16_t* X;   // [M][K]
    const uint16_t* W;   // [N][K]
    uint16_t* Y;         // plain: [M][N]; swiglu: act [M][N/2]
    const uint16_t* R;   // plain: residual [M][N] or null (may equal Y)
    float* part;         // non-null: write fp32 partials [split][M][N], no epilogue
    const float* wscale; // fp8 weights: fp32 scale per weight row [N] (row n of W times wscale[n])
    int M, N, K, klen;
    // rope_append
    uint16_t* q_out;     // [M][Hq][D]
    uint8_t* k_base;
    uint8_t* v_base;
    const int32_t* block_tables;
    const int32_t* seq_lens;
    const uint64_t* offsets_f16;
    const float* inv_freq;
    int hq, hkv, D, block_size, mbps, row_bytes;
};

// The store of one wave's 16 weight rows x 16*MB tokens: acc[j][r] = output
// (token m_base + 16j + ln, wave row 4lg + r), wave rows 0..7 = weight rows
// rowA + 0..7 and 8..15 = rowB + 0..7.  With p.part set: fp32 partials of
// split blockIdx.y, else the EPI epilogue.
template <int MB, int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p, f32x4 (&acc)[MB], int rowA,
                                              int rowB, int m_base, int ln, int lg) {
    const bool hi = lg >= 2;
    const int cw = 4 * (lg & 1);
    if (p.wscale != nullptr) {
        // fp8 weights: the row scale multiplies the whole dot product
        const float* sc = p.wscale + (hi ? rowB : rowA) + cw;
        const f32x4 s4 = {sc[0], sc[1], sc[2], sc[3]};
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[j] *= s4;
    }
    if (p.part != nullptr) {
        const int n = (hi ? rowB : rowA) + cw;
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            const int m = m_base + 16 * j + ln;
            if (m >= p.M) continue;
            *reinterpret_cast<f32x4*>(p.part + (static_cast<size_t>(blockIdx.y) * p.M + m) * p.N + n) = acc[j];
        }
        return;
    }
    if constexpr (EPI == kEpiPlain) {
        const int n = rowA + 4 * lg;
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            const int m = m_base + 16 * j + ln;
            if (m >= p.M) continue;
            f32x4 v = acc[j];
            if (p.R != nullptr) v = add_residual(v, p.R + static_cast<size_t>(m) * p.N + n);
            *reinterpret_cast<u32x2*>(p.Y + static_cast<size_t>(m) * p.N + n) = pack4_bf16(v);
        }
    } else if constexpr (EPI == kEpiSwiglu) {
        const int I = p.N / 2;
        const int col = rowA + cw;
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            f32x4 g, u;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float own = bf16_round_f32(acc[j][r]);
                const float other = __shfl_xor(own, 32);
                g[r] = hi ? other : own;
                u[r] = hi ? own : other;
            }
            const int m = m_base + 16 * j + ln;
            if (hi || m >= p.M) continue;
            f32x4 a;
#pragma unroll
            for (int r = 0; r < 4; ++r) a[r] = swiglu_bf16(g[r], u[r]);
            *reinterpret_cast<u32x2*>(p.Y + static_cast<size_t>(m) * I + col) = pack4_bf16(a);
        }
    } else {
        const int D = p.D;
        const int head = rowA / D;                // wave-uniform
        const int i0 = rowA - head * D + cw;      // rotation pair of r = 0
        const bool rotate = head < p.hq + p.hkv;
        const int e0 = i0 + (hi ? D / 2 : 0);     // element of r = 0 in the head
        float ifr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) ifr[r] = rotate ? p.inv_freq[i0 + r] : 0.0f;
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            f32x4 own, other;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                own[r] = bf16_round_f32(acc[j][r]);
                other[r] = __shfl_xor(own[r], 32);
            }
            const int m = m_base + 16 * j + ln;
            if (m >= p.M) continue;
            const int pos = p.seq_lens[m] - 1;
            if (pos < 0 || pos >= p.mbps * p.block_size) continue;   // no token / past the table
            f32x4 out = own;
            if (rotate) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float cs, sn;
                    rope_cos_sin(pos, ifr[r], &cs, &sn);
                    out[r] = hi ? rope_second(other[r], own[r], cs, sn)
                                : rope_first(own[r], other[r], cs, sn);
                }
            }
            uint16_t* dst;
            if (head < p.hq) {
                dst = p.q_out + (static_cast<size_t>(m) * p.hq + head) * D + e0;
            } else {
                const int lb = pos / p.block_size;
                const uint64_t page =
                    p.offsets_f16[p.block_tables[static_cast<size_t>(m) * p.mbps + lb]] * 2ull +
                    static_cast<uint64_t>(pos - lb * p.block_size) * p.row_bytes;
                uint8_t* region = head < p.hq + p.hkv ? p.k_base : p.v_base;
                const int kvh = head < p.hq + p.hkv ? head - p.hq : head - p.hq - p.hkv;
                dst = reinterpret_cast<uint16_t*>(region + page + static_cast<uint64_t>(kvh) * D * 2) + e0;
            }
            *reinterpret_cast<u32x2*>(dst) = pack4_bf16(out);
        }
    }
}

// Weight-streaming GEMM.  Workgroup = NW waves, of which the first CW stream
// 16 weight rows each (NW = CW = 4 without helper waves; split products NW =
// 8 with CW = 4, or 6 for the QKV / RoPE product; unsplit plain and SwiGLU
// products NW = 12 with CW = 8, or NW = CW = 8 without helpers; the NW - CW
// helper waves do all of the activation staging) x up to 16*MB tokens x one
// K split of `klen`, walked in chunks of KCH:
//  * each wave's weight chunk (16 rows x KCH) goes HBM -> registers with
//    whole-line streaming loads (8 rows x 128 B per instruction) and is put
//    into MFMA A layout by fix_lines, one line at a time; chunk c+1 is in
//    flight while chunk c is consumed, so every weight byte is read once and
//    never touches LDS;
//  * the activation chunk (M x KCH) is staged in LDS, double-buffered, 16-byte
//    pieces XOR-swizzled by row so that B-operand reads are conflict-free;
//    one barrier per chunk;
//  * activation rows past M are clamped (their outputs are never stored).
// (Measured alternatives that were not faster at the Llama-3-8B decode
// shapes: a persistent grid over (row block, k chunk) tiles with a 6-deep
// ring; direct-to-LDS activation loads with a 3-deep weight ring; a 3-deep
// register weight ring (two chunks always in flight; also fully unrolled, so
// that no wait lands inside a chunk's math: still 4% slower -- more weight
// requests in flight lower the DRAM efficiency); buffer loads with
// padded LDS rows; 8-wave workgroups at 2 or 4 waves per SIMD; waves that
// each take a quarter of every chunk's k range over all 64 rows (no LDS
// staging or per-chunk barrier, but a row's lines are then read by four
// drifting waves: 20% slower); for M > 128, waves of 32 rows x 128 tokens in
// 4- or 8-wave workgroups (halves the activation reads per MFMA, but two waves
// then stream each weight line: 20-40% slower); summing the split partials inside this kernel
// by the last workgroup of each tile, whose coherent stores and arrival count
// put several memory round trips on every tile's tail; for the split products,
// 8-wave workgroups whose two wave groups take alternate k halves (summed in
// LDS), a 3-deep weight ring, and 6-wave workgroups of 96 rows for QKV (the
// product itself 15% faster, but the attention kernel launched two kernels
// later then loses more than that: its one-wave workgroups land unevenly on
// the SIMDs after a kernel whose workgroups are not a multiple of four waves;
// two helper waves make the same grid 8-wave and keep the gain, and they gain
// more when they take over the activation staging); 7 streaming waves and a
// helper for gate/up (256 workgroups: slower than 224 of 8 streaming waves).)
template <int MB, int KCH, int EPI, bool WF8 = false, int NW = 4, int CW = NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW > 8 ? 3 : 2)))
void gemm_bf16_stream(GemmParams p) {
    constexpr int NT = NW * 64;
    // 128-byte lines per weight row per chunk (fp8 weights: half as many)
    constexpr int LINES = WF8 ? KCH / 128 : KCH / 64;
    constexpr int KC = KCH / 32;             // MFMA k-steps per chunk
    constexpr int PIECES = KCH / 8;          // 16-byte pieces per activation row
    constexpr int MROWS = 16 * MB;
    // threads that stage the activation chunks: all of them, or (CW < NW)
    // only the NW - CW helper waves, while the CW streaming waves never
    // touch the activation path
    static_assert(CW >= 1 && CW <= NW, "streaming waves must be 1..NW");
    constexpr bool SPEC = CW < NW;
    constexpr int XN = SPEC ? (NW - CW) * 64 : NT;
    constexpr int XLOADS = MROWS * PIECES / XN;
    constexpr int XROWSTEP = XN / PIECES;    // activation rows per load round
    static_assert(XLOADS * XN == MROWS * PIECES, "activation chunk must split over the threads");
    constexpr int ROWB = PIECES * 16;         // LDS row; 16-byte pieces XOR-swizzled by row
    constexpr int XBUF = MROWS * ROWB;
    __shared__ __attribute__((aligned(16))) uint8_t xs[2 * XBUF];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 15, lg = lane >> 4;
    const bool low8 = ln < 8;
    const int K = p.K;
    const int m_base = blockIdx.z * MROWS;
    const int kbeg = blockIdx.y * p.klen;
    const int nchunks = p.klen / KCH;
    const uint32_t rowb = static_cast<uint32_t>(K) * (WF8 ? 1 : 2);   // weight row bytes

    // the first CW waves stream weight rows; the rest (CW < NW) only stage
    // the activation chunks
    const bool streams = !SPEC || wave < CW;
    // weight rows of this wave: rowA + 0..7 (MFMA rows 0..7), rowB + 0..7 (8..15)
    const int gw = blockIdx.x * CW + wave;
    int rowA, rowB;
    if constexpr (EPI == kEpiRope) {
        const int wph = p.D / 16;            // waves per head: 8 rotation pairs each
        const int head = gw / wph;
        rowA = head * p.D + (gw - head * wph) * 8;
        rowB = rowA + p.D / 2;
    } else if constexpr (EPI == kEpiSwiglu) {
        rowA = gw * 8;
        rowB = p.N / 2 + gw * 8;
    } else {
        rowA = gw * 16;
        rowB = rowA + 8;
    }

    const uint32_t piece = ((ln >> 3) * 4 + lg) * 16;
    const uint8_t* wp0 = reinterpret_cast<const uint8_t*>(p.W) + (rowA + (ln & 7)) * static_cast<size_t>(rowb) +
                         piece + static_cast<size_t>(kbeg) * (WF8 ? 1 : 2);
    const uint8_t* wp1 = reinterpret_cast<const uint8_t*>(p.W) + (rowB + (ln & 7)) * static_cast<size_t>(rowb) +
                         piece + static_cast<size_t>(kbeg) * (WF8 ? 1 : 2);
    auto load_w = [&](u32x4* dst, int c) {
#pragma unroll
        for (int c2 = 0; c2 < LINES; ++c2) {
            const size_t o = static_cast<size_t>(c) * KCH * (WF8 ? 1 : 2) + c2 * 128;
            dst[2 * c2] = load_stream(wp0 + o);
            dst[2 * c2 + 1] = load_stream(wp1 + o);
        }
    };
    const int xt = SPEC ? tid - CW * 64 : tid;   // index among the staging threads
    u32x4 xr[XLOADS];
    auto load_x = [&](int c) {
#pragma unroll
        for (int i = 0; i < XLOADS; ++i) {
            const int m = min(m_base + xt / PIECES + i * XROWSTEP, p.M - 1);
            xr[i] = *reinterpret_cast<const u32x4*>(p.X + static_cast<size_t>(m) * K + kbeg + c * KCH +
                                                    (xt % PIECES) * 8);
        }
    };
    auto store_x = [&](int buf) {
#pragma unroll
        for (int i = 0; i < XLOADS; ++i) {
            const int r = xt / PIECES + i * XROWSTEP, pc = xt % PIECES;
            *reinterpret_cast<u32x4*>(xs + buf * XBUF + r * ROWB + ((pc ^ (r & (PIECES - 1))) * 16)) = xr[i];
        }
    };

    f32x4 acc[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) acc[j] = f32x4{0, 0, 0, 0};

    // one MFMA k-step: A operand a (16 weight rows), B from activation piece pc
    auto kstep = [&](const u32x4& a, int pc, int buf) {
        u32x4 b[MB];
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            const int r = 16 * j + ln;
            b[j] = *reinterpret_cast<const u32x4*>(xs + buf * XBUF + r * ROWB +
                                                   ((pc ^ (r & (PIECES - 1))) * 16));
        }
#pragma unroll
        for (int j = 0; j < MB; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b[j]), acc[j], 0, 0, 0);
    };
    auto compute = [&](u32x4* wa, int buf) {
        if constexpr (WF8) {
            // a fixed-up half line holds 16 fp8 weights per lane, k = base +
            // 16 lg + 0..15; each 8 of them (exactly bf16 after conversion)
            // are one k-step, against activation piece base/8 + 2 lg (+1)
#pragma unroll
            for (int c2 = 0; c2 < LINES; ++c2) {
                fix_lines(wa[2 * c2], wa[2 * c2 + 1], low8);
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const u32x4& raw = wa[2 * c2 + hh];
                    const int pc = (c2 * 128 + hh * 64) / 8 + 2 * lg;
                    kstep(fp8x8_to_bf16(raw[0], raw[1]), pc, buf);
                    kstep(fp8x8_to_bf16(raw[2], raw[3]), pc + 1, buf);
                }
            }
            return;
        }
#pragma unroll
        for (int c2 = 0; c2 < LINES; ++c2) {
            fix_lines(wa[2 * c2], wa[2 * c2 + 1], low8);
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int kc = 2 * c2 + kk;
                const int pc = 4 * kc + lg;
                u32x4 b[MB];
#pragma unroll
                for (int j = 0; j < MB; ++j) {
                    const int r = 16 * j + ln;
                    b[j] = *reinterpret_cast<const u32x4*>(xs + buf * XBUF + r * ROWB +
                                                           ((pc ^ (r & (PIECES - 1))) * 16));
                }
#pragma unroll
                for (int j = 0; j < MB; ++j)
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, wa[kc]), __builtin_bit_cast(bf16x8, b[j]), acc[j],
                        0, 0, 0);
            }
        }
        (void)KC;
    };

    if constexpr (SPEC) {
        // Chunk c lives in buffer c & 1. Barrier 0 follows chunk 0's
        // staging; barrier c + 1 follows both the streaming waves' reads of
        // chunk c and the helpers' stores of chunk c + 1 into the other
        // buffer (whose previous chunk, c - 1, was read before barrier c).
        // Both sides pass nchunks barriers.
        if (!streams) {
            load_x(0);
            store_x(0);
            if (nchunks > 1) load_x(1);
            __syncthreads();
            for (int c = 0; c + 1 < nchunks; ++c) {
                store_x((c + 1) & 1);             // registers loaded one chunk ago
                if (c + 2 < nchunks) load_x(c + 2);
                __syncthreads();
            }
            return;
        }
        u32x4 wa0[2 * LINES], wa1[2 * LINES];
        load_w(wa0, 0);
        __syncthreads();
        auto sstep = [&](u32x4* now, u32x4* later, int c, auto more_tag) {
            constexpr bool MORE = decltype(more_tag)::value;
            if constexpr (MORE) load_w(later, c + 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(now, c & 1);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (MORE) __syncthreads();
        };
        using More = std::integral_constant<bool, true>;
        using Last = std::integral_constant<bool, false>;
        int c = 0;
        for (; c + 2 < nchunks; c += 2) {
            sstep(wa0, wa1, c, More{});
            sstep(wa1, wa0, c + 1, More{});
        }
        if (c + 1 < nchunks) {
            sstep(wa0, wa1, c, More{});
            sstep(wa1, wa0, c + 1, Last{});
        } else {
            sstep(wa0, wa1, c, Last{});
        }
        gemm_epilogue<MB, EPI>(p, acc, rowA, rowB, m_base, ln, lg);
        return;
    }
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

    gemm_epilogue<MB, EPI>(p, acc, rowA, rowB, m_base, ln, lg);
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
    *reinterpret_cast<u32x2*>(Y + i) = pack4_bf16(s);
}

// act[m][j..j+3] = swiglu of the split sums of gate (column j) and up
// (column I + j); 4 outputs per thread.
__global__ __launch_bounds__(256) void gemm_split_swiglu(const float* __restrict__ part,
                                                         uint16_t* __restrict__ act, int M, int I,
                                                         int splits) {
    const int i = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= M * I) return;
    const int m = i / I, j = i - m * I;
    const size_t MN = static_cast<size_t>(M) * 2 * I;
    const float* g0 = part + static_cast<size_t>(m) * 2 * I + j;
    f32x4 g = *reinterpret_cast<const f32x4*>(g0);
    f32x4 u = *reinterpret_cast<const f32x4*>(g0 + I);
    for (int k = 1; k < splits; ++k) {
        g += *reinterpret_cast<const f32x4*>(g0 + k * MN);
        u += *reinterpret_cast<const f32x4*>(g0 + k * MN + I);
    }
    f32x4 a;
#pragma unroll
    for (int r = 0; r < 4; ++r) a[r] = swiglu_bf16(bf16_round_f32(g[r]), bf16_round_f32(u[r]));
    *reinterpret_cast<u32x2*>(act + i) = pack4_bf16(a);
}

// K splits: the smallest divisor of K/kch giving at least `target` workgroups
// (KCMM_GEMM_WGS, default 256: fewer, longer splits measured faster than
// 512-1024 at the Llama-3-8B decode shapes) with each split at least two
// chunks long; at most 16.
int choose_splits(int N, int K, int kch, int mgroups) {
    const int chunks = K / kch;
    const int forced = dev::tunable_or(dev::Tun::kGemmSplits, 0);
    if (forced >= 1 && forced <= 16 && chunks % forced == 0) return forced;
    const int target = dev::tunable_or(dev::Tun::kGemmWgs, 256);
    const int tiles = (N / 64) * mgroups;
    int best = 1;
    for (int s = 1; s <= std::min(chunks, 16); ++s) {
        if (chunks % s) continue;
        if (chunks / s < 2 && s > 1) break;
        best = s;
        if (tiles * s >= target) break;
    }
    return best;
}

// Tile shape by M: token blocks per pass (the activation chunk, M x KCH
// bf16, is 32 KiB).
// fp8 weights need at least 128-element chunks (one 128-byte weight line).
template <typename F>
bool by_m(int M, F&& f, bool wf8 = false) {
    if (M <= 16) return f(std::integral_constant<int, 1>{}, std::integral_constant<int, 256>{});
    if (M <= 32) return f(std::integral_constant<int, 2>{}, std::integral_constant<int, 256>{});
    if (M <= 64) return f(std::integral_constant<int, 4>{}, std::integral_constant<int, 256>{});
    if (M <= 128) return f(std::integral_constant<int, 8>{}, std::integral_constant<int, 128>{});
    if (wf8) return f(std::integral_constant<int, 16>{}, std::integral_constant<int, 128>{});
    return f(std::integral_constant<int, 16>{}, std::integral_constant<int, 64>{});
}

int splits_for(int M, int N, int K, bool wf8 = false) {
    int s = 1;
    by_m(M, [&](auto mb, auto kch) {
        const int mgroups = (M + 16 * mb.value - 1) / (16 * mb.value);
        s = choose_splits(N, K, kch.value, mgroups);
        return true;
    }, wf8);
    return s;
}

// Launch the streaming kernel with `splits` K splits; splits > 1 or
// want_partials writes fp32 partials [splits][M][N] to the stream's workspace
// (returned in *part) instead of running the epilogue.
template <int EPI, bool WF8 = false>
bool launch_stream(GemmParams p, int splits, bool want_partials, float** part, uint64_t stream,
                   std::string* err) {
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    p.part = nullptr;
    if (splits > 1 || want_partials) {
        void* ws = nullptr;
        if (!dev::stream_workspace(stream, 1, static_cast<size_t>(splits) * p.M * p.N * sizeof(float),
                                   &ws, false, err))
            return false;
        p.part = static_cast<float*>(ws);
    }
    if (part) *part = p.part;
    p.klen = p.K / splits;
    return by_m(p.M, [&](auto mb, auto kch) {
        constexpr int MB = decltype(mb)::value, KCH = decltype(kch)::value;
        if constexpr (WF8 && KCH < 128) {
            *err = "fp8 weights need 128-element chunks";
            return false;
        } else {
            const unsigned mg = static_cast<unsigned>((p.M + 16 * MB - 1) / (16 * MB));
            // unsplit plain and SwiGLU products (the lm_head and gate/up at
            // decode): 8-wave workgroups, so that one staged activation
            // chunk serves 128 weight rows (KCMM_GEMM_WAVES=4 keeps 4-wave
            // workgroups)
            bool wide = false;
            if constexpr (EPI == kEpiPlain || EPI == kEpiSwiglu)
                wide = p.part == nullptr && p.N % 128 == 0 &&
                       dev::tunable_or(dev::Tun::kGemmWaves, 8) == 8;
            // split products at one token group (QKV, O and down at decode):
            // 8-wave workgroups in which helper waves stage the activation
            // chunks and the streaming waves only stream weights and run the
            // MFMAs, so that the two paths overlap (KCMM_GEMM_HELPERS=0 keeps
            // 4-wave workgroups). A product whose 16-row waves over all
            // splits number 256 x 6 (QKV at 4 splits: 384 four-wave
            // workgroups, two on half the CUs) takes 6 streaming waves, one
            // workgroup per CU; other split products 4.
            bool helpers = false;
            if constexpr (EPI == kEpiRope || EPI == kEpiPlain) {
                helpers = mg == 1 && p.part != nullptr &&
                          dev::tunable_or(dev::Tun::kGemmHelpers, 1) != 0;
                const int waves16 = p.N / 16;   // per split
                if (helpers && waves16 % 6 == 0 && waves16 / 6 * splits == 256)
                    hipLaunchKernelGGL((gemm_bf16_stream<MB, KCH, EPI, WF8, 8, 6>),
                                       dim3(waves16 / 6, splits, 1), dim3(512), 0, s, p);
                else if (helpers)
                    hipLaunchKernelGGL((gemm_bf16_stream<MB, KCH, EPI, WF8, 8, 4>),
                                       dim3(p.N / 64, splits, 1), dim3(512), 0, s, p);
            }
            // unsplit plain and SwiGLU products: 12-wave workgroups, 8 waves
            // streaming 128 weight rows and 4 helpers staging activations
            // (three waves per SIMD; fp8 gate/up and the lm_head gain, bf16
            // gate/up is unchanged)
            if constexpr (EPI == kEpiPlain || EPI == kEpiSwiglu) {
                if (wide && mg == 1 && dev::tunable_or(dev::Tun::kGemmHelpers, 1) != 0) {
                    hipLaunchKernelGGL((gemm_bf16_stream<MB, KCH, EPI, WF8, 12, 8>),
                                       dim3(p.N / 128, 1, 1), dim3(768), 0, s, p);
                    wide = false;
                    helpers = true;
                }
            }
            if (wide) {
                if constexpr (EPI == kEpiPlain || EPI == kEpiSwiglu) {
                    const dim3 grid(p.N / 128, 1, mg);
                    hipLaunchKernelGGL((gemm_bf16_stream<MB, KCH, EPI, WF8, 8>), grid, dim3(512), 0,
                                       s, p);
                }
            } else if (!helpers) {
                const dim3 grid(p.N / 64, splits, mg);
                hipLaunchKernelGGL((gemm_bf16_stream<MB, KCH, EPI, WF8>), grid, dim3(256), 0, s, p);
            }
            KCMM_HIP_CHECK(hipGetLastError(), err);
            return true;
        }
    }, WF8);
}

// launch_stream on bf16 weights, or on fp8-e4m3 weights when p.wscale is set
template <int EPI>
bool launch_weights(const GemmParams& p, int splits, bool want_partials, float** part,
                    uint64_t stream, std::string* err) {
    if (p.wscale != nullptr)
        return launch_stream<EPI, true>(p, splits, want_partials, part, stream, err);
    return launch_stream<EPI>(p, splits, want_partials, part, stream, err);
}

bool shape_ok(uint32_t m, uint32_t n, uint32_t k, std::string* err) {
    if (m == 0 || n % 64 != 0 || k % 256 != 0 || n == 0 || k == 0) {
        *err = "gemm_bf16 needs m > 0, n % 64 == 0 and k % 256 == 0";
        return false;
    }
    if (static_cast<uint64_t>(m) * k >= (1ull << 31) || static_cast<uint64_t>(n) * k >= (1ull << 31) ||
        static_cast<uint64_t>(m) * n >= (1ull << 29)) {
        *err = "gemm_bf16 operand too large";
        return false;
    }
    return true;
}

GemmParams base_params(uint64_t x, uint64_t w, uint32_t m, uint32_t n, uint32_t k) {
    GemmParams p{};
    p.X = reinterpret_cast<const uint16_t*>(x);
    p.W = reinterpret_cast<const uint16_t*>(w);
    p.M = static_cast<int>(m);
    p.N = static_cast<int>(n);
    p.K = static_cast<int>(k);
    return p;
}

}  // namespace

namespace dev {

bool gemm_split_reduce_launch(const float* part, uint16_t* y, const uint16_t* r, int mn,
                              int splits, uint64_t stream, std::string* err) {
    hipLaunchKernelGGL(gemm_split_reduce, dim3((mn / 4 + 255) / 256), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), part, y, r, mn, splits);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

bool gemm_bf16(uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t n, uint32_t k,
               uint64_t stream, std::string* err, uint64_t residual) {
    if (!shape_ok(m, n, k, err)) return false;
    // many tokens: the LDS-tiled MFMA kernel (KCMM_GEMM_TILED=0 keeps the
    // weight-stream kernel)
    if (m > 128 && dev::tunable_or(dev::Tun::kGemmTiled, 1) != 0)
        return gemm_bf16_tiled(x, w, y, m, n, k, stream, residual, err);
    GemmParams p = base_params(x, w, m, n, k);
    p.Y = reinterpret_cast<uint16_t*>(y);
    p.R = reinterpret_cast<const uint16_t*>(residual);
    const int splits = splits_for(p.M, p.N, p.K);
    float* part = nullptr;
    if (!launch_stream<kEpiPlain>(p, splits, false, &part, stream, err)) return false;
    if (splits > 1) {
        const int MN = p.M * p.N;
        hipLaunchKernelGGL(gemm_split_reduce, dim3((MN / 4 + 255) / 256), dim3(256), 0,
                           reinterpret_cast<hipStream_t>(stream), part, p.Y, p.R, MN, splits);
        KCMM_HIP_CHECK(hipGetLastError(), err);
    }
    return true;
}

bool gemm_plan(uint32_t m, uint32_t n, uint32_t k, bool fp8_weights, GemmPlan* plan,
               std::string* err) {
    if (!shape_ok(m, n, k, err)) return false;
    *plan = GemmPlan{};
    if (m > 128 && dev::tunable_or(dev::Tun::kGemmTiled, 1) != 0) {
        plan->kernel = 1;
        gemm_tiled_plan(m, n, k, &plan->splits, &plan->tile);
    } else {
        plan->kernel = 0;
        plan->splits = splits_for(static_cast<int>(m), static_cast<int>(n), static_cast<int>(k),
                                  fp8_weights);
        plan->tile = -1;
    }
    plan->partial_bytes = plan->splits > 1
                              ? static_cast<uint64_t>(plan->splits) * m * n * sizeof(float)
                              : 0;
    return true;
}

bool gemm_fp8w_bf16(uint64_t x, uint64_t w8, uint64_t wscale, uint64_t y, uint32_t m, uint32_t n,
                    uint32_t k, uint64_t stream, std::string* err, uint64_t residual) {
    if (!shape_ok(m, n, k, err)) return false;
    if (wscale == 0) {
        *err = "fp8 weights need their row scales";
        return false;
    }
    // many tokens: the LDS-tiled kernel (KCMM_GEMM_TILED=0 keeps the
    // weight-stream kernel)
    if (m > 128 && dev::tunable_or(dev::Tun::kGemmTiled, 1) != 0)
        return gemm_tiled(x, w8, wscale, y, m, n, k, stream, residual, err);
    GemmParams p = base_params(x, w8, m, n, k);
    p.Y = reinterpret_cast<uint16_t*>(y);
    p.R = reinterpret_cast<const uint16_t*>(residual);
    p.wscale = reinterpret_cast<const float*>(wscale);
    const int splits = splits_for(p.M, p.N, p.K, true);
    float* part = nullptr;
    if (!launch_stream<kEpiPlain, true>(p, splits, false, &part, stream, err)) return false;
    if (splits > 1) return gemm_split_reduce_launch(part, p.Y, p.R, p.M * p.N, splits, stream, err);
    return true;
}

bool gemm_bf16_partials(uint64_t x, uint64_t w, uint32_t m, uint32_t n, uint32_t k,
                        uint64_t stream, float** part, int* splits, std::string* err,
                        uint64_t wscale) {
    if (!shape_ok(m, n, k, err)) return false;
    GemmParams p = base_params(x, w, m, n, k);
    p.wscale = reinterpret_cast<const float*>(wscale);
    *splits = splits_for(p.M, p.N, p.K, wscale != 0);
    return launch_weights<kEpiPlain>(p, *splits, true, part, stream, err);
}

bool gemm_bf16_swiglu(uint64_t x, uint64_t w_gate_up, uint64_t act, uint32_t m, uint32_t inter,
                      uint32_t k, uint64_t stream, std::string* err, uint64_t wscale) {
    if (inter == 0 || inter % 32 != 0) {
        *err = "gemm_bf16_swiglu needs intermediate % 32 == 0";
        return false;
    }
    if (!shape_ok(m, 2 * inter, k, err)) return false;
    GemmParams p = base_params(x, w_gate_up, m, 2 * inter, k);
    p.Y = reinterpret_cast<uint16_t*>(act);
    p.wscale = reinterpret_cast<const float*>(wscale);
    const int splits = splits_for(p.M, p.N, p.K, wscale != 0);
    float* part = nullptr;
    if (!launch_weights<kEpiSwiglu>(p, splits, false, &part, stream, err)) return false;
    if (splits > 1) {
        const int n = p.M * static_cast<int>(inter);
        hipLaunchKernelGGL(gemm_split_swiglu, dim3((n / 4 + 255) / 256), dim3(256), 0,
                           reinterpret_cast<hipStream_t>(stream), part, p.Y, p.M,
                           static_cast<int>(inter), splits);
        KCMM_HIP_CHECK(hipGetLastError(), err);
    }
    return true;
}

bool gemm_bf16_rope_append(uint64_t x, uint64_t w_qkv, uint32_t m, uint32_t k,
                           const RopeAppendArgs& a, std::string* err, uint64_t wscale) {
    const uint32_t D = a.head_dim;
    const uint64_t n = static_cast<uint64_t>(a.num_q_heads + 2 * a.kv_heads) * D;
    if (D == 0 || D % 16 != 0 || n % 64 != 0 || a.num_q_heads == 0 || a.kv_heads == 0 ||
        m != a.batch) {
        *err = "gemm_bf16_rope_append needs head_dim % 16 == 0, (Hq + 2 Hkv) * head_dim % 64 == 0 "
               "and one token per sequence";
        return false;
    }
    if (!shape_ok(m, static_cast<uint32_t>(n), k, err)) return false;
    if (a.dtype == kDtFP8) {
        // fp8 pages take their rows through the fp8 page writer: the
        // projection leaves fp32 partials, the RoPE kernel sums them
        float* part = nullptr;
        int splits = 1;
        return gemm_bf16_partials(x, w_qkv, m, static_cast<uint32_t>(n), k, a.stream, &part,
                                  &splits, err, wscale) &&
               rope_append_from_partials(a, part, splits, err);
    }
    GemmParams p = base_params(x, w_qkv, m, static_cast<uint32_t>(n), k);
    p.q_out = reinterpret_cast<uint16_t*>(a.q_out);
    p.k_base = reinterpret_cast<uint8_t*>(a.k_base);
    p.v_base = reinterpret_cast<uint8_t*>(a.v_base);
    p.block_tables = reinterpret_cast<const int32_t*>(a.block_tables);
    p.seq_lens = reinterpret_cast<const int32_t*>(a.seq_lens);
    p.offsets_f16 = reinterpret_cast<const uint64_t*>(a.offsets_f16);
    p.inv_freq = reinterpret_cast<const float*>(a.inv_freq);
    p.hq = static_cast<int>(a.num_q_heads);
    p.hkv = static_cast<int>(a.kv_heads);
    p.D = static_cast<int>(D);
    p.block_size = static_cast<int>(a.block_size);
    p.mbps = static_cast<int>(a.mbps);
    p.row_bytes = static_cast<int>(a.row_bytes);
    p.wscale = reinterpret_cast<const float*>(wscale);
    const int splits = splits_for(p.M, p.N, p.K, wscale != 0);
    float* part = nullptr;
    if (!launch_weights<kEpiRope>(p, splits, false, &part, a.stream, err)) return false;
    if (splits > 1) return rope_append_from_partials(a, part, splits, err);
    return true;
}

}  // namespace dev
}  // namespace kcmm
