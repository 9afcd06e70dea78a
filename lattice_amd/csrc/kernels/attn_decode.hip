// Paged decode attention for gfx950 (MI355X).
//
// Semantics (ref src/cuda/kernels/kcmm_vllm_paged_attn.cu:10-102): for every
// sequence b and query head h, with kv head g = h*Hkv/Hq and L = seq_lens[b],
//   out[b][h] = sum_t softmax_t(scale * q[b][h].K[t]) V[t],  t < L,
// where token t of sequence b lives in page block_tables[b][t/bs] at byte
// offset offsets_f16[page]*2, row (t%bs), kv head g, of the layer's K / V
// region.  L <= 0 writes zeros.  Accumulation is fp32.
//
// MI355X design (the reference uses one scalar thread per (b, h)):
//  * the work is the list of 32-token tiles of every (sequence b, block of
//    HW kv heads), b-major; every workgroup of HW waves (wave w = kv head
//    hb*HW + w of the block) streams an equal contiguous slice of that list,
//    so a ragged batch leaves no tail of idle CUs, and the waves of a
//    workgroup read the same tokens' rows of neighbouring heads together:
//    with HW = Hkv a workgroup reads whole token rows (all heads, 2 KiB
//    contiguous at the Llama-3-8B shape) instead of one head's 256-byte
//    pieces at a 2 KiB stride (used for fp8 pages, HW = 8; 16-bit pages
//    run HW = 1, one wave per workgroup);
//  * one tile read serves all G = Hq/Hkv query heads of its kv head (GQA
//    reuse: each K/V byte is read from HBM once);
//  * every load instruction covers eight tokens x 128 contiguous bytes (whole
//    cache lines, nontemporal); one DPP row rotation and one select per dword
//    then turn two such loads into MFMA operand layout (16 tokens x 64 bytes);
//  * page addresses are wave-uniform scalar loads issued one tile ahead;
//  * S^T = K Q^T on v_mfma_f32_16x16x32 (token rows x head columns), online
//    softmax in the log2 domain with cross-lane max by lane shuffles;
//  * O^T += V^T P^T on the same MFMA: V^T is produced in registers by
//    multiplying each V fragment with a 0/1 selection matrix (exact for
//    16-bit values), so the kernel touches no LDS;
//  * a (b, g) whose tiles lie inside one wave's slice is normalised and
//    written by that wave; one that spans waves leaves fp32 partials
//    (unnormalised output, max, denominator) that attn_decode_merge combines
//    by log-sum-exp.
#include <algorithm>
#include <atomic>
#include <climits>
#include <mutex>
#include <string>
#include <vector>
#include <cmath>
#include <cstdlib>
#include <type_traits>
#include <utility>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

// Device scratch of the no-allocation entry point
// (kcmm_paged_attn_decode_bf16_noalloc_on_stream): the streaming kernel's
// idle-load region, partial results and segment table, carved from one
// file-scope array instead of the per-stream workspace.  Every GPU holds its
// own copy for the life of the process; host code uses only the address
// hipGetSymbolAddress reports for the current device.
constexpr size_t kNoAllocScratchBytes = size_t(24) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;

// Per device: the address of `scratch` there (hipGetSymbolAddress, once),
// and one event (created once) that marks the end of the last no-alloc
// call's kernels.  A call on a different stream waits on that event first,
// so calls on two streams of one GPU take turns with the array instead of
// overwriting each other's partials.  All no-alloc calls hold g_noalloc_mu
// from that wait until their own event record.
struct NoAllocDevice {
    uint8_t* scratch = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool used = false;
};
std::mutex g_noalloc_mu;
NoAllocDevice g_noalloc[kMaxDevices];

// Event timing of the streaming kernel (dev::attn_stream_timing_start /
// stop): event pairs created at start on the then-current device and taken
// in order by the streaming-kernel launches that follow on that device.  Off
// by default; a launch under graph capture takes no pair.
struct StreamTiming {
    std::atomic<bool> on{false};
    std::mutex mu;
    int device = -1;
    uint32_t next = 0;
    std::vector<hipEvent_t> ev;   // pair i: ev[2i] before the launch, ev[2i+1] after it
};
StreamTiming g_timing;

// The event pair for a streaming-kernel launch on s: {nullptr, nullptr}
// when timing is off, every pair is taken, s is capturing or belongs to
// another device.
std::pair<hipEvent_t, hipEvent_t> timing_pair(hipStream_t s) {
    if (!g_timing.on.load(std::memory_order_acquire)) return {nullptr, nullptr};
    std::lock_guard<std::mutex> lk(g_timing.mu);
    int dev = -1;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (!g_timing.on.load(std::memory_order_relaxed) || 2 * (g_timing.next + 1) > g_timing.ev.size() ||
        hipGetDevice(&dev) != hipSuccess || dev != g_timing.device ||
        hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return {nullptr, nullptr};
    const uint32_t i = g_timing.next++;
    return {g_timing.ev[2 * i], g_timing.ev[2 * i + 1]};
}

// The current device's state, set up on its first call; g_noalloc_mu held.
bool noalloc_device(NoAllocDevice** out, std::string* err) {
    int dev = 0;
    KCMM_HIP_CHECK(hipGetDevice(&dev), err);
    if (dev < 0 || dev >= kMaxDevices) {
        *err = "decode attention (no-alloc): device ordinal out of range";
        return false;
    }
    NoAllocDevice& d = g_noalloc[dev];
    if (d.scratch == nullptr) {
        void* p = nullptr;
        KCMM_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), err);
        KCMM_HIP_CHECK(hipEventCreateWithFlags(&d.done, hipEventDisableTiming), err);
        d.scratch = static_cast<uint8_t*>(p);
    }
    *out = &d;
    return true;
}

struct AttnParams {
    const uint8_t* q;       // [B][Hq][D] 16-bit elements
    uint8_t* out;           // [B][Hq][D]
    const uint8_t* k_base;
    const uint8_t* v_base;
    const int32_t* block_tables;
    const int32_t* seq_lens;
    const uint64_t* offsets_f16;
    float* part_acc;        // [units][G][D]: [waves][2] (slot 0: head of slice, 1: tail),
                            // then [B][Hkv][kSegPieces] from seg_unit0
    float* part_ml;         // [units][G][2]  (max in log2 units, denominator)
    size_t seg_unit0;       // first segment-indexed unit
    int2* seg_info;         // [B][Hkv]: (first slice, slices) of each (b, g); slices <= 1: no merge
    int batch, num_q_heads, kv_heads, group, block_size, mbps;
    int row_bytes, data_bytes;
    int hw;                 // waves per workgroup = kv heads per head block (divides Hkv)
    int total_waves;        // slices = workgroups of the streaming kernel
    int min_tiles;          // smallest slice a wave takes
    float scale_log2;       // scale * log2(e)
};

// Pieces 0 .. kSegPieces-1 of a split (b, g) are stored at units indexed by
// (b, g), so the merge can load them before it has read the segment record;
// later pieces stay at the unit of their slice's wave.
constexpr int kSegPieces = 4;

__device__ __forceinline__ float wave_max_across_groups(float x) {
    // lanes j, j+16, j+32, j+48 hold the same column; combine them.
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

__device__ __forceinline__ float wave_sum_across_groups(float x) {
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

__device__ __forceinline__ int wave_sum(int x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == kDtF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                       0);
}

// Tokens of sequence b that attention reads (ref kernel: the table holds at
// most mbps * bs of them).
__device__ __forceinline__ int clamp_len(int L, int cap) { return L < 0 ? 0 : (L > cap ? cap : L); }
__device__ __forceinline__ int tiles_of(int L) { return (L + 31) >> 5; }

// Slice length of one workgroup for `total` tiles.
__device__ __forceinline__ int wave_slice(int total, const AttnParams& p) {
    const int per = (total + p.total_waves - 1) / p.total_waves;
    return per > p.min_tiles ? per : p.min_tiles;
}

// One 32-token tile: 2 halves of 16 tokens, KC 16-byte fragments per lane
// each; after fix_lines, k[h][kc] of lane (ln, lg) holds bytes
// (4kc + lg)*16 .. +16 of token 16h + ln's head row (the MFMA A layout).
template <int KC>
struct Tile {
    u32x4 k[2][KC];
    u32x4 v[2][KC];
};

// Row rotation by 8 inside each 16-lane row (DPP row_ror:8; its own inverse).
__device__ __forceinline__ uint32_t ror8(uint32_t x) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x128, 0xF, 0xF, false));
}

// x was loaded as: lane (r, lg) <- token (r & 7), bytes (4*(r >> 3) + lg)*16
// of a 128-byte line; y the same for tokens 8..15.  Afterwards x holds the
// first 64 bytes of tokens 0..15 and y the second 64 bytes, lane r = token r.
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

// B operand of a 16x16x32 MFMA that selects 16 consecutive k indices:
// E[k][j] = (k == 16*sub + j).  Multiplying an A operand by it returns the
// selected A columns in C layout, i.e. transposed relative to the A layout.
template <int DT>
__device__ __forceinline__ u32x4 select_operand(int sub, int ln, int lg) {
    constexpr uint32_t one = DT == kDtF16 ? 0x3C00u : 0x3F80u;
    u32x4 e = u32x4{0, 0, 0, 0};
    const int k = 16 * sub + ln;          // the k that column ln selects
    if ((k >> 3) == lg) {
        const int t = k & 7;              // item within the lane's 8 k values
        e[t >> 1] = (t & 1) ? (one << 16) : one;
    }
    return e;
}

// Two fp32 values that hold exactly representable 16-bit values -> packed pair.
template <int DT>
__device__ __forceinline__ uint32_t pack_exact(float lo, float hi) {
    if constexpr (DT == kDtF16) {
        return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
    } else {
        return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
    }
}

// Online-softmax update of one tile (see the file comment for the layouts).
template <int DT, int D>
__device__ __forceinline__ void compute_tile(const Tile<D / 32>& t, const u32x4* qf,
                                             const u32x4* esel, int tbase, int L,
                                             float scale_log2, float& m_run, float& l_run,
                                             f32x4* acc, int lg) {
    constexpr int KC = D / 32;
    constexpr int DB = D / 16;
    f32x4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        s[h] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) s[h] = mfma16x16x32<DT>(t.k[h][kc], qf[kc], s[h]);
    }
    float sv[8];
    float mt = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = tbase + h * 16 + lg * 4 + r;
            const float x = tok < L ? s[h][r] * scale_log2 : -INFINITY;
            sv[h * 4 + r] = x;
            mt = fmaxf(mt, x);
        }
    }
    mt = wave_max_across_groups(mt);
    const float m_new = fmaxf(m_run, mt);
    const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
    float pv[8];
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        pv[i] = __builtin_amdgcn_exp2f(sv[i] - m_new);
        psum += pv[i];
    }
    l_run = l_run * corr + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < DB; ++i) acc[i] *= corr;

    // P^T as the B operand: k-slot (lg, i) = token (i<4 ? 4lg+i : 16+4lg+i-4).
    u32x4 pf;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        pf[i] = f32_to_elem<DT>(pv[2 * i]) | (f32_to_elem<DT>(pv[2 * i + 1]) << 16);
    // V^T for the PV product, by selection MFMAs, one 16-dim block at a time
    // (keeps few transposed values live): lane (dim ln, group lg) receives
    // V[h*16 + 4lg + r][16db + ln] for r = 0..3 from half h.
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        const f32x4 v0 = mfma16x16x32<DT>(t.v[0][db >> 1], esel[db & 1], f32x4{0, 0, 0, 0});
        const f32x4 v1 = mfma16x16x32<DT>(t.v[1][db >> 1], esel[db & 1], f32x4{0, 0, 0, 0});
        u32x4 va;
        va[0] = pack_exact<DT>(v0[0], v0[1]);
        va[1] = pack_exact<DT>(v0[2], v0[3]);
        va[2] = pack_exact<DT>(v1[0], v1[1]);
        va[3] = pack_exact<DT>(v1[2], v1[3]);
        acc[db] = mfma16x16x32<DT>(va, pf, acc[db]);
    }
}

// Eight e4m3 values (two dwords) -> eight bf16, exactly (every e4m3 value
// is a bf16 value); the page scale is applied outside, in fp32.
__device__ __forceinline__ u32x4 fp8x8_to_bf16(uint32_t d0, uint32_t d1) {
    u32x4 r;
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, false));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, 1.0f, true));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, false));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, 1.0f, true));
    return r;
}

// fp8 page tile (head_dim 128): t.k[h][0] holds bytes 16lg..16lg+15 and
// t.k[h][1] bytes 64+16lg..+15 of token 16h + ln's head row.  MFMA k-step kc
// takes the eight elements at (kc>>1)*64 + (kc&1)*8 + 16lg; Q is read in the
// same order.  S is scaled by the K scale of each token's (page, kv head),
// P by the V scale before the PV product (l uses the unscaled P), so the
// result equals attention over the dequantized pages.  acc[db] then holds
// the dims given by fp8_dim_offset.
__device__ __forceinline__ void compute_tile_fp8(const Tile<2>& t, const u32x4* qf,
                                                 const u32x4* esel, int tbase, int L,
                                                 float scale_log2, const float* ks,
                                                 const float* vs, float& m_run, float& l_run,
                                                 f32x4* acc, int lg) {
    f32x4 s[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        s[h] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
            const u32x4& raw = t.k[h][kc >> 1];
            const u32x4 a = (kc & 1) ? fp8x8_to_bf16(raw[2], raw[3]) : fp8x8_to_bf16(raw[0], raw[1]);
            s[h] = mfma16x16x32<kDtBF16>(a, qf[kc], s[h]);
        }
    }
    // rows 4lg + r of half h are tokens of 8-token group 2h (lg < 2) or 2h+1
    float sv[8];
    float mt = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float kscale = (lg < 2 ? ks[2 * h] : ks[2 * h + 1]) * scale_log2;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = tbase + h * 16 + lg * 4 + r;
            const float x = tok < L ? s[h][r] * kscale : -INFINITY;
            sv[h * 4 + r] = x;
            mt = fmaxf(mt, x);
        }
    }
    mt = wave_max_across_groups(mt);
    const float m_new = fmaxf(m_run, mt);
    const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
    float pv[8];
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        pv[i] = __builtin_amdgcn_exp2f(sv[i] - m_new);
        psum += pv[i];
    }
    l_run = l_run * corr + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] *= corr;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float vscale = lg < 2 ? vs[2 * h] : vs[2 * h + 1];
#pragma unroll
        for (int r = 0; r < 4; ++r) pv[h * 4 + r] *= vscale;
    }
    u32x4 pf;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        pf[i] = f32_to_elem<kDtBF16>(pv[2 * i]) | (f32_to_elem<kDtBF16>(pv[2 * i + 1]) << 16);
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
        const u32x4& r0 = t.v[0][kc >> 1];
        const u32x4& r1 = t.v[1][kc >> 1];
        const u32x4 f0 = (kc & 1) ? fp8x8_to_bf16(r0[2], r0[3]) : fp8x8_to_bf16(r0[0], r0[1]);
        const u32x4 f1 = (kc & 1) ? fp8x8_to_bf16(r1[2], r1[3]) : fp8x8_to_bf16(r1[0], r1[1]);
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const f32x4 v0 = mfma16x16x32<kDtBF16>(f0, esel[sub], f32x4{0, 0, 0, 0});
            const f32x4 v1 = mfma16x16x32<kDtBF16>(f1, esel[sub], f32x4{0, 0, 0, 0});
            u32x4 va;
            va[0] = pack_exact<kDtBF16>(v0[0], v0[1]);
            va[1] = pack_exact<kDtBF16>(v0[2], v0[3]);
            va[2] = pack_exact<kDtBF16>(v1[0], v1[1]);
            va[3] = pack_exact<kDtBF16>(v1[2], v1[3]);
            acc[2 * kc + sub] = mfma16x16x32<kDtBF16>(va, pf, acc[2 * kc + sub]);
        }
    }
}

// First of the four consecutive dims that lane group lg holds in acc[db]
// (rows 4lg .. 4lg+3 of the O^T block).
template <bool F8>
__device__ __forceinline__ int dim_offset(int db, int lg) {
    if constexpr (F8) {
        const int kc = db >> 1, sub = db & 1;
        return (kc >> 1) * 64 + (kc & 1) * 8 + 32 * sub + 4 * lg + (lg >= 2 ? 8 : 0);
    } else {
        return 16 * db + 4 * lg;
    }
}

// Streaming decode attention: workgroup s of HW waves takes the slice
// [s*per, s*per + per) of the b-major (sequence, head block, tile) list, wave
// w the kv head hb*HW + w of each entry, with P tiles in flight per wave.
// The waves share nothing (no LDS, no barrier): the workgroup only places
// the waves that read one token row's heads on one CU at one time.
// Read-only tables come as separate restrict arguments so that wave-uniform
// reads of them compile to scalar loads, which do not wait behind the vector
// loads in flight.  Past the end of its slice a wave keeps issuing loads, of
// `idle` (a small workspace region that stays in L2), so that every step has
// the same loads outstanding and the waits stay exact.
template <int DT, int D, int BS, int P>
__global__ __launch_bounds__(P == 2 ? 512 : 256) __attribute__((amdgpu_waves_per_eu(P == 2 ? 2 : 1)))
void attn_decode_stream(AttnParams p, const int32_t* __restrict__ bt,
                        const int32_t* __restrict__ sl, const uint64_t* __restrict__ offs,
                        const uint8_t* __restrict__ kreg, const uint8_t* __restrict__ vreg,
                        const uint8_t* __restrict__ idle) {
    constexpr bool F8 = DT == kDtFP8;
    constexpr int MDT = F8 ? kDtBF16 : DT;     // MFMA, q and out element type
    constexpr int EB = F8 ? 1 : 2;             // bytes per K/V element
    constexpr int KC = D / 32;                 // MFMA k-steps per 16-token half
    constexpr int LINES = D * EB / 128;        // 128-byte lines per head row
    constexpr int TK = 2 * LINES;              // loaded fragments per half
    constexpr int DB = D / 16;
    static_assert(!F8 || D == 128, "fp8 pages take the streaming path at head_dim 128");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int ln = lane & 15;
    const int lg = lane >> 4;
    const int bs = BS > 0 ? BS : p.block_size;
    const int cap = p.mbps * bs;
    const int Hkv = p.kv_heads;
    const int HW = p.hw;
    const int NHB = Hkv / HW;
    const int G = p.group;

    // ---- this workgroup's slice of the tile list ----
    // lane i of chunk c describes sequence c + i: clamped length, tiles
    auto chunk_vals = [&](int c, int& Lc, int& v) {
        const int bb = c + lane;
        Lc = bb < p.batch ? clamp_len(sl[bb], cap) : 0;
        v = NHB * tiles_of(Lc);
    };
    auto inclusive_scan = [&](int v) {
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(v, o);
            if (lane >= o) v += y;
        }
        return v;
    };
    int L0, v0;
    chunk_vals(0, L0, v0);
    const int incl0 = inclusive_scan(v0);
    int total = __shfl(incl0, 63);
    for (int c = 64; c < p.batch; c += 64) {
        int Lc, v;
        chunk_vals(c, Lc, v);
        total += wave_sum(v);
    }
    total = __builtin_amdgcn_readfirstlane(total);
    const int per = wave_slice(total, p);

    // sequences without tokens: zero rows, nothing to merge
    for (int bb = blockIdx.x; bb < p.batch; bb += gridDim.x) {
        if (clamp_len(sl[bb], cap) > 0) continue;
        uint16_t* o = reinterpret_cast<uint16_t*>(p.out) + static_cast<size_t>(bb) * p.num_q_heads * D;
        for (int e = threadIdx.x; e < p.num_q_heads * D; e += HW * 64) o[e] = 0;
        for (int e = threadIdx.x; e < Hkv; e += HW * 64) p.seg_info[bb * Hkv + e] = int2{0, 0};
    }

    const int slice = static_cast<int>(blockIdx.x);
    const int gw = slice * HW + wave;   // this wave's partial-result rows
    const int t0 = slice * per;
    if (t0 >= total) return;
    const int n = min(per, total - t0);

    // sequence holding tile t0, its first tile and its length
    int b = 0, start = 0, Lb = 0;
    {
        unsigned long long hit = __ballot(incl0 > t0);
        if (hit) {
            const int j = __ffsll(static_cast<long long>(hit)) - 1;
            b = j;
            start = __shfl(incl0 - v0, j);
            Lb = __shfl(L0, j);
        } else {
            int base = __shfl(incl0, 63);
            for (int c = 64; c < p.batch; c += 64) {
                int Lc, v;
                chunk_vals(c, Lc, v);
                const int incl = inclusive_scan(v);
                hit = __ballot(base + incl > t0);
                if (hit) {
                    const int j = __ffsll(static_cast<long long>(hit)) - 1;
                    b = c + j;
                    start = base + __shfl(incl - v, j);
                    Lb = __shfl(Lc, j);
                    break;
                }
                base += __shfl(incl, 63);
            }
        }
    }

    // Cursor over the tile list: (sequence, kv head, tile, length, tiles);
    // g = hb*HW + wave advances by HW from one head block to the next.
    struct Cur {
        int b, g, t, L, nt;
        float ks[F8 ? 4 : 1], vs[F8 ? 4 : 1];   // fp8: page scales of the 8-token groups
    };
    Cur ic;  // next tile to issue
    ic.b = __builtin_amdgcn_readfirstlane(b);
    ic.L = __builtin_amdgcn_readfirstlane(Lb);
    ic.nt = tiles_of(ic.L);
    {
        const int rem = t0 - __builtin_amdgcn_readfirstlane(start);
        const int hb = rem / ic.nt;
        ic.g = hb * HW + wave;
        ic.t = rem - hb * ic.nt;
    }
    auto advance = [&](Cur& c) {
        if (++c.t < c.nt) return;
        c.t = 0;
        if ((c.g += HW) < Hkv) return;
        c.g = wave;
        ++c.b;
        c.L = clamp_len(sl[c.b], cap);
        c.nt = tiles_of(c.L);
        // sequences without tokens own no tiles (the slice never ends in them)
        while (c.nt == 0 && c.b + 1 < p.batch) {
            ++c.b;
            c.L = clamp_len(sl[c.b], cap);
            c.nt = tiles_of(c.L);
        }
    };
    // Page-relative byte address of each 8-token group of a tile; groups past
    // the sequence re-read its last group (masked).
    // (fp8: also reads the groups' K / V page scales, a tile ahead of use)
    auto group_bases = [&](Cur& c, uint64_t* gb) {
        const int last8 = (c.L - 1) & ~7;
        const int32_t* row = bt + static_cast<size_t>(c.b) * p.mbps;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int tok = min(c.t * 32 + q * 8, last8);
            const int lb = tok / bs;
            const uint64_t page = offs[row[lb]] * 2ull;
            gb[q] = page + static_cast<uint32_t>((tok - lb * bs) * p.row_bytes + c.g * D * EB);
            if constexpr (F8) {
                const uint64_t sc = page + static_cast<uint32_t>(p.data_bytes + c.g * 4);
                c.ks[q] = *reinterpret_cast<const float*>(kreg + sc);
                c.vs[q] = *reinterpret_cast<const float*>(vreg + sc);
            }
        }
    };

    const uint32_t lo = static_cast<uint32_t>((ln & 7) * p.row_bytes + ((ln >> 3) * 4 + lg) * 16);
    const bool low8 = ln < 8;
    auto issue = [&](Tile<TK>& tl, bool real, const uint64_t* gb) {
        const uint8_t* kb = real ? kreg : idle;
        const uint8_t* vb = real ? vreg : idle;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int c2 = 0; c2 < LINES; ++c2) {
                const uint32_t o = lo + c2 * 128;
                const uint64_t g0 = real ? gb[2 * h] : 0;
                const uint64_t g1 = real ? gb[2 * h + 1] : 0;
                tl.k[h][2 * c2] = load_stream(kb + g0 + o);
                tl.k[h][2 * c2 + 1] = load_stream(kb + g1 + o);
                tl.v[h][2 * c2] = load_stream(vb + g0 + o);
                tl.v[h][2 * c2 + 1] = load_stream(vb + g1 + o);
            }
    };
    // Q^T as the B operand: lane (head ln, group lg) holds Q[ln][kc*32+8lg .. +8].
    // Columns ln >= G repeat head G-1; they are computed and never stored.
    auto load_q = [&](u32x4* qd, const Cur& c) {
        const uint8_t* qrow = p.q + (static_cast<size_t>(c.b) * p.num_q_heads + c.g * G +
                                     min(ln, G - 1)) * D * 2;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            const int e0 = F8 ? (kc >> 1) * 64 + (kc & 1) * 8 + 16 * lg : kc * 32 + lg * 8;
            qd[kc] = *reinterpret_cast<const u32x4*>(qrow + e0 * 2);
        }
    };

    const u32x4 esel[2] = {select_operand<MDT>(0, ln, lg), select_operand<MDT>(1, ln, lg)};
    float m_run = -INFINITY;  // running max (log2 domain) of column ln
    float l_run = 0.0f;       // this lane's share of the softmax denominator
    f32x4 acc[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) acc[i] = f32x4{0, 0, 0, 0};

    // Segment end: normalise and store, or leave a partial in slot
    // 0 (segment began in an earlier slice) / 1 (continues in a later one).
    auto flush = [&](const Cur& c, bool began_here, int i) {
        const float l = wave_sum_across_groups(l_run);
        const bool complete = began_here && c.t == c.nt - 1;
        if (began_here && lane == 0) {
            // the slice where (b, g) begins tells the merge where its parts are
            const int first = t0 + i - c.t;
            const int slices = complete ? 1 : (first + c.nt - 1) / per - slice + 1;
            p.seg_info[c.b * Hkv + c.g] = int2{slice, slices};
        }
        if (ln < G) {
            if (complete) {
                const float inv = 1.0f / l;
                uint16_t* o = reinterpret_cast<uint16_t*>(p.out) +
                              (static_cast<size_t>(c.b) * p.num_q_heads + c.g * G + ln) * D;
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    u32x2 w;
                    w[0] = f32_to_elem<MDT>(acc[db][0] * inv) | (f32_to_elem<MDT>(acc[db][1] * inv) << 16);
                    w[1] = f32_to_elem<MDT>(acc[db][2] * inv) | (f32_to_elem<MDT>(acc[db][3] * inv) << 16);
                    *reinterpret_cast<u32x2*>(o + dim_offset<F8>(db, lg)) = w;
                }
            } else {
                const int piece = slice - (t0 + i - c.t) / per;   // 0 when began_here
                const size_t unit =
                    piece < kSegPieces
                        ? p.seg_unit0 + static_cast<size_t>(c.b * Hkv + c.g) * kSegPieces + piece
                        : static_cast<size_t>(gw) * 2;
                float* pa = p.part_acc + (unit * G + ln) * D;
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    *reinterpret_cast<f32x4*>(pa + dim_offset<F8>(db, lg)) = acc[db];
                if (lg == 0) {
                    p.part_ml[(unit * G + ln) * 2 + 0] = m_run;
                    p.part_ml[(unit * G + ln) * 2 + 1] = l;
                }
            }
        }
        m_run = -INFINITY;
        l_run = 0.0f;
#pragma unroll
        for (int i = 0; i < DB; ++i) acc[i] = f32x4{0, 0, 0, 0};
    };

    // ---- pipeline: buf[k] holds tile i with i % P == k; while tile i is
    // consumed, tiles i+1 .. i+P-1 are in flight and the page addresses of
    // tile i+P are being fetched ----
    u32x4 qf[KC];
    Cur cq[P];
    Tile<TK> buf[P];
    uint64_t gb[4];
    load_q(qf, ic);
    bool began_here = ic.t == 0;
    group_bases(ic, gb);
#pragma unroll
    for (int k = 0; k < P - 1; ++k) {
        cq[k] = ic;
        issue(buf[k], k < n, gb);
        if (k + 1 < n) {
            advance(ic);
            group_bases(ic, gb);
        }
    }

    // With P >= 3 the Q of a new (b, g) is read ahead into qn, before the
    // tile loads of the step, so that waiting for it never drains the tiles
    // in flight behind it (P == 2 has no such tile: qf is refilled directly).
    u32x4 qn[P > 2 ? KC : 1];
    bool q_ready = false;
    auto step = [&](auto phase, int i) {
        constexpr int j = decltype(phase)::value;
        constexpr int jn = (j + P - 1) % P;
        if constexpr (P > 2) {
            // take the Q read ahead for this tile before qn is refilled
            if (q_ready) {
#pragma unroll
                for (int kc = 0; kc < KC; ++kc) qf[kc] = qn[kc];
                q_ready = false;
            }
            if (i + 1 < n && cq[(j + 1) % P].t == 0) load_q(qn, cq[(j + 1) % P]);
        }
        cq[jn] = ic;
        issue(buf[jn], i + P - 1 < n, gb);
        if (i + P < n) {
            advance(ic);
            group_bases(ic, gb);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (i < n) {
            const Cur c = cq[j];
            Tile<TK>& now = buf[j];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int c2 = 0; c2 < LINES; ++c2) {
                    fix_lines(now.k[h][2 * c2], now.k[h][2 * c2 + 1], low8);
                    fix_lines(now.v[h][2 * c2], now.v[h][2 * c2 + 1], low8);
                }
            const int tbase = c.t * 32;
            if (tbase + 32 > c.L) {
                // rows past the sequence may hold anything (even NaN): zero
                // the V rows so that the selection products stay exact
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const bool dead = tbase + h * 16 + ln >= c.L;
#pragma unroll
                    for (int kc = 0; kc < TK; ++kc)
                        if (dead) now.v[h][kc] = u32x4{0, 0, 0, 0};
                }
            }
            if constexpr (F8)
                compute_tile_fp8(now, qf, esel, tbase, c.L, p.scale_log2, c.ks, c.vs, m_run, l_run,
                                 acc, lg);
            else
                compute_tile<DT, D>(now, qf, esel, tbase, c.L, p.scale_log2, m_run, l_run, acc, lg);
            if (i == n - 1 || c.t == c.nt - 1) flush(c, began_here, i);
            if (i + 1 < n && cq[(j + 1) % P].t == 0) {
                // a new (b, g) starts with tile i+1
                if constexpr (P > 2) q_ready = true;
                else load_q(qf, cq[(j + 1) % P]);  // waited for with tile i+1
                began_here = true;
            }
        }
    };
    for (int i = 0; i < n; i += P) {
        step(std::integral_constant<int, 0>{}, i);
        step(std::integral_constant<int, 1>{}, i + 1);
        if constexpr (P > 2) step(std::integral_constant<int, 2>{}, i + 2);
        if constexpr (P > 3) step(std::integral_constant<int, 3>{}, i + 3);
    }
}

// Log-sum-exp merge, one wave per (b, kv head g) that spans several slices
// of the streaming kernel: part k of the np parts from slice wa on sits at
// the (b, g) unit k for k < kSegPieces and in slot 0 of the wave for g of
// slice wa+k after that (wave rows (wa + k) * HW + g % HW).  The
// (max, denominator) pairs of parts 0..kSegPieces-1 (one part per lane) and
// the accumulators of the first QP parts are loaded together with the
// segment record, so a (b, g) of at most kSegPieces parts takes one memory
// step; parts past kSegPieces wait for the record.  The weights reach every
// lane through v_readlane.  NO = outputs per lane rounded up to a power of
// two; loads past np read stale units whose values are masked out.
template <int DT, int D, int NO>
__global__ __launch_bounds__(64) void attn_decode_merge(AttnParams p,
                                                        const int2* __restrict__ info) {
    constexpr int NJ = NO * 64 / D > 0 ? NO * 64 / D : 1;   // heads covered (power of two)
    constexpr int QP = NO >= 16 ? 2 : 32 / NO > 4 ? 4 : 32 / NO;   // parts per round
    static_assert(QP <= kSegPieces, "the first round's accumulators are segment-indexed");
    const int lane = threadIdx.x;
    const int G = p.group;
    const int b = blockIdx.x / p.kv_heads;
    const int g = blockIdx.x - b * p.kv_heads;
    const int n_out = G * D / 64;      // lane holds outputs lane + 64e, e < n_out
    const size_t seg0 = p.seg_unit0 + static_cast<size_t>(blockIdx.x) * kSegPieces;

    // first round, before the record: (max, denominator) of part min(lane, 3)
    // and the accumulators of parts 0 .. QP-1
    float m[NJ], l[NJ], v[QP][NO];
    {
        const size_t u0 = seg0 + min(lane, kSegPieces - 1);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const size_t u = (u0 * G + min(j, G - 1)) * 2;
            m[j] = p.part_ml[u];
            l[j] = p.part_ml[u + 1];
        }
#pragma unroll
        for (int q = 0; q < QP; ++q) {
            const float* pa = p.part_acc + (seg0 + q) * G * D + lane;
#pragma unroll
            for (int e = 0; e < NO; ++e) v[q][e] = pa[min(e, n_out - 1) * 64];
        }
    }
    const int2 si = info[blockIdx.x];
    const int wa = si.x, np = si.y;
    if (np <= 1) return;
    const int gofs = g % p.hw;
    auto unit = [&](int k) -> size_t {
        return k < kSegPieces ? seg0 + k : (static_cast<size_t>(wa + k) * p.hw + gofs) * 2;
    };
    auto load_parts = [&](float (&v)[QP][NO], int k0) {
#pragma unroll
        for (int q = 0; q < QP; ++q) {
            const float* pa = p.part_acc + unit(min(k0 + q, np - 1)) * G * D + lane;
#pragma unroll
            for (int e = 0; e < NO; ++e) v[q][e] = pa[min(e, n_out - 1) * 64];
        }
    };

    float mx[NJ], ls[NJ], acc[NO];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        mx[j] = -INFINITY;
        ls[j] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < NO; ++e) acc[e] = 0.0f;
    for (int k0 = 0; k0 < np; k0 += 64) {
        const bool live = k0 + lane < np;
        const int k = min(k0 + lane, np - 1);
        // lanes whose part is not among the ones loaded above
        if (k0 > 0 || (np > kSegPieces && lane >= kSegPieces)) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const size_t u = (unit(k) * G + min(j, G - 1)) * 2;
                m[j] = p.part_ml[u];
                l[j] = p.part_ml[u + 1];
            }
        }
        if (k0 > 0) load_parts(v, k0);   // in flight with the (max, denominator) loads
        float w[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            float cm = live ? m[j] : -INFINITY;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) cm = fmaxf(cm, __shfl_xor(cm, o));
            const float nm = fmaxf(mx[j], cm);
            const float corr = mx[j] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mx[j] - nm);
            w[j] = live ? __builtin_amdgcn_exp2f(m[j] - nm) : 0.0f;
            float wl = w[j] * l[j];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) wl += __shfl_xor(wl, o);
            ls[j] = ls[j] * corr + wl;
            mx[j] = nm;
#pragma unroll
            for (int e = 0; e < NO; ++e)
                if (e * 64 / D == j) acc[e] *= corr;
        }
        const int kn = min(64, np - k0);
        for (int kk0 = 0; kk0 < kn; kk0 += QP) {
            if (kk0 > 0) load_parts(v, k0 + kk0);
#pragma unroll
            for (int q = 0; q < QP; ++q) {
                const int kk = min(kk0 + q, kn - 1);
#pragma unroll
                for (int e = 0; e < NO; ++e) {
                    const float wt = __int_as_float(
                        __builtin_amdgcn_readlane(__float_as_int(w[e * 64 / D]), kk));
                    acc[e] += kk0 + q < kn ? wt * v[q][e] : 0.0f;
                }
            }
        }
    }
    uint16_t* out = reinterpret_cast<uint16_t*>(p.out) +
                    (static_cast<size_t>(b) * p.num_q_heads + g * G) * D + lane;
#pragma unroll
    for (int e = 0; e < NO; ++e)
        if (e < n_out) out[e * 64] = static_cast<uint16_t>(f32_to_elem<DT>(acc[e] / ls[e * 64 / D]));
}

template <int DT, int D>
void launch_merge(AttnParams& p, hipStream_t s) {
    const int n_out = p.group * D / 64;
    const dim3 grid(p.batch * p.kv_heads), block(64);
    if (n_out <= 1)
        hipLaunchKernelGGL((attn_decode_merge<DT, D, 1>), grid, block, 0, s, p, p.seg_info);
    else if (n_out <= 2)
        hipLaunchKernelGGL((attn_decode_merge<DT, D, 2>), grid, block, 0, s, p, p.seg_info);
    else if (n_out <= 4)
        hipLaunchKernelGGL((attn_decode_merge<DT, D, 4>), grid, block, 0, s, p, p.seg_info);
    else if (n_out <= 8)
        hipLaunchKernelGGL((attn_decode_merge<DT, D, 8>), grid, block, 0, s, p, p.seg_info);
    else if (n_out <= 16)
        hipLaunchKernelGGL((attn_decode_merge<DT, D, 16>), grid, block, 0, s, p, p.seg_info);
    else
        hipLaunchKernelGGL((attn_decode_merge<DT, D, 32>), grid, block, 0, s, p, p.seg_info);
}

// Any-shape decode attention (head_dim <= 256, any GQA map, any block size;
// f16, bf16, fp32 and fp8 pages): one workgroup per (sequence, query head),
// the same online-softmax recurrence as the reference kernel
// (ref kcmm_vllm_paged_attn.cu:10-102), with the positions spread over the
// workgroup instead of walked by one thread:
//  * lanes form teams of T (a power of two, 4..64) with 4 consecutive head
//    dims per lane; teams take positions round-robin, kGenUnroll at a time
//    (every K and V load of those positions issued before the first is
//    used), each team keeping its own running max, denominator and
//    accumulator;
//  * the page offsets (and fp8 scales) of kGenChunk positions are staged in
//    LDS before the chunk is walked, so a position costs one dependent load
//    (its K/V row), not three (table entry, offset, row);
//  * at the end the teams' states are rescaled to the common max and summed
//    through LDS.
constexpr int kGenThreads = 512;
constexpr int kGenChunk = 1024;
constexpr int kGenUnroll = 4;
constexpr int kGenMaxTeams = kGenThreads / 4;

// Four consecutive elements d0..d0+3 of a K/V row (zeros past head_dim);
// VEC: head_dim % 4 == 0, so the four are one aligned vector load.
template <int DT, bool VEC>
__device__ __forceinline__ void gen_load4(const uint8_t* row, int d0, int head_dim, float sc,
                                          float (&x)[4]) {
    if constexpr (VEC) {
        if (d0 >= head_dim) {
            x[0] = x[1] = x[2] = x[3] = 0.0f;
            return;
        }
        if constexpr (DT == kDtF32) {
            const float4 v = *reinterpret_cast<const float4*>(row + d0 * 4);
            x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
        } else if constexpr (DT == kDtFP8) {
            const uint32_t w = *reinterpret_cast<const uint32_t*>(row + d0);
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = fp8e4m3_to_f32((w >> (8 * i)) & 0xFFu) * sc;
        } else {
            const uint2 w = *reinterpret_cast<const uint2*>(row + d0 * 2);
            x[0] = elem_to_f32<DT>(w.x & 0xFFFFu);
            x[1] = elem_to_f32<DT>(w.x >> 16);
            x[2] = elem_to_f32<DT>(w.y & 0xFFFFu);
            x[3] = elem_to_f32<DT>(w.y >> 16);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = d0 + i;
            if (d >= head_dim) {
                x[i] = 0.0f;
            } else if constexpr (DT == kDtF32) {
                x[i] = reinterpret_cast<const float*>(row)[d];
            } else if constexpr (DT == kDtFP8) {
                x[i] = fp8e4m3_to_f32(row[d]) * sc;
            } else {
                x[i] = elem_to_f32<DT>(reinterpret_cast<const uint16_t*>(row)[d]);
            }
        }
    }
}

template <int DT, bool VEC>
__global__ __launch_bounds__(kGenThreads) void attn_decode_generic(AttnParams p, int head_dim,
                                                                   float scale, int tlog2) {
    constexpr bool F8 = DT == kDtFP8;
    __shared__ uint64_t s_page[kGenChunk + 1];
    __shared__ float s_ks[F8 ? kGenChunk + 1 : 1], s_vs[F8 ? kGenChunk + 1 : 1];
    __shared__ float s_m[kGenMaxTeams], s_s[kGenMaxTeams];
    __shared__ float s_acc[kGenThreads * 4];

    const int bh = blockIdx.x;
    const int b = bh / p.num_q_heads;
    const int h = bh - b * p.num_q_heads;
    const int kvh = h * p.kv_heads / p.num_q_heads;  // ref kcmm_vllm_paged_attn.cu:40
    const int tid = threadIdx.x;
    const int T = 1 << tlog2;
    const int nteams = blockDim.x >> tlog2;
    const int team = tid >> tlog2;
    const int d0 = (tid & (T - 1)) * 4;
    const int L = min(p.seq_lens[b], p.mbps * p.block_size);
    // q/out: f16 for f16 pools, fp32 for fp32 pools, bf16 otherwise
    const size_t io_off = (static_cast<size_t>(b) * p.num_q_heads + h) * head_dim * io_bytes<DT>();
    const uint8_t* qrow = p.q + io_off;
    uint8_t* orow = p.out + io_off;
    if (L <= 0) {
        for (int d = tid; d < head_dim; d += blockDim.x) io_store<DT>(orow, d, 0.0f);
        return;
    }
    float qv[4], acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        qv[i] = d0 + i < head_dim ? io_load<DT>(qrow, d0 + i) : 0.0f;
        acc[i] = 0.0f;
    }
    const uint64_t head_off = static_cast<uint64_t>(kvh) * head_dim * kv_elem_bytes<DT>();
    const int32_t* table = p.block_tables + static_cast<size_t>(b) * p.mbps;
    float m = -INFINITY, s = 0.0f;
    for (int c0 = 0; c0 < L; c0 += kGenChunk) {
        const int c1 = min(L, c0 + kGenChunk);
        const int lb0 = c0 / p.block_size;
        const int nb = (c1 - 1) / p.block_size - lb0 + 1;   // <= kGenChunk + 1
        __syncthreads();                                    // the last chunk's readers are done
        for (int i = tid; i < nb; i += blockDim.x) {
            const uint64_t page = p.offsets_f16[table[lb0 + i]] * 2ull;
            s_page[i] = page;
            if constexpr (F8) {
                s_ks[i] = *reinterpret_cast<const float*>(p.k_base + page + p.data_bytes + kvh * 4);
                s_vs[i] = *reinterpret_cast<const float*>(p.v_base + page + p.data_bytes + kvh * 4);
            }
        }
        __syncthreads();
        for (int pos = c0 + team; pos < c1; pos += nteams * kGenUnroll) {
            float kx[kGenUnroll][4], vx[kGenUnroll][4], dot[kGenUnroll];
#pragma unroll
            for (int u = 0; u < kGenUnroll; ++u) {
                const int pp = pos + u * nteams;
                if (pp < c1) {
                    const int lb = pp / p.block_size;
                    const int j = lb - lb0;
                    const uint64_t roff = s_page[j] +
                                          static_cast<uint64_t>(pp - lb * p.block_size) * p.row_bytes +
                                          head_off;
                    gen_load4<DT, VEC>(p.k_base + roff, d0, head_dim, F8 ? s_ks[j] : 1.0f, kx[u]);
                    gen_load4<DT, VEC>(p.v_base + roff, d0, head_dim, F8 ? s_vs[j] : 1.0f, vx[u]);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) kx[u][i] = vx[u][i] = 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < kGenUnroll; ++u)
                dot[u] = qv[0] * kx[u][0] + qv[1] * kx[u][1] + qv[2] * kx[u][2] + qv[3] * kx[u][3];
            for (int o = T >> 1; o > 0; o >>= 1) {
#pragma unroll
                for (int u = 0; u < kGenUnroll; ++u) dot[u] += __shfl_xor(dot[u], o);
            }
            float mx = m;
#pragma unroll
            for (int u = 0; u < kGenUnroll; ++u) {
                dot[u] = pos + u * nteams < c1 ? dot[u] * scale : -INFINITY;
                mx = fmaxf(mx, dot[u]);
            }
            const float corr = kexp<DT>(m - mx);            // m = -inf: 0
            s *= corr;
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] *= corr;
#pragma unroll
            for (int u = 0; u < kGenUnroll; ++u) {
                const float e = kexp<DT>(dot[u] - mx);      // -inf (past the chunk): 0
                s += e;
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] += e * vx[u][i];
            }
            m = mx;
        }
    }
    // combine the teams: rescale each to the common max, sum through LDS
    if ((tid & (T - 1)) == 0) {
        s_m[team] = m;
        s_s[team] = s;
    }
    __syncthreads();
    float M = -INFINITY;
    for (int t = 0; t < nteams; ++t) M = fmaxf(M, s_m[t]);
    const float f = m == -INFINITY ? 0.0f : kexp<DT>(m - M);
#pragma unroll
    for (int i = 0; i < 4; ++i) s_acc[team * T * 4 + d0 + i] = acc[i] * f;
    __syncthreads();
    float S = 0.0f;
    for (int t = 0; t < nteams; ++t)
        if (s_m[t] != -INFINITY) S += s_s[t] * kexp<DT>(s_m[t] - M);
    const float inv = 1.0f / S;
    for (int d = tid; d < head_dim; d += blockDim.x) {
        float o = 0.0f;
        for (int t = 0; t < nteams; ++t) o += s_acc[t * T * 4 + d];
        io_store<DT>(orow, d, o * inv);
    }
}

template <int DT>
void launch_generic(const AttnParams& p, int head_dim, float scale, hipStream_t s) {
    int tlog2 = 2;
    while ((4 << tlog2) < head_dim) ++tlog2;               // 4 * T >= head_dim, T <= 64
    // few (sequence, head) pairs: the whole 512-lane workgroup per pair;
    // enough pairs to fill the chip: 256 lanes each
    const long long pairs = static_cast<long long>(p.batch) * p.num_q_heads;
    if (pairs == 0) return;
    const int threads = pairs >= 1024 ? 256 : kGenThreads;
    const dim3 grid(static_cast<unsigned>(pairs));
    if (head_dim % 4 == 0)
        hipLaunchKernelGGL((attn_decode_generic<DT, true>), grid, dim3(threads), 0, s, p, head_dim,
                           scale, tlog2);
    else
        hipLaunchKernelGGL((attn_decode_generic<DT, false>), grid, dim3(threads), 0, s, p, head_dim,
                           scale, tlog2);
}

int env_int(dev::Tun t, int dflt, int lo, int hi) {
    int x = 0;
    if (!dev::tunable(t, &x)) return dflt;
    return x < lo || x > hi ? dflt : x;
}

// Tunables (read once per process, dev::tunable):
// KCMM_ATTN_WAVES waves of the streaming kernel (default by page type),
// KCMM_ATTN_HW waves per workgroup (kv heads read together; the largest
// divisor of Hkv not above it is used), KCMM_ATTN_MIN_TILES the smallest
// slice a workgroup takes, KCMM_ATTN_DEPTH tiles in flight (2 or 3; 3 keeps
// at most 4 waves per workgroup).
int stream_waves(int dtype) {
    return env_int(dev::Tun::kAttnWaves, dtype == kDtFP8 ? 2048 : 1024, 1, 1 << 20);
}
// Measured in the full decode step (Llama-3-8B shape, three runs each):
// 16-bit pages are as fast with one-wave workgroups as with head blocks (the
// layer step is 1% faster with HW = 1), fp8 pages gain 3% at HW = 8.
int stream_hw(int dtype) { return env_int(dev::Tun::kAttnHw, dtype == kDtFP8 ? 8 : 1, 1, 8); }
int stream_min_tiles() { return env_int(dev::Tun::kAttnMinTiles, 8, 1, 1 << 16); }
int stream_depth() { return env_int(dev::Tun::kAttnDepth, 2, 2, 3); }

template <int DT, int D, int BS>
bool launch_stream(AttnParams& p, hipStream_t s, bool no_alloc, std::string* err) {
    static_assert(D * (DT == kDtFP8 ? 1 : 2) % 128 == 0, "head rows are whole 128-byte lines");
    const long long cap = static_cast<long long>(p.mbps) * p.block_size;
    const long long tmax = static_cast<long long>(p.batch) * p.kv_heads * ((cap + 31) / 32);
    if (cap > INT_MAX || tmax > (1LL << 30)) {
        *err = "decode attention: batch x context too large";
        return false;
    }
    if (p.batch == 0) return true;
    const int depth = stream_depth();
    int hw = std::min(stream_hw(DT), depth == 3 ? 4 : 8);
    while (p.kv_heads % hw) --hw;
    p.hw = hw;
    p.min_tiles = stream_min_tiles();
    const long long lists = tmax / p.kv_heads * (p.kv_heads / hw);   // entries of the slice list
    const long long want = (lists + p.min_tiles - 1) / p.min_tiles;
    p.total_waves = static_cast<int>(
        std::max(1LL, std::min<long long>(std::max(1, stream_waves(DT) / hw), want)));
    // slice-indexed units, then kSegPieces per (b, g); G rows of each
    p.seg_unit0 = static_cast<size_t>(p.total_waves) * hw * 2;
    const size_t units =
        (p.seg_unit0 + static_cast<size_t>(p.batch) * p.kv_heads * kSegPieces) * p.group;
    // idle-load region first: it must cover one tile's lane addresses
    const size_t idle_bytes = (static_cast<size_t>(8) * p.row_bytes + 1023) & ~static_cast<size_t>(255);
    const size_t part_bytes = idle_bytes + ((units * (D + 2) * sizeof(float) + 255) & ~size_t(255));
    const size_t info_bytes = static_cast<size_t>(p.batch) * p.kv_heads * sizeof(int2);
    void* ws = nullptr;
    void* info = nullptr;
    std::unique_lock<std::mutex> noalloc_lock;
    NoAllocDevice* nd = nullptr;
    bool capturing = false;
    if (no_alloc) {
        // nothing here needs to start zeroed: every partial and segment
        // record is written before it is read
        if (part_bytes + info_bytes > kNoAllocScratchBytes) {
            *err = "decode attention (no-alloc): this batch needs " +
                   std::to_string(part_bytes + info_bytes) + " bytes of scratch, the static "
                   "scratch holds " + std::to_string(kNoAllocScratchBytes);
            return false;
        }
        noalloc_lock = std::unique_lock<std::mutex>(g_noalloc_mu);
        if (!noalloc_device(&nd, err)) return false;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        KCMM_HIP_CHECK(hipStreamIsCapturing(s, &cs), err);
        // under graph capture the caller orders the graph's nodes
        capturing = cs != hipStreamCaptureStatusNone;
        if (!capturing && nd->used && nd->last != s)
            KCMM_HIP_CHECK(hipStreamWaitEvent(s, nd->done, 0), err);
        ws = nd->scratch;
        info = nd->scratch + part_bytes;
    } else {
        if (!dev::stream_workspace(reinterpret_cast<uint64_t>(s), 0, part_bytes, &ws, false, err) ||
            !dev::stream_workspace(reinterpret_cast<uint64_t>(s), 2, info_bytes, &info, false, err))
            return false;
    }
    const uint8_t* idle = static_cast<const uint8_t*>(ws);
    p.part_ml = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + idle_bytes);
    p.part_acc = p.part_ml + units * 2;
    p.seg_info = static_cast<int2*>(info);
    const auto tp = timing_pair(s);
    if (tp.first != nullptr) KCMM_HIP_CHECK(hipEventRecord(tp.first, s), err);
    if (depth == 3)
        hipLaunchKernelGGL((attn_decode_stream<DT, D, BS, 3>), dim3(p.total_waves), dim3(64 * hw),
                           0, s, p, p.block_tables, p.seq_lens, p.offsets_f16, p.k_base, p.v_base,
                           idle);
    else
        hipLaunchKernelGGL((attn_decode_stream<DT, D, BS, 2>), dim3(p.total_waves), dim3(64 * hw),
                           0, s, p, p.block_tables, p.seq_lens, p.offsets_f16, p.k_base, p.v_base,
                           idle);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    if (tp.second != nullptr) KCMM_HIP_CHECK(hipEventRecord(tp.second, s), err);
    launch_merge<DT == kDtFP8 ? kDtBF16 : DT, D>(p, s);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    if (no_alloc && !capturing) {
        KCMM_HIP_CHECK(hipEventRecord(nd->done, s), err);
        nd->last = s;
        nd->used = true;
    }
    return true;
}

template <int DT, int D>
bool launch_stream_bs(AttnParams& p, hipStream_t s, bool no_alloc, std::string* err) {
    if (p.block_size == 16) return launch_stream<DT, D, 16>(p, s, no_alloc, err);
    return launch_stream<DT, D, 0>(p, s, no_alloc, err);
}

template <int DT>
bool launch_dt(AttnParams& p, int head_dim, hipStream_t s, bool no_alloc, std::string* err) {
    if (head_dim == 64) return launch_stream_bs<DT, 64>(p, s, no_alloc, err);
    return launch_stream_bs<DT, 128>(p, s, no_alloc, err);
}

}  // namespace

namespace dev {

bool attn_decode(const AttnDecodeArgs& a, std::string* err) {
    AttnParams p{};
    p.q = reinterpret_cast<const uint8_t*>(a.q);
    p.out = reinterpret_cast<uint8_t*>(a.out);
    p.k_base = reinterpret_cast<const uint8_t*>(a.k_base);
    p.v_base = reinterpret_cast<const uint8_t*>(a.v_base);
    p.block_tables = reinterpret_cast<const int32_t*>(a.block_tables);
    p.seq_lens = reinterpret_cast<const int32_t*>(a.seq_lens);
    p.offsets_f16 = reinterpret_cast<const uint64_t*>(a.offsets_f16);
    p.batch = static_cast<int>(a.batch);
    p.num_q_heads = static_cast<int>(a.num_q_heads);
    p.kv_heads = static_cast<int>(a.kv_heads);
    p.group = p.num_q_heads / p.kv_heads;
    p.block_size = static_cast<int>(a.block_size);
    p.mbps = static_cast<int>(a.mbps);
    p.row_bytes = static_cast<int>(a.row_bytes);
    p.data_bytes = static_cast<int>(a.data_bytes);
    p.scale_log2 = a.scale * 1.4426950408889634f;
    hipStream_t s = reinterpret_cast<hipStream_t>(a.stream);

    // Streaming MFMA path: whole GQA groups of at most 16 heads, pages made of
    // 8-token groups; 16-bit pages at head_dim 64 or 128, fp8 pages at 128.
    const bool grouped = p.num_q_heads % p.kv_heads == 0 && p.group <= 16;
    const bool stream_dim = a.head_dim == 64 || a.head_dim == 128;
    int generic_flag = 0;
    const bool force_generic = dev::tunable(dev::Tun::kAttnGeneric, &generic_flag);
    if (grouped && a.block_size % 8 == 0 && !force_generic) {
        if (a.dtype == kDtFP8 && a.head_dim == 128)
            return launch_stream_bs<kDtFP8, 128>(p, s, a.no_alloc, err);
        if (a.dtype == kDtF16 && stream_dim) return launch_dt<kDtF16>(p, a.head_dim, s, a.no_alloc, err);
        if (a.dtype == kDtBF16 && stream_dim)
            return launch_dt<kDtBF16>(p, a.head_dim, s, a.no_alloc, err);
    }
    const int hd = static_cast<int>(a.head_dim);
    switch (a.dtype) {
        case kDtF16: launch_generic<kDtF16>(p, hd, a.scale, s); break;
        case kDtBF16: launch_generic<kDtBF16>(p, hd, a.scale, s); break;
        case kDtF32: launch_generic<kDtF32>(p, hd, a.scale, s); break;
        default: launch_generic<kDtFP8>(p, hd, a.scale, s); break;
    }
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

bool attn_stream_timing_start(uint32_t max_calls, std::string* err) {
    if (max_calls == 0 || max_calls > (1u << 16)) {
        *err = "attention timing: max_calls must be 1..65536";
        return false;
    }
    std::lock_guard<std::mutex> lk(g_timing.mu);
    if (g_timing.on.load()) {
        *err = "attention timing already started";
        return false;
    }
    KCMM_HIP_CHECK(hipGetDevice(&g_timing.device), err);
    g_timing.ev.assign(2 * static_cast<size_t>(max_calls), nullptr);
    for (auto& e : g_timing.ev) {
        if (hipEventCreate(&e) != hipSuccess) {
            for (auto& f : g_timing.ev)
                if (f != nullptr) (void)hipEventDestroy(f);
            g_timing.ev.clear();
            *err = "attention timing: hipEventCreate failed";
            return false;
        }
    }
    g_timing.next = 0;
    g_timing.on.store(true, std::memory_order_release);
    return true;
}

bool attn_stream_timing_stop(double* avg_us, uint32_t* count, std::string* err) {
    std::lock_guard<std::mutex> lk(g_timing.mu);
    if (!g_timing.on.load()) {
        *err = "attention timing not started";
        return false;
    }
    g_timing.on.store(false);
    double total_ms = 0.0;
    bool ok = true;
    for (uint32_t i = 0; i < g_timing.next && ok; ++i) {
        float ms = 0.0f;
        ok = hipEventSynchronize(g_timing.ev[2 * i + 1]) == hipSuccess &&
             hipEventElapsedTime(&ms, g_timing.ev[2 * i], g_timing.ev[2 * i + 1]) == hipSuccess;
        total_ms += ms;
    }
    const uint32_t n = g_timing.next;
    for (auto& e : g_timing.ev) (void)hipEventDestroy(e);
    g_timing.ev.clear();
    g_timing.next = 0;
    if (!ok) {
        *err = "attention timing: event query failed";
        return false;
    }
    *count = n;
    *avg_us = n > 0 ? total_ms * 1e3 / n : 0.0;
    return true;
}

}  // namespace dev
}  // namespace kcmm
