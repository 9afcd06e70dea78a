// Causal chunked-prefill attention over paged K/V for gfx950 (MI355X).
//
// Contract (the reference prefills one token per decode step, ref
// src/model/transformer.rs:50-65; this follows the varlen-with-paged-KV form
// vLLM uses for chunked prefill): sequence b holds seq_lens[b] tokens in the
// cache; its last len_b = qsl[b+1] - qsl[b] are this chunk's queries, whose
// K/V are already appended.  Query i of b is at position
// p = seq_lens[b] - len_b + i and attends to keys 0..p.  q/out rows are
// [qsl[b] + i][Hq][D]; GQA head map g = h / (Hq/Hkv).  Accumulation is fp32.
//
// MI355X design (the decode kernel's tile machinery, with query columns):
//  * workgroup = 4 waves on one (sequence b, kv head g, block of query
//    tokens); wave w takes 2 blocks of 16 MFMA columns, a column being one
//    (query token, head of the GQA group) pair, heads fastest;
//  * each wave walks 32-key tiles up to its last query's position, the next
//    tile in flight while one is consumed; a tile's keys come in whole
//    128-byte lines (8 keys per load) put into MFMA layout by one DPP row
//    rotation + select per dword (the four waves read the same keys, so the
//    loads are cached ones);
//  * S^T = K Q^T on v_mfma_f32_16x16x32, causal mask per column, online
//    softmax in the log2 domain per column; O^T += V^T P^T with V^T made by
//    0/1 selection MFMAs once per tile and shared by both column blocks.
#include <algorithm>
#include <climits>
#include <cmath>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

struct PrefillParams {
    const uint8_t* q;
    uint8_t* out;
    int batch, num_q_heads, kv_heads, group, block_size, mbps;
    int row_bytes, data_bytes, head_dim;
    float scale_log2;
    float scale;
};

template <int DT>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (DT == kDtF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                       0);
}

__device__ __forceinline__ uint32_t ror8(uint32_t x) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_mov_dpp(static_cast<int>(x), 0x128, 0xF, 0xF, false));
}

// x: lane (r, lg) <- key (r & 7), bytes (4*(r >> 3) + lg)*16 of a 128-byte
// line; y: keys 8..15.  Afterwards lane r = key r, x bytes 16lg..+15 and y
// bytes 64+16lg..+15 of the line (MFMA A layout).
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

// E[k][j] = (k == 16*sub + j): selects 16 consecutive k indices (transposes).
template <int DT>
__device__ __forceinline__ u32x4 select_operand(int sub, int ln, int lg) {
    constexpr uint32_t one = DT == kDtF16 ? 0x3C00u : 0x3F80u;
    u32x4 e = u32x4{0, 0, 0, 0};
    const int k = 16 * sub + ln;
    if ((k >> 3) == lg) {
        const int t = k & 7;
        e[t >> 1] = (t & 1) ? (one << 16) : one;
    }
    return e;
}

template <int DT>
__device__ __forceinline__ uint32_t pack_exact(float lo, float hi) {
    if constexpr (DT == kDtF16) return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
    else return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

__device__ __forceinline__ float col_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    return fmaxf(x, __shfl_xor(x, 32));
}

template <int KC>
struct KvTile {
    u32x4 k[2][KC];
    u32x4 v[2][KC];
};

// Workgroups over (query-token block, kv head), kv head fastest: blockIdx.x
// = block * Hkv + g.  Workgroups are dealt to the 8 XCDs round-robin, so with
// 8 kv heads every XCD serves one head and its L2 holds that head's pages
// (shared prefixes included) for all sequences.
template <int DT, int D, int G>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1)))
void attn_prefill_mfma(PrefillParams p, const uint8_t* __restrict__ kreg,
                       const uint8_t* __restrict__ vreg, const int32_t* __restrict__ bt,
                       const int32_t* __restrict__ sl, const int32_t* __restrict__ qsl,
                       const uint64_t* __restrict__ offs) {
    constexpr int KC = D / 32;
    constexpr int LINES = D / 64;
    constexpr int DB = D / 16;
    constexpr int TPB = 16 / G;          // query tokens per 16-column block
    constexpr int TW = 2 * TPB;          // per wave
    constexpr int TWG = 4 * TW;          // per workgroup
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ln = lane & 15, lg = lane >> 4;
    const bool low8 = ln < 8;
    const int g = static_cast<int>(blockIdx.x) % p.kv_heads;
    const int item = static_cast<int>(blockIdx.x) / p.kv_heads;
    const int bs = p.block_size;

    // ---- sequence and token block of this workgroup ----
    int b = -1, blk = 0;
    {
        int base = 0;
        for (int c = 0; c < p.batch; c += 64) {
            const int bb = c + lane;
            const int n = bb < p.batch ? qsl[bb + 1] - qsl[bb] : 0;
            const int v = n > 0 ? (n + TWG - 1) / TWG : 0;
            int incl = v;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o);
                if (lane >= o) incl += y;
            }
            const unsigned long long hit = __ballot(base + incl > item);
            if (hit) {
                const int j = __ffsll(static_cast<long long>(hit)) - 1;
                b = c + j;
                blk = item - (base + __shfl(incl - v, j));
                break;
            }
            base += __shfl(incl, 63);
        }
    }
    b = __builtin_amdgcn_readfirstlane(b);
    if (b < 0) return;
    blk = __builtin_amdgcn_readfirstlane(blk);
    const int q0 = qsl[b];
    const int len = qsl[b + 1] - q0;
    const int L = min(sl[b], p.mbps * bs);
    const int first_pos = L - len;           // position of the chunk's first query
    const int tok0 = blk * TWG + wave * TW;  // this wave's first query (chunk index)
    if (tok0 >= len) return;
    // queries before position 0 (more queries than cached tokens) see no key;
    // their rows are written as zeros
    const int tok_last = min(tok0 + TW, len) - 1;
    const int nkeys = max(0, first_pos + tok_last + 1);
    const int ntiles = (nkeys + 31) / 32;

    // ---- columns: query token (clamped into the chunk; extra columns are
    // computed on a duplicate and never stored) and its position ----
    int qpos[2];
    u32x4 qf[2][KC];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int t = min(tok0 + qb * TPB + ln / G, len - 1);
        qpos[qb] = first_pos + t;
        const uint8_t* qrow =
            p.q + ((static_cast<size_t>(q0) + t) * p.num_q_heads + g * G + ln % G) * D * 2;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
            qf[qb][kc] = *reinterpret_cast<const u32x4*>(qrow + (kc * 32 + lg * 8) * 2);
    }

    const int32_t* row = bt + static_cast<size_t>(b) * p.mbps;
    const uint32_t lo = static_cast<uint32_t>((ln & 7) * p.row_bytes + ((ln >> 3) * 4 + lg) * 16);
    const int last8 = (L - 1) & ~7;
    auto load_tile = [&](KvTile<KC>& tl, int kt) {
        uint64_t gb[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int tok = min(kt * 32 + q * 8, last8);
            const int lb = tok / bs;
            gb[q] = offs[row[lb]] * 2ull +
                    static_cast<uint32_t>((tok - lb * bs) * p.row_bytes + g * D * 2);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int c2 = 0; c2 < LINES; ++c2) {
                const uint32_t o = lo + c2 * 128;
                tl.k[h][2 * c2] = *reinterpret_cast<const u32x4*>(kreg + gb[2 * h] + o);
                tl.k[h][2 * c2 + 1] = *reinterpret_cast<const u32x4*>(kreg + gb[2 * h + 1] + o);
                tl.v[h][2 * c2] = *reinterpret_cast<const u32x4*>(vreg + gb[2 * h] + o);
                tl.v[h][2 * c2 + 1] = *reinterpret_cast<const u32x4*>(vreg + gb[2 * h + 1] + o);
            }
    };

    const u32x4 esel[2] = {select_operand<DT>(0, ln, lg), select_operand<DT>(1, ln, lg)};
    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.0f, 0.0f};
    f32x4 acc[2][DB];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int i = 0; i < DB; ++i) acc[qb][i] = f32x4{0, 0, 0, 0};

    auto consume = [&](KvTile<KC>& t, int kt) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int c2 = 0; c2 < LINES; ++c2) {
                fix_lines(t.k[h][2 * c2], t.k[h][2 * c2 + 1], low8);
                fix_lines(t.v[h][2 * c2], t.v[h][2 * c2 + 1], low8);
            }
        const int kbase = kt * 32;
        if (kbase + 32 > L) {
            // key rows past the sequence may hold anything: zero V for exact selection
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const bool dead = kbase + h * 16 + ln >= L;
#pragma unroll
                for (int kc = 0; kc < KC; ++kc)
                    if (dead) t.v[h][kc] = u32x4{0, 0, 0, 0};
            }
        }
        u32x4 pf[2];
        float corr[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            f32x4 s[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                s[h] = f32x4{0, 0, 0, 0};
#pragma unroll
                for (int kc = 0; kc < KC; ++kc) s[h] = mfma16<DT>(t.k[h][kc], qf[qb][kc], s[h]);
            }
            float sv[8];
            float mt = -INFINITY;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = kbase + h * 16 + lg * 4 + r;
                    const float x = key <= qpos[qb] ? s[h][r] * p.scale_log2 : -INFINITY;
                    sv[h * 4 + r] = x;
                    mt = fmaxf(mt, x);
                }
            mt = col_max(mt);
            const float m_new = fmaxf(m_run[qb], mt);
            // a column with no key yet (m_new = -inf) keeps weight 0
            corr[qb] = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run[qb] - m_new);
            float psum = 0.0f;
            float pv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                pv[i] = m_new == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sv[i] - m_new);
                psum += pv[i];
            }
            l_run[qb] = l_run[qb] * corr[qb] + psum;
            m_run[qb] = m_new;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                pf[qb][i] = f32_to_elem<DT>(pv[2 * i]) | (f32_to_elem<DT>(pv[2 * i + 1]) << 16);
        }
#pragma unroll
        for (int db = 0; db < DB; ++db) {
            const f32x4 v0 = mfma16<DT>(t.v[0][db >> 1], esel[db & 1], f32x4{0, 0, 0, 0});
            const f32x4 v1 = mfma16<DT>(t.v[1][db >> 1], esel[db & 1], f32x4{0, 0, 0, 0});
            u32x4 va;
            va[0] = pack_exact<DT>(v0[0], v0[1]);
            va[1] = pack_exact<DT>(v0[2], v0[3]);
            va[2] = pack_exact<DT>(v1[0], v1[1]);
            va[3] = pack_exact<DT>(v1[2], v1[3]);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) acc[qb][db] = mfma16<DT>(va, pf[qb], acc[qb][db] * corr[qb]);
        }
    };

    if (ntiles > 0) {   // (no tile at all: the sequence has no visible key)
        KvTile<KC> ta, tb;
        load_tile(ta, 0);
        int kt = 0;
        for (; kt + 1 < ntiles; kt += 2) {
            load_tile(tb, kt + 1);
            __builtin_amdgcn_sched_barrier(0);
            consume(ta, kt);
            if (kt + 2 < ntiles) load_tile(ta, kt + 2);
            __builtin_amdgcn_sched_barrier(0);
            consume(tb, kt + 1);
        }
        if (kt < ntiles) consume(ta, kt);
    }

    // ---- store the columns that are real queries ----
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const float l = l_run[qb] + __shfl_xor(l_run[qb], 16);
        const float lt = l + __shfl_xor(l, 32);
        const int t = tok0 + qb * TPB + ln / G;
        if (t < len) {
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            uint16_t* o = reinterpret_cast<uint16_t*>(p.out) +
                          ((static_cast<size_t>(q0) + t) * p.num_q_heads + g * G + ln % G) * D + 4 * lg;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                u32x2 w;
                w[0] = f32_to_elem<DT>(acc[qb][db][0] * inv) | (f32_to_elem<DT>(acc[qb][db][1] * inv) << 16);
                w[1] = f32_to_elem<DT>(acc[qb][db][2] * inv) | (f32_to_elem<DT>(acc[qb][db][3] * inv) << 16);
                *reinterpret_cast<u32x2*>(o + 16 * db) = w;
            }
        }
    }
}

// Any-shape fallback (head_dim <= 256, any GQA map, any block size, fp8
// pages with bf16 q/out): one wave per (query row, q head), lanes split the
// head dimension, online softmax over keys 0..p.
template <int DT>
__global__ __launch_bounds__(64) void attn_prefill_generic(PrefillParams p,
                                                           const uint8_t* __restrict__ kreg,
                                                           const uint8_t* __restrict__ vreg,
                                                           const int32_t* __restrict__ bt,
                                                           const int32_t* __restrict__ sl,
                                                           const int32_t* __restrict__ qsl,
                                                           const uint64_t* __restrict__ offs) {
    constexpr int QDT = DT == kDtFP8 ? kDtBF16 : DT;
    const int lane = threadIdx.x;
    const int rowi = blockIdx.x / p.num_q_heads;
    const int h = blockIdx.x - rowi * p.num_q_heads;
    const int D = p.head_dim;
    int b = 0;
    while (b + 1 < p.batch && qsl[b + 1] <= rowi) ++b;
    const int len = qsl[b + 1] - qsl[b];
    const int L = min(sl[b], p.mbps * p.block_size);
    const int pos = L - len + (rowi - qsl[b]);
    const int kvh = h * p.kv_heads / p.num_q_heads;
    uint16_t* orow = reinterpret_cast<uint16_t*>(p.out) + (static_cast<size_t>(rowi) * p.num_q_heads + h) * D;
    if (pos < 0) {
        for (int d = lane; d < D; d += 64) orow[d] = 0;
        return;
    }
    const uint16_t* qrow = reinterpret_cast<const uint16_t*>(p.q) + (static_cast<size_t>(rowi) * p.num_q_heads + h) * D;
    float qv[4], acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        qv[i] = d < D ? elem_to_f32<QDT>(qrow[d]) : 0.0f;
        acc[i] = 0.0f;
    }
    const int esize = DT == kDtFP8 ? 1 : 2;
    float m = -INFINITY, s = 0.0f;
    for (int key = 0; key <= pos; ++key) {
        const int lb = key / p.block_size;
        const int off = key - lb * p.block_size;
        const uint64_t page = offs[bt[static_cast<size_t>(b) * p.mbps + lb]] * 2ull;
        const uint64_t roff = page + static_cast<uint64_t>(off) * p.row_bytes +
                              static_cast<uint64_t>(kvh) * D * esize;
        float ks = 1.0f, vs = 1.0f;
        if constexpr (DT == kDtFP8) {
            ks = *reinterpret_cast<const float*>(kreg + page + p.data_bytes + kvh * 4);
            vs = *reinterpret_cast<const float*>(vreg + page + p.data_bytes + kvh * 4);
        }
        float dot = 0.0f, vv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + 64 * i;
            float kx = 0.0f, vx = 0.0f;
            if (d < D) {
                if constexpr (DT == kDtFP8) {
                    kx = fp8e4m3_to_f32(kreg[roff + d]) * ks;
                    vx = fp8e4m3_to_f32(vreg[roff + d]) * vs;
                } else {
                    kx = elem_to_f32<DT>(reinterpret_cast<const uint16_t*>(kreg + roff)[d]);
                    vx = elem_to_f32<DT>(reinterpret_cast<const uint16_t*>(vreg + roff)[d]);
                }
            }
            dot += qv[i] * kx;
            vv[i] = vx;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
        dot *= p.scale;
        const float m_new = fmaxf(m, dot);
        const float e = __expf(dot - m_new);
        const float corr = __expf(m - m_new);
        s = s * corr + e;
        m = m_new;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = acc[i] * corr + e * vv[i];
    }
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        if (d < D) orow[d] = static_cast<uint16_t>(f32_to_elem<QDT>(acc[i] * inv));
    }
}

template <int DT, int D, int G>
bool launch_mfma(const dev::AttnPrefillArgs& a, PrefillParams& p, hipStream_t s, std::string* err) {
    constexpr int TWG = 4 * 2 * (16 / G);
    const long long blocks =
        (static_cast<long long>(a.total_query_tokens) / TWG + a.batch + 1) * p.kv_heads;
    if (blocks > INT_MAX) {
        *err = "prefill: too many query tokens";
        return false;
    }
    hipLaunchKernelGGL((attn_prefill_mfma<DT, D, G>), dim3(static_cast<unsigned>(blocks)),
                       dim3(256), 0, s, p, reinterpret_cast<const uint8_t*>(a.k_base),
                       reinterpret_cast<const uint8_t*>(a.v_base),
                       reinterpret_cast<const int32_t*>(a.block_tables),
                       reinterpret_cast<const int32_t*>(a.seq_lens),
                       reinterpret_cast<const int32_t*>(a.query_start_loc),
                       reinterpret_cast<const uint64_t*>(a.offsets_f16));
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

template <int DT, int D>
bool launch_group(const dev::AttnPrefillArgs& a, PrefillParams& p, hipStream_t s, std::string* err) {
    switch (p.group) {
        case 1: return launch_mfma<DT, D, 1>(a, p, s, err);
        case 2: return launch_mfma<DT, D, 2>(a, p, s, err);
        case 4: return launch_mfma<DT, D, 4>(a, p, s, err);
        case 8: return launch_mfma<DT, D, 8>(a, p, s, err);
        default: return launch_mfma<DT, D, 16>(a, p, s, err);
    }
}

}  // namespace

namespace dev {

bool attn_prefill(const AttnPrefillArgs& a, std::string* err) {
    PrefillParams p{};
    p.q = reinterpret_cast<const uint8_t*>(a.q);
    p.out = reinterpret_cast<uint8_t*>(a.out);
    p.batch = static_cast<int>(a.batch);
    p.num_q_heads = static_cast<int>(a.num_q_heads);
    p.kv_heads = static_cast<int>(a.kv_heads);
    p.group = p.num_q_heads / p.kv_heads;
    p.block_size = static_cast<int>(a.block_size);
    p.mbps = static_cast<int>(a.mbps);
    p.row_bytes = static_cast<int>(a.row_bytes);
    p.data_bytes = static_cast<int>(a.data_bytes);
    p.head_dim = static_cast<int>(a.head_dim);
    p.scale = a.scale;
    p.scale_log2 = a.scale * 1.4426950408889634f;
    hipStream_t s = reinterpret_cast<hipStream_t>(a.stream);
    if (a.total_query_tokens == 0 || a.batch == 0) return true;

    const int G = p.group;
    const bool mfma_group = p.num_q_heads % p.kv_heads == 0 && (G == 1 || G == 2 || G == 4 ||
                                                                G == 8 || G == 16);
    const bool mfma_dim = a.head_dim == 64 || a.head_dim == 128;
    if (a.dtype != kDtFP8 && mfma_group && mfma_dim && a.block_size % 8 == 0 &&
        std::getenv("KCMM_ATTN_GENERIC") == nullptr) {
        if (a.dtype == kDtF16)
            return a.head_dim == 64 ? launch_group<kDtF16, 64>(a, p, s, err)
                                    : launch_group<kDtF16, 128>(a, p, s, err);
        return a.head_dim == 64 ? launch_group<kDtBF16, 64>(a, p, s, err)
                                : launch_group<kDtBF16, 128>(a, p, s, err);
    }
    const dim3 grid(a.total_query_tokens * a.num_q_heads);
    const auto* kb = reinterpret_cast<const uint8_t*>(a.k_base);
    const auto* vb = reinterpret_cast<const uint8_t*>(a.v_base);
    const auto* btp = reinterpret_cast<const int32_t*>(a.block_tables);
    const auto* slp = reinterpret_cast<const int32_t*>(a.seq_lens);
    const auto* qp = reinterpret_cast<const int32_t*>(a.query_start_loc);
    const auto* op = reinterpret_cast<const uint64_t*>(a.offsets_f16);
    switch (a.dtype) {
        case kDtF16:
            hipLaunchKernelGGL(attn_prefill_generic<kDtF16>, grid, dim3(64), 0, s, p, kb, vb, btp,
                               slp, qp, op);
            break;
        case kDtBF16:
            hipLaunchKernelGGL(attn_prefill_generic<kDtBF16>, grid, dim3(64), 0, s, p, kb, vb, btp,
                               slp, qp, op);
            break;
        default:
            hipLaunchKernelGGL(attn_prefill_generic<kDtFP8>, grid, dim3(64), 0, s, p, kb, vb, btp,
                               slp, qp, op);
            break;
    }
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

}  // namespace dev
}  // namespace kcmm
