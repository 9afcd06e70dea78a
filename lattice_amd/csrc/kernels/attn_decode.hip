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
//  * one workgroup of WAVES wavefronts per (b, kv head, chunk of CHUNK
//    tokens); every page slice a workgroup reads serves all G = Hq/Hkv query
//    heads of its kv head (GQA reuse: each K/V byte is read from HBM once);
//  * a wave walks 32-token tiles; each lane issues 16-byte loads straight
//    into MFMA operand layout -- no LDS for K;
//  * S^T = K Q^T on v_mfma_f32_16x16x32 (token rows x head columns), online
//    softmax in the log2 domain with cross-lane max by lane shuffles;
//  * O^T += V^T P^T on the same MFMA: V goes through wave-private LDS to be
//    read transposed; P^T is already in B-operand layout in registers;
//  * waves of a workgroup merge in LDS; the chunks of one (b, g) merge by
//    log-sum-exp in whichever workgroup finishes last (split-K over long
//    contexts in a single launch).
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

struct AttnParams {
    const uint8_t* q;       // [B][Hq][D] 16-bit elements
    uint8_t* out;           // [B][Hq][D]
    const uint8_t* k_base;
    const uint8_t* v_base;
    const int32_t* block_tables;
    const int32_t* seq_lens;
    const uint64_t* offsets_f16;
    float* part_acc;        // [B][Hkv][max_chunks][G][D]
    float* part_ml;         // [B][Hkv][max_chunks][G][2]
    int* counters;          // [B][Hkv] chunk arrivals (zero between launches)
    int batch, num_q_heads, kv_heads, group, block_size, mbps, max_chunks;
    int row_bytes, data_bytes;
    float scale_log2;       // scale * log2(e)
};

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

// Byte offset (inside a region) of token `pos` of sequence b, kv head kvh.
template <int BS>
__device__ __forceinline__ uint64_t token_offset(const AttnParams& p, int b, int kvh, int pos,
                                                 int head_bytes) {
    const int bs = BS > 0 ? BS : p.block_size;
    const int lb = pos / bs;
    const int off = pos - lb * bs;
    const int blk = p.block_tables[static_cast<size_t>(b) * p.mbps + lb];
    return p.offsets_f16[blk] * 2ull + static_cast<uint64_t>(off) * p.row_bytes +
           static_cast<uint64_t>(kvh) * head_bytes;
}

constexpr int kPad = 4;  // LDS row padding (elements): keeps transposed reads conflict-free

// One 32-token tile: 2 halves of 16 tokens, KC 16-byte fragments per lane each.
template <int KC>
struct Tile {
    u32x4 k[2][KC];
    u32x4 v[2][KC];
};

template <int KC>
__device__ __forceinline__ void load_tile(Tile<KC>& t, const uint8_t* k_base,
                                          const uint8_t* v_base, const uint64_t off[2],
                                          int lg) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint8_t* kr = k_base + off[h] + lg * 16;
        const uint8_t* vr = v_base + off[h] + lg * 16;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            t.k[h][kc] = *reinterpret_cast<const u32x4*>(kr + kc * 64);
            t.v[h][kc] = *reinterpret_cast<const u32x4*>(vr + kc * 64);
        }
    }
}

// Online-softmax update of one tile (see the file comment for the layouts).
template <int DT, int D>
__device__ __forceinline__ void compute_tile(const Tile<D / 32>& t, const u32x4* qf, int tbase,
                                             int L, float scale_log2, float& m_run,
                                             float& l_run, f32x4* acc, uint16_t* vl, int ln,
                                             int lg) {
    constexpr int KC = D / 32;
    constexpr int DB = D / 16;
    constexpr int ROW = D + kPad;
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

    // V rows into wave-private LDS (row = token in tile), then V^T reads.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            uint16_t* dst = vl + (h * 16 + ln) * ROW + kc * 32 + lg * 8;
            reinterpret_cast<u32x2*>(dst)[0] = u32x2{t.v[h][kc][0], t.v[h][kc][1]};
            reinterpret_cast<u32x2*>(dst)[1] = u32x2{t.v[h][kc][2], t.v[h][kc][3]};
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int db = 0; db < DB; ++db) {
        const uint16_t* col = vl + db * 16 + ln;
        u32x4 va;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t0 = (2 * i < 4) ? 4 * lg + 2 * i : 16 + 4 * lg + 2 * i - 4;
            const uint32_t lo = col[t0 * ROW];
            const uint32_t hi = col[(t0 + 1) * ROW];
            va[i] = lo | (hi << 16);
        }
        acc[db] = mfma16x16x32<DT>(va, pf, acc[db]);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Workgroup = WAVES wavefronts on one (sequence b, kv head, chunk of CHUNK
// tokens); wave w owns tiles [w*TPW, (w+1)*TPW) of the chunk.  Chunks of a
// sequence longer than CHUNK write fp32 partials (unnormalised output, max,
// denominator); the last workgroup of that (b, kv head) to finish -- found
// with a device-scope counter -- merges them by log-sum-exp and resets the
// counter, so one launch does split-K end to end.
template <int DT, int D, int BS, int WAVES, int TPW>
__global__ __launch_bounds__(WAVES * 64) void attn_decode_mfma(AttnParams p) {
    constexpr int KC = D / 32;
    constexpr int DB = D / 16;
    constexpr int CHUNK = WAVES * TPW * 32;
    constexpr int ROW = D + kPad;
    constexpr int HEAD_BYTES = D * 2;
    constexpr int LDS_ELEMS = WAVES * 32 * ROW;
    static_assert((WAVES * D * 16 + WAVES * 32) * 4 <= LDS_ELEMS * 2, "merge area exceeds LDS");

    __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_ELEMS];
    __shared__ int last_flag;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int ln = lane & 15;
    const int lg = lane >> 4;

    int bid = blockIdx.x;
    const int kvh = bid % p.kv_heads;
    bid /= p.kv_heads;
    const int b = bid % p.batch;
    const int chunk = bid / p.batch;
    const int G = p.group;
    const int bs = BS > 0 ? BS : p.block_size;
    const int L = min(p.seq_lens[b], p.mbps * bs);

    if (L <= 0) {
        if (chunk == 0) {
            uint16_t* o = reinterpret_cast<uint16_t*>(p.out) +
                          (static_cast<size_t>(b) * p.num_q_heads + kvh * G) * D;
            for (int i = threadIdx.x; i < G * D; i += WAVES * 64) o[i] = 0;
        }
        return;
    }
    const int n_chunks = (L + CHUNK - 1) / CHUNK;
    if (chunk >= n_chunks) return;

    const int tok0 = chunk * CHUNK + wave * TPW * 32;
    const int ntiles = max(0, min(TPW, (L - tok0 + 31) / 32));

    // Page addresses of every tile this wave will read, fetched up front so
    // the dependent table -> offset -> data loads are not paid per tile.
    uint64_t toff[TPW][2];
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int pos = min(tok0 + t * 32 + h * 16 + ln, L - 1);
            toff[t][h] = token_offset<BS>(p, b, kvh, pos, HEAD_BYTES);
        }

    // Q^T as the B operand: lane (head ln, group lg) holds Q[ln][kc*32+8lg .. +8].
    u32x4 qf[KC];
    {
        const bool valid = ln < G;
        const uint8_t* qrow =
            p.q + (static_cast<size_t>(b) * p.num_q_heads + kvh * G + (valid ? ln : 0)) * D * 2;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            u32x4 v = *reinterpret_cast<const u32x4*>(qrow + (kc * 32 + lg * 8) * 2);
            qf[kc] = valid ? v : u32x4{0, 0, 0, 0};
        }
    }

    float m_run = -INFINITY;  // running max (log2 domain) of column ln
    float l_run = 0.0f;       // this lane's share of the softmax denominator
    f32x4 acc[DB];
#pragma unroll
    for (int i = 0; i < DB; ++i) acc[i] = f32x4{0, 0, 0, 0};
    uint16_t* vl = lds + wave * 32 * ROW;

    // Two tiles in flight: the loads of tile t+1 are issued before tile t is
    // consumed.
    Tile<KC> ta, tb;
    if (ntiles > 0) load_tile<KC>(ta, p.k_base, p.v_base, toff[0], lg);
#pragma unroll
    for (int t = 0; t < TPW; t += 2) {
        if (t < ntiles) {
            if (t + 1 < ntiles) load_tile<KC>(tb, p.k_base, p.v_base, toff[t + 1], lg);
            compute_tile<DT, D>(ta, qf, tok0 + t * 32, L, p.scale_log2, m_run, l_run, acc, vl, ln,
                                lg);
        }
        if (t + 1 < ntiles) {
            if (t + 2 < ntiles && t + 2 < TPW)
                load_tile<KC>(ta, p.k_base, p.v_base, toff[(t + 2) % TPW], lg);
            compute_tile<DT, D>(tb, qf, tok0 + (t + 1) * 32, L, p.scale_log2, m_run, l_run, acc,
                                vl, ln, lg);
        }
    }

    l_run = wave_sum_across_groups(l_run);

    // ---- merge the waves of this workgroup in LDS ----
    __syncthreads();
    float* mrg = reinterpret_cast<float*>(lds);   // [WAVES][D][16] then [WAVES][16][2]
    float* mrg_ml = mrg + WAVES * D * 16;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) mrg[(wave * D + db * 16 + lg * 4 + r) * 16 + ln] = acc[db][r];
    if (lg == 0) {
        mrg_ml[(wave * 16 + ln) * 2 + 0] = m_run;
        mrg_ml[(wave * 16 + ln) * 2 + 1] = l_run;
    }
    __syncthreads();

    uint16_t* out_bh = reinterpret_cast<uint16_t*>(p.out) +
                       (static_cast<size_t>(b) * p.num_q_heads + kvh * G) * D;
    const size_t unit0 = (static_cast<size_t>(b) * p.kv_heads + kvh) * p.max_chunks;
    for (int i = threadIdx.x; i < G * D; i += WAVES * 64) {
        const int j = i / D;
        const int d = i - j * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, mrg_ml[(w * 16 + j) * 2]);
        float lsum = 0.0f, o = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float mw = mrg_ml[(w * 16 + j) * 2];
            const float wgt = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
            lsum += wgt * mrg_ml[(w * 16 + j) * 2 + 1];
            o += wgt * mrg[(w * D + d) * 16 + j];
        }
        if (n_chunks == 1) {
            out_bh[i] = static_cast<uint16_t>(f32_to_elem<DT>(o / lsum));
        } else {
            // Agent-scope stores write through to the device coherence point,
            // so the merging workgroup (possibly on another XCD) sees them
            // without a whole-L2 write-back.
            const size_t u = (unit0 + chunk) * G + j;
            __hip_atomic_store(&p.part_acc[u * D + d], o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == 0) {
                __hip_atomic_store(&p.part_ml[u * 2 + 0], M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&p.part_ml[u * 2 + 1], lsum, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (n_chunks == 1) return;

    // ---- split-K: the last chunk of (b, kv head) to arrive merges ----
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // partial stores acknowledged
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = __hip_atomic_fetch_add(&p.counters[b * p.kv_heads + kvh], 1,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = (prev == n_chunks - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    for (int i = threadIdx.x; i < G * D; i += WAVES * 64) {
        const int j = i / D;
        const int d = i - j * D;
        float M = -INFINITY;
        for (int c = 0; c < n_chunks; ++c)
            M = fmaxf(M, __hip_atomic_load(&p.part_ml[((unit0 + c) * G + j) * 2], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT));
        float lsum = 0.0f, o = 0.0f;
        for (int c = 0; c < n_chunks; ++c) {
            const size_t u = (unit0 + c) * G + j;
            const float mc = __hip_atomic_load(&p.part_ml[u * 2], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
            const float wgt = __builtin_amdgcn_exp2f(mc - M);
            lsum += wgt * __hip_atomic_load(&p.part_ml[u * 2 + 1], __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
            o += wgt * __hip_atomic_load(&p.part_acc[u * D + d], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        }
        out_bh[i] = static_cast<uint16_t>(f32_to_elem<DT>(o / lsum));
    }
    if (threadIdx.x == 0)   // ready for the next launch
        __hip_atomic_store(&p.counters[b * p.kv_heads + kvh], 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Any-shape fallback (head_dim <= 256, any GQA map, any block size, fp8
// pages): one wavefront per (b, query head), lanes split the head dimension,
// the same online-softmax recurrence as the reference kernel.
template <int DT>
__global__ __launch_bounds__(64) void attn_decode_generic(AttnParams p, int head_dim,
                                                          float scale) {
    const int bh = blockIdx.x;
    const int b = bh / p.num_q_heads;
    const int h = bh - b * p.num_q_heads;
    const int kvh = h * p.kv_heads / p.num_q_heads;  // ref kcmm_vllm_paged_attn.cu:40
    const int lane = threadIdx.x;
    const int L = min(p.seq_lens[b], p.mbps * p.block_size);
    // q/out are 16-bit (f16 for f16 pools, bf16 otherwise).
    constexpr int QDT = DT == kDtFP8 ? kDtBF16 : DT;
    const uint16_t* qrow =
        reinterpret_cast<const uint16_t*>(p.q) + (static_cast<size_t>(b) * p.num_q_heads + h) * head_dim;
    uint16_t* orow = reinterpret_cast<uint16_t*>(p.out) +
                     (static_cast<size_t>(b) * p.num_q_heads + h) * head_dim;
    if (L <= 0) {
        for (int d = lane; d < head_dim; d += 64) orow[d] = 0;
        return;
    }
    float qv[4], acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        qv[i] = d < head_dim ? elem_to_f32<QDT>(qrow[d]) : 0.0f;
        acc[i] = 0.0f;
    }
    const int esize = DT == kDtFP8 ? 1 : 2;
    float m = -INFINITY, s = 0.0f;
    for (int pos = 0; pos < L; ++pos) {
        const int lb = pos / p.block_size;
        const int off = pos - lb * p.block_size;
        const int blk = p.block_tables[static_cast<size_t>(b) * p.mbps + lb];
        const uint64_t page = p.offsets_f16[blk] * 2ull;
        const uint64_t roff = page + static_cast<uint64_t>(off) * p.row_bytes +
                              static_cast<uint64_t>(kvh) * head_dim * esize;
        float ks = 1.0f, vs = 1.0f;
        if constexpr (DT == kDtFP8) {
            ks = *reinterpret_cast<const float*>(p.k_base + page + p.data_bytes + kvh * 4);
            vs = *reinterpret_cast<const float*>(p.v_base + page + p.data_bytes + kvh * 4);
        }
        float dot = 0.0f;
        float vv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + 64 * i;
            float kx = 0.0f, vx = 0.0f;
            if (d < head_dim) {
                if constexpr (DT == kDtFP8) {
                    kx = fp8e4m3_to_f32(p.k_base[roff + d]) * ks;
                    vx = fp8e4m3_to_f32(p.v_base[roff + d]) * vs;
                } else {
                    kx = elem_to_f32<DT>(reinterpret_cast<const uint16_t*>(p.k_base + roff)[d]);
                    vx = elem_to_f32<DT>(reinterpret_cast<const uint16_t*>(p.v_base + roff)[d]);
                }
            }
            dot += qv[i] * kx;
            vv[i] = vx;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
        dot *= scale;
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
        if (d < head_dim) orow[d] = static_cast<uint16_t>(f32_to_elem<QDT>(acc[i] * inv));
    }
}

constexpr int kWaves = 4;

// Tiles (of 32 tokens) per wave; the chunk of one workgroup is
// kWaves * tpw * 32 tokens.  KCMM_ATTN_TPW overrides the default.
int tiles_per_wave() {
    static int v = [] {
        const char* e = std::getenv("KCMM_ATTN_TPW");
        int x = e ? std::atoi(e) : 4;
        return (x == 1 || x == 2 || x == 4 || x == 8) ? x : 4;
    }();
    return v;
}

template <int DT, int D, int BS, int TPW>
bool launch_mfma_tpw(AttnParams& p, hipStream_t s, std::string* err) {
    constexpr int CHUNK = kWaves * TPW * 32;
    const int bs = BS > 0 ? BS : p.block_size;
    const long long max_tok = static_cast<long long>(p.mbps) * bs;
    p.max_chunks = static_cast<int>((max_tok + CHUNK - 1) / CHUNK);
    const long long grid = static_cast<long long>(p.kv_heads) * p.batch * p.max_chunks;
    if (grid > 0x7fffffffLL) {
        *err = "decode attention grid too large";
        return false;
    }
    const size_t units = static_cast<size_t>(p.batch) * p.kv_heads * p.max_chunks * p.group;
    if (p.max_chunks > 1) {
        void* ws = nullptr;
        void* cnt = nullptr;
        if (!dev::stream_workspace(reinterpret_cast<uint64_t>(s), 0,
                                   units * (D + 2) * sizeof(float), &ws, false, err) ||
            !dev::stream_workspace(reinterpret_cast<uint64_t>(s), 2,
                                   static_cast<size_t>(p.batch) * p.kv_heads * sizeof(int), &cnt,
                                   true, err))
            return false;
        p.part_ml = static_cast<float*>(ws);
        p.part_acc = p.part_ml + units * 2;
        p.counters = static_cast<int*>(cnt);
    }
    hipLaunchKernelGGL((attn_decode_mfma<DT, D, BS, kWaves, TPW>), dim3(static_cast<unsigned>(grid)),
                       dim3(kWaves * 64), 0, s, p);
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

template <int DT, int D, int BS>
bool launch_mfma(AttnParams& p, hipStream_t s, std::string* err) {
    switch (tiles_per_wave()) {
        case 1: return launch_mfma_tpw<DT, D, BS, 1>(p, s, err);
        case 8: return launch_mfma_tpw<DT, D, BS, 8>(p, s, err);
        case 2: return launch_mfma_tpw<DT, D, BS, 2>(p, s, err);
        default: return launch_mfma_tpw<DT, D, BS, 4>(p, s, err);
    }
}

template <int DT, int D>
bool launch_mfma_bs(AttnParams& p, hipStream_t s, std::string* err) {
    if (p.block_size == 16) return launch_mfma<DT, D, 16>(p, s, err);
    return launch_mfma<DT, D, 0>(p, s, err);
}

template <int DT>
bool launch_dt(AttnParams& p, int head_dim, hipStream_t s, std::string* err) {
    switch (head_dim) {
        case 64: return launch_mfma_bs<DT, 64>(p, s, err);
        case 128: return launch_mfma_bs<DT, 128>(p, s, err);
        case 256: return launch_mfma_bs<DT, 256>(p, s, err);
        default: break;
    }
    *err = "unsupported head_dim for the MFMA path";
    return false;
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

    const bool grouped = p.num_q_heads % p.kv_heads == 0 && p.group <= 16;
    const bool mfma_dim = a.head_dim == 64 || a.head_dim == 128 || a.head_dim == 256;
    const bool force_generic = std::getenv("KCMM_ATTN_GENERIC") != nullptr;
    if (a.dtype != kDtFP8 && grouped && mfma_dim && !force_generic) {
        if (a.dtype == kDtF16) return launch_dt<kDtF16>(p, a.head_dim, s, err);
        return launch_dt<kDtBF16>(p, a.head_dim, s, err);
    }
    const dim3 grid(a.batch * a.num_q_heads);
    switch (a.dtype) {
        case kDtF16:
            hipLaunchKernelGGL(attn_decode_generic<kDtF16>, grid, dim3(64), 0, s, p,
                               static_cast<int>(a.head_dim), a.scale);
            break;
        case kDtBF16:
            hipLaunchKernelGGL(attn_decode_generic<kDtBF16>, grid, dim3(64), 0, s, p,
                               static_cast<int>(a.head_dim), a.scale);
            break;
        default:
            hipLaunchKernelGGL(attn_decode_generic<kDtFP8>, grid, dim3(64), 0, s, p,
                               static_cast<int>(a.head_dim), a.scale);
            break;
    }
    KCMM_HIP_CHECK(hipGetLastError(), err);
    return true;
}

}  // namespace dev
}  // namespace kcmm
