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
// MI355X design (flash attention over LDS-staged pages; f16 / bf16 pages,
// and fp8-e4m3 pages at head_dim 128, dequantized to bf16 as their rows are
// stored to LDS):
//  * workgroup = 8 waves (2 per SIMD) on one (sequence b, kv head g, block
//    of query tokens); wave w owns 32 MFMA columns (2 blocks of 16), a
//    column being one (query token, head of the GQA group) pair, heads
//    fastest, with its Q rows held in registers for the whole key loop;
//  * the workgroup walks 32-key tiles up to its last query's position: the
//    512 threads gather a tile's K and V rows (16 B each, coalesced per row)
//    into registers one tile ahead, store them to a double-buffered LDS
//    tile of padded rows, and every wave computes from LDS, so each key
//    row leaves L2 once per workgroup instead of once per wave;
//  * page bases come two tiles ahead (block table one tile before offsets),
//    so no load waits on a dependent load inside the loop;
//  * S^T = K Q^T on v_mfma_f32_16x16x32 (K rows by ds_read_b128); V^T comes
//    straight from the row-major V tile by the gfx950 transposing LDS read
//    ds_read_b64_tr_b16, then O^T += V^T P^T; one V^T fragment serves both
//    of the wave's column blocks;
//  * causal masking only on tiles that cross a column's position; online
//    softmax in the log2 domain, rescaling only when a column's maximum grows
//    by more than 8 (until then P <= 2^8, harmless in fp32 / 16-bit).
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
    int row_bytes, data_bytes, head_dim, bs_shift;
    float scale_log2;
    float scale;
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

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

// Two fp32 -> one dword of 16-bit elements (round to nearest even).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    if constexpr (DT == kDtF16) {
        const f16x2 v = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
        return __builtin_bit_cast(uint32_t, v);
    } else {
        const bf16x2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
        return __builtin_bit_cast(uint32_t, v);
    }
}

// NaN-propagating maximum (v_maximum3_f32): unlike fmaxf it needs no
// canonicalization of MFMA results.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Maximum / sum over the 4 lanes (l, l^16, l^32, l^48) holding one MFMA
// output column.  v_permlane16_swap(x, x) leaves x[l] in one result and
// x[l ^ 16] in the other (v_permlane32_swap: x[l ^ 32]), so a symmetric
// operation of the pair reduces across rows with VALU ops only.
__device__ __forceinline__ float xor16_pair(float x, bool mx) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    const float a = __uint_as_float(r[0]), c = __uint_as_float(r[1]);
    return mx ? vmax(a, c) : a + c;
}
__device__ __forceinline__ float xor32_pair(float x, bool mx) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    const float a = __uint_as_float(r[0]), c = __uint_as_float(r[1]);
    return mx ? vmax(a, c) : a + c;
}
__device__ __forceinline__ float col_max(float x) { return xor32_pair(xor16_pair(x, true), true); }

// ds_read_b64_tr_b16 on a 16-lane group: lane (a + 4s) gives the address of
// 4 consecutive 16-bit elements M[a + 4s][0..3]; lane (4a + e) receives
// M[a][e], M[a + 4][e], M[a + 8][e], M[a + 12][e].  With lane a + 4s pointing
// at V[key0 + s][d0 + 4a], lane i gets V[key0 + 0..3][d0 + i].
__device__ __forceinline__ u32x2 lds_read_tr(const uint8_t* p) {
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
    return __builtin_bit_cast(u32x2, v);
}

template <int D, int KT>
struct Shape {
    static constexpr int CH = D / 8;          // 16-byte chunks per key row
    static constexpr int KC = D / 32;         // k-steps of S^T = K Q^T
    static constexpr int DB = D / 16;         // 16-row blocks of O^T
    // Padded LDS rows, 32 bytes past the row's data for both K and V: the
    // K fragment reads (ds_read_b128, 16 keys x 16 B) and the transposing V
    // reads are then free of bank conflicts on gfx950 (measured: a 16-byte
    // pad on K rows costs every K read 8 LDS cycles instead of 4), and every
    // fragment offset stays linear in (key block, chunk), an instruction
    // immediate.
    static constexpr int KROW = 2 * D + 32;
    static constexpr int VROW = 2 * D + 32;
    static constexpr int KTILE = KT * KROW;
    static constexpr int BUF = KTILE + KT * VROW;   // one K + V tile of KT keys
};

// Workgroups over (query-token block, kv head), kv head fastest: blockIdx.x
// = item * Hkv + g, items in longest-first order (see below).  Workgroups are dealt to the 8 XCDs round-robin, so with
// 8 kv heads every XCD serves one head and its L2 holds that head's pages
// (shared prefixes included) for all sequences.
template <int DT, int D, int G, int NW, int NCB, int KT>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void attn_prefill_mfma(PrefillParams p, const uint8_t* __restrict__ kreg,
                       const uint8_t* __restrict__ vreg, const int32_t* __restrict__ bt,
                       const int32_t* __restrict__ sl, const int32_t* __restrict__ qsl,
                       const uint64_t* __restrict__ offs) {
    using S = Shape<D, KT>;
    constexpr int KC = S::KC, DB = S::DB;
    // fp8-e4m3 pages: rows are gathered as 8-bit codes (half the bytes) and
    // dequantized with their page's scale to bf16 as they are stored to LDS;
    // from there on the tile is a bf16 tile (MFMA, q and out in bf16)
    constexpr bool F8 = DT == kDtFP8;
    constexpr int MDT = F8 ? kDtBF16 : DT;
    constexpr int EB = F8 ? 1 : 2;                // bytes per K/V element in the page
    constexpr int CH = D * EB / 16;               // 16-byte chunks per key row in the page
    constexpr int NKB = KT / 16;         // 16-key blocks of S^T per tile
    constexpr int NKS = KT / 32;         // 32-key k-steps of P V per tile
    constexpr int NT = NW * 64;          // threads
    constexpr int CPT = 2 * KT * CH / NT;   // 16-byte chunks per thread per tile (K and V)
    static_assert(CPT >= 1 && 2 * KT * CH % NT == 0, "tile does not split over the threads");
    constexpr int TPB = 16 / G;          // query tokens per column block
    constexpr int TPW = NCB * TPB;       // per wave
    constexpr int TWG = NW * TPW;        // per workgroup
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * S::BUF];   // 2 x (K tile, V tile)

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ln = lane & 15, lg = lane >> 4;
    const int g = static_cast<int>(blockIdx.x) % p.kv_heads;
    const int item = static_cast<int>(blockIdx.x) / p.kv_heads;

    // ---- sequence and token block of this workgroup ----
    // Items are dealt longest first: rank r = 0 is every sequence's last
    // token block (the most keys under the causal mask), r = 1 the block
    // before it, and so on; within a rank, sequences in order.  For chunks of
    // equal length this is longest-processing-time order, so the workgroups
    // that start last are the short ones and the rounds end together.
    int b = -1, blk = 0;
    {
        auto blocks_of = [&](int bb) {   // token blocks of sequence bb (0 past the batch)
            const int n = bb < p.batch ? qsl[bb + 1] - qsl[bb] : 0;
            return n > 0 ? (n + TWG - 1) / TWG : 0;
        };
        const int v0 = blocks_of(lane);   // the first 64 sequences stay in registers
        int base = 0;                      // items of the ranks before r
        for (int r = 0; b < 0; ++r) {
            int cnt = 0;
            for (int c = 0; c < p.batch; c += 64) {
                const int v = c == 0 ? v0 : blocks_of(c + lane);
                cnt += __popcll(__ballot(v > r));
            }
            if (cnt == 0) break;          // no item of this rank: a spare workgroup
            if (item < base + cnt) {
                int j = item - base;       // the j-th sequence (in order) with more than r blocks
                for (int c = 0; c < p.batch; c += 64) {
                    const int v = c == 0 ? v0 : blocks_of(c + lane);
                    unsigned long long m = __ballot(v > r);
                    const int n = __popcll(m);
                    if (j < n) {
                        for (int k = 0; k < j; ++k) m &= m - 1;
                        const int bit = __ffsll(static_cast<long long>(m)) - 1;
                        b = c + bit;
                        blk = __shfl(v, bit) - 1 - r;
                        break;
                    }
                    j -= n;
                }
                break;
            }
            base += cnt;
        }
    }
    b = __builtin_amdgcn_readfirstlane(b);
    if (b < 0) return;                     // whole workgroup: uniform
    blk = __builtin_amdgcn_readfirstlane(blk);
    const int q0 = qsl[b];
    const int len = qsl[b + 1] - q0;
    const int L = min(sl[b], p.mbps << p.bs_shift);
    const int first_pos = L - len;         // position of the chunk's first query
    const int tok0_wg = blk * TWG;
    // queries before position 0 (more queries than cached tokens) see no key;
    // their rows are written as zeros
    const int nt_wg = (max(0, first_pos + min(tok0_wg + TWG, len)) + KT - 1) / KT;
    const int tok0 = tok0_wg + wave * TPW;  // this wave's first query (chunk index)
    const bool wave_live = tok0 < len;
    const int tok_last = min(tok0 + TPW, len) - 1;
    const int nt_w = wave_live ? (max(0, first_pos + tok_last + 1) + KT - 1) / KT : 0;
    const int qmin = first_pos + tok0;     // smallest position among the wave's columns

    // ---- columns: query token (clamped into the chunk; extra columns are
    // computed on a duplicate and never stored) and its position ----
    int qpos[NCB];
    u32x4 qf[NCB][KC];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
        const int t = max(0, min(tok0 + cb * TPB + ln / G, len - 1));
        qpos[cb] = first_pos + t;
        const uint8_t* qrow =
            p.q + ((static_cast<size_t>(q0) + t) * p.num_q_heads + g * G + ln % G) * D * 2;
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
            qf[cb][kc] = *reinterpret_cast<const u32x4*>(qrow + (kc * 32 + lg * 8) * 2);
    }
    // Q loads stay first: the first tile store then waits for them too, and
    // no wait inside the key loop is left counting them
    __builtin_amdgcn_sched_barrier(0);

    // ---- tile gather: chunk q = tid + NT * i of the tile's 2 x KT x CH
    // chunks is (tensor q / (KT CH), key (q / CH) % KT, chunk q % CH); keys
    // past the sequence read its last row (finite; P = 0 there) ----
    auto c_tensor = [&](int i) { return (tid + NT * i) / (KT * CH); };
    auto c_key = [&](int i) { return ((tid + NT * i) / CH) % KT; };
    const int tc = tid % CH;
    const int32_t* row = bt + static_cast<size_t>(b) * p.mbps;
    const int bmask = (1 << p.bs_shift) - 1;
    const uint32_t head_off = static_cast<uint32_t>(g * D * EB + tc * 16);
    auto key_tok = [&](int kt, int i) { return min(kt * KT + c_key(i), L - 1); };
    auto page_entry = [&](int kt, int i) { return row[key_tok(kt, i) >> p.bs_shift]; };
    // Loaded values pass through an empty asm where they are used, so the
    // compiler cannot fold their arithmetic back next to the load (which
    // would wait there for the loads issued just before).
    auto page_offs = [&](int entry) {
        asm volatile("" : "+v"(entry));
        return offs[entry];
    };
    // With two chunks per thread (KT * CH == NT: 16-bit pages at head_dim
    // 128 with 32-key tiles, fp8 pages with 64-key tiles) chunk 0 is a K row
    // piece and chunk 1 the V piece of the same key at the same place, so one
    // page lookup and one address serve both (for fp8, with the page's two
    // scales).
    constexpr int NPG = CPT == 2 ? 1 : CPT;   // page lookups per thread per tile
    static_assert(CPT != 2 || KT * CH == NT, "chunks 0 and 1 share their key");
    u32x4 gch[CPT];
    float gsc[F8 ? CPT : 1];   // fp8: the chunk's page scale for kv head g
    auto gather = [&](int kt, const uint64_t (&pg)[NPG]) {
        if constexpr (NPG == 1 && CPT == 2) {
            uint64_t page = pg[0];
            asm volatile("" : "+v"(page));
            const uint64_t a =
                page * 2ull + (__umul24(key_tok(kt, 0) & bmask, p.row_bytes) + head_off);
            gch[0] = *reinterpret_cast<const u32x4*>(kreg + a);
            gch[1] = *reinterpret_cast<const u32x4*>(vreg + a);
            if constexpr (F8) {
                const uint64_t sa = page * 2ull + static_cast<uint32_t>(p.data_bytes + g * 4);
                gsc[0] = *reinterpret_cast<const float*>(kreg + sa);
                gsc[1] = *reinterpret_cast<const float*>(vreg + sa);
            }
        } else {
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                uint64_t page = pg[i];
                asm volatile("" : "+v"(page));
                const uint8_t* reg = c_tensor(i) ? vreg : kreg;
                const uint64_t a =
                    page * 2ull + (__umul24(key_tok(kt, i) & bmask, p.row_bytes) + head_off);
                gch[i] = *reinterpret_cast<const u32x4*>(reg + a);
                if constexpr (F8)
                    gsc[i] = *reinterpret_cast<const float*>(
                        reg + page * 2ull + static_cast<uint32_t>(p.data_bytes + g * 4));
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int k = c_key(i);
            const int off = c_tensor(i) ? S::KTILE + k * S::VROW : k * S::KROW;
            if constexpr (F8) {
                // 16 codes -> 16 bf16 = bf16(e4m3 value * scale), 32 bytes
                u32x4 lo, hi;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const auto a = __builtin_amdgcn_cvt_pk_f32_fp8(gch[i][w], false);
                    const auto b = __builtin_amdgcn_cvt_pk_f32_fp8(gch[i][w], true);
                    const uint32_t x = pack2<kDtBF16>(a[0] * gsc[i], a[1] * gsc[i]);
                    const uint32_t y = pack2<kDtBF16>(b[0] * gsc[i], b[1] * gsc[i]);
                    if (w < 2) {
                        lo[2 * w] = x;
                        lo[2 * w + 1] = y;
                    } else {
                        hi[2 * w - 4] = x;
                        hi[2 * w - 3] = y;
                    }
                }
                *reinterpret_cast<u32x4*>(&lds[buf * S::BUF + off + tc * 32]) = lo;
                *reinterpret_cast<u32x4*>(&lds[buf * S::BUF + off + tc * 32 + 16]) = hi;
            } else {
                *reinterpret_cast<u32x4*>(&lds[buf * S::BUF + off + tc * 16]) = gch[i];
            }
        }
    };

    // l (the softmax denominator) accumulates on the MFMA as ones x P^T: every
    // row of lsum[cb] holds the column sums of the 16-bit P used for O
    const u32x4 ones = MDT == kDtF16 ? u32x4{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u}
                                    : u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
    float m_run[NCB], nmu[NCB];
    bool all_seen = false;   // every column of the wave has a finite maximum
    f32x4 lsum[NCB];
    f32x4 acc[NCB][DB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
        m_run[cb] = -INFINITY;
        nmu[cb] = 0.0f;
        lsum[cb] = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < DB; ++i) acc[cb][i] = f32x4{0, 0, 0, 0};
    }

    // LDS byte offsets of this lane's fragments: K (key ln of a 16-key block,
    // chunk lg of a 32-element k-step); V^T (lane a + 4s reads key 4lg + s of
    // a 16-key block, elements 4a..4a+3 of a 16-element d block)
    const int k_lane = ln * S::KROW + lg * 16;
    const int v_lane = S::KTILE + (4 * lg + (ln >> 2)) * S::VROW + (ln & 3) * 8;

    // One KT-key tile in two phases.  softmax_phase: S^T = K Q^T, causal
    // mask (only on a tile that crosses some column's position), column
    // maxima, lazy rescale, P into pf and l += ones x P^T.  pv_phase:
    // O^T += V^T P^T in 32-key k-steps.
    auto softmax_phase = [&](int buf, int kt, u32x4 (&pf)[NCB][NKS]) {
        const uint8_t* kb = lds + buf * S::BUF + k_lane;
        f32x4 s[NCB][NKB];
#pragma unroll
        for (int hb = 0; hb < NKB; ++hb) {
            u32x4 kf[KC];
#pragma unroll
            for (int kc = 0; kc < KC; ++kc)
                kf[kc] = *reinterpret_cast<const u32x4*>(kb + hb * 16 * S::KROW + kc * 64);
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                s[cb][hb] = f32x4{0, 0, 0, 0};
#pragma unroll
                for (int kc = 0; kc < KC; ++kc)
                    s[cb][hb] = mfma16<MDT>(kf[kc], qf[cb][kc], s[cb][hb]);
            }
        }
        if (kt * KT + KT - 1 > qmin) {
            const int key0 = kt * KT + 4 * lg;
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
                for (int hb = 0; hb < NKB; ++hb)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (key0 + 16 * hb + r > qpos[cb]) s[cb][hb][r] = -INFINITY;
        }
        // exp arguments s * scale_log2 - m with the running column maxima m
        // (-m kept in nmu; 0 for a column with no visible key yet, whose P is
        // then 0 through its masked scores).  The maxima are recomputed only
        // when some argument exceeds 7.99 -- a column maximum may have grown
        // by more than 8 -- or while some column has seen no key: for
        // |m| < 2^16 (the rounding of m + 8 below 0.01) this takes the exact
        // rule below on every tile where it would rescale, and skips the
        // cross-lane maxima on the others.
        float arg[NCB][NKB][4];
        auto args = [&]() {
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
                for (int hb = 0; hb < NKB; ++hb)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        arg[cb][hb][r] = fmaf(s[cb][hb][r], p.scale_log2, nmu[cb]);
        };
        args();
        float amax = -INFINITY;
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int hb = 0; hb < NKB; ++hb)
                amax = vmax(amax, vmax(vmax(arg[cb][hb][0], arg[cb][hb][1]),
                                       vmax(arg[cb][hb][2], arg[cb][hb][3])));
        if (__builtin_amdgcn_ballot_w64(amax > 7.99f) || !all_seen) {
            // column maxima of the raw scores (scale > 0), masked keys -inf
            float mt[NCB];
            bool grow[NCB];
            bool any_grow = false;
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                float x = -INFINITY;
#pragma unroll
                for (int hb = 0; hb < NKB; ++hb)
                    x = vmax(x, vmax(vmax(s[cb][hb][0], s[cb][hb][1]), vmax(s[cb][hb][2], s[cb][hb][3])));
                mt[cb] = col_max(x) * p.scale_log2;
                // rescale only when the column maximum grows by more than 8
                grow[cb] = mt[cb] > m_run[cb] + 8.0f;
                any_grow |= grow[cb];
            }
            if (__builtin_amdgcn_ballot_w64(any_grow)) {
#pragma unroll
                for (int cb = 0; cb < NCB; ++cb) {
                    if (!__builtin_amdgcn_ballot_w64(grow[cb])) continue;
                    // (a column that does not grow keeps its scale exactly)
                    const float corr = grow[cb] ? __builtin_amdgcn_exp2f(m_run[cb] - mt[cb]) : 1.0f;
                    lsum[cb] *= corr;
#pragma unroll
                    for (int db = 0; db < DB; ++db) acc[cb][db] *= corr;
                    m_run[cb] = grow[cb] ? mt[cb] : m_run[cb];
                }
                bool unseen = false;
#pragma unroll
                for (int cb = 0; cb < NCB; ++cb) {
                    nmu[cb] = m_run[cb] == -INFINITY ? 0.0f : -m_run[cb];
                    unseen |= m_run[cb] == -INFINITY;
                }
                all_seen = !__builtin_amdgcn_ballot_w64(unseen);
                args();
            }
        }
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
            for (int j = 0; j < NKS; ++j) {
                // k-step j: keys 4lg..+3 of block 2j, then of block 2j + 1
                float pv[8];
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        pv[4 * h + r] = __builtin_amdgcn_exp2f(arg[cb][2 * j + h][r]);
#pragma unroll
                for (int i = 0; i < 4; ++i) pf[cb][j][i] = pack2<MDT>(pv[2 * i], pv[2 * i + 1]);
                lsum[cb] = mfma16<MDT>(ones, pf[cb][j], lsum[cb]);
            }
        }
    };
    auto pv_phase = [&](int buf, const u32x4 (&pf)[NCB][NKS]) {
#pragma unroll
        for (int j = 0; j < NKS; ++j) {
            const uint8_t* vb = lds + buf * S::BUF + v_lane + 32 * j * S::VROW;
            u32x4 vf[DB];
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const u32x2 lo = lds_read_tr(vb + db * 32);
                const u32x2 hi = lds_read_tr(vb + 16 * S::VROW + db * 32);
                vf[db] = u32x4{lo[0], lo[1], hi[0], hi[1]};
            }
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    acc[cb][db] = mfma16<MDT>(vf[db], pf[cb][j], acc[cb][db]);
        }
    };

    if (nt_wg > 0) {   // (no tile at all: no column has a visible key)
        uint64_t pg[NPG];
        int ent[NPG];
#pragma unroll
        for (int i = 0; i < NPG; ++i) pg[i] = page_offs(page_entry(0, i));
        gather(0, pg);
#pragma unroll
        for (int i = 0; i < NPG; ++i) pg[i] = page_offs(page_entry(1, i));
#pragma unroll
        for (int i = 0; i < NPG; ++i) ent[i] = page_entry(2, i);
        store_tile(0);
        gather(1, pg);
#pragma unroll
        for (int i = 0; i < NPG; ++i) pg[i] = page_offs(ent[i]);       // tile 2
#pragma unroll
        for (int i = 0; i < NPG; ++i) ent[i] = page_entry(3, i);        // tile 3
        __syncthreads();
        // Gathers past the last tile read clamped (valid) rows and are never
        // consumed; issuing them unconditionally keeps every iteration's
        // load sequence identical, so the compiler's counter waits stay exact.
        // Two tiles per trip, so each LDS buffer index is a constant (an odd
        // count runs one trip with nothing to compute on its second tile).
        auto step = [&](int kt, int buf) {
            if (kt < nt_w) {
                u32x4 pf[NCB][NKS];
                softmax_phase(buf, kt, pf);
                pv_phase(buf, pf);
            }
            store_tile(buf ^ 1);
            __syncthreads();
            gather(kt + 2, pg);
#pragma unroll
            for (int i = 0; i < NPG; ++i) pg[i] = page_offs(ent[i]);   // tile kt + 3
#pragma unroll
            for (int i = 0; i < NPG; ++i) ent[i] = page_entry(kt + 4, i);
        };
        for (int kt = 0; kt < nt_wg; kt += 2) {
            step(kt, 0);
            step(kt + 1, 1);
        }
    }

    // ---- store the columns that are real queries ----
    if (!wave_live) return;
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
        const float lt = lsum[cb][0];
        const int t = tok0 + cb * TPB + ln / G;
        if (t < len) {
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            uint16_t* o = reinterpret_cast<uint16_t*>(p.out) +
                          ((static_cast<size_t>(q0) + t) * p.num_q_heads + g * G + ln % G) * D +
                          4 * lg;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                u32x2 w;
                w[0] = pack2<MDT>(acc[cb][db][0] * inv, acc[cb][db][1] * inv);
                w[1] = pack2<MDT>(acc[cb][db][2] * inv, acc[cb][db][3] * inv);
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
    // q/out: f16 for f16 pools, fp32 for fp32 pools, bf16 otherwise
    const size_t io_off = (static_cast<size_t>(rowi) * p.num_q_heads + h) * D * io_bytes<DT>();
    uint8_t* orow = reinterpret_cast<uint8_t*>(p.out) + io_off;
    if (pos < 0) {
        for (int d = lane; d < D; d += 64) io_store<DT>(orow, d, 0.0f);
        return;
    }
    const uint8_t* qrow = reinterpret_cast<const uint8_t*>(p.q) + io_off;
    float qv[4], acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        qv[i] = d < D ? io_load<DT>(qrow, d) : 0.0f;
        acc[i] = 0.0f;
    }
    const int esize = kv_elem_bytes<DT>();
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
                } else if constexpr (DT == kDtF32) {
                    kx = reinterpret_cast<const float*>(kreg + roff)[d];
                    vx = reinterpret_cast<const float*>(vreg + roff)[d];
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
        const float e = kexp<DT>(dot - m_new);
        const float corr = kexp<DT>(m - m_new);
        s = s * corr + e;
        m = m_new;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = acc[i] * corr + e * vv[i];
    }
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        if (d < D) io_store<DT>(orow, d, acc[i] * inv);
    }
}

template <int DT, int D, int G>
bool launch_mfma(const dev::AttnPrefillArgs& a, PrefillParams& p, hipStream_t s, std::string* err) {
    // 8 waves of 32 columns (2 waves per SIMD), 32 keys per tile.  Measured
    // on the Cfg3 shape (MI355X): 64-key tiles ~4% slower on bf16 pages, equal
    // on fp8 pages, ~11% slower at head_dim 64; 4-wave workgroups (two per
    // CU) ~10% slower; 64 columns per wave does not fit 2 waves per SIMD.
    constexpr int NW = 8, NCB = 2, KT = 32;
    constexpr int TWG = NW * NCB * (16 / G);
    const long long blocks =
        (static_cast<long long>(a.total_query_tokens) / TWG + a.batch + 1) * p.kv_heads;
    if (blocks > INT_MAX) {
        *err = "prefill: too many query tokens";
        return false;
    }
    hipLaunchKernelGGL((attn_prefill_mfma<DT, D, G, NW, NCB, KT>), dim3(static_cast<unsigned>(blocks)),
                       dim3(NW * 64), 0, s, p, reinterpret_cast<const uint8_t*>(a.k_base),
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
    p.bs_shift = 0;
    while ((1u << p.bs_shift) < a.block_size) ++p.bs_shift;
    p.scale = a.scale;
    p.scale_log2 = a.scale * 1.4426950408889634f;
    hipStream_t s = reinterpret_cast<hipStream_t>(a.stream);
    if (a.total_query_tokens == 0 || a.batch == 0) return true;

    const int G = p.group;
    const bool mfma_group = p.num_q_heads % p.kv_heads == 0 && (G == 1 || G == 2 || G == 4 ||
                                                                G == 8 || G == 16);
    const bool mfma_dim = a.head_dim == 64 || a.head_dim == 128;
    const bool pow2_bs = (1u << p.bs_shift) == a.block_size;
    // (the MFMA kernel takes column maxima of the raw scores: scale > 0)
    const bool mfma_type = a.dtype == kDtF16 || a.dtype == kDtBF16 ||
                           (a.dtype == kDtFP8 && a.head_dim == 128);
    int generic_flag = 0;
    if (mfma_type && mfma_group && mfma_dim && pow2_bs && a.scale > 0.0f &&
        !dev::tunable(dev::Tun::kAttnGeneric, &generic_flag)) {
        if (a.dtype == kDtFP8) return launch_group<kDtFP8, 128>(a, p, s, err);
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
        case kDtF32:
            hipLaunchKernelGGL(attn_prefill_generic<kDtF32>, grid, dim3(64), 0, s, p, kb, vb, btp,
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
