/*
 * oracle.c -- CPU restatement of the reference's decode-step data path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for tests/, smoke()
 * and the CPU baseline of bench.py.  Never linked into the product.
 *
 * Build: make -C oracle   (gcc -O3 -fopenmp; no reference sources are used)
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define SB_BYTES ((size_t)2 * 1024 * 1024)

/* ======================================================================
 * Numeric formats (the reference is f16-only, ref pool.rs:203-204; bf16 and
 * fp8 follow their published definitions: bf16 = upper half of IEEE binary32
 * with round-to-nearest-even, OCP FP8 e4m3fn with RNE and saturation).
 * ====================================================================== */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t oracle_f32_to_bf16(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE binary16 with RNE, gradual underflow and overflow to infinity
 * (ref: half 2.7.1 f16::from_f32, used at llama_transformer.rs:70). */
uint16_t oracle_f32_to_f16(float x) {
    uint32_t u = f2u(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;          /* NaN */
    if (a >= 0x477ff000u) return sign | 0x7c00u;         /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                               /* below 2^-14: subnormal */
        /* value = a * 2^24 in units of the f16 subnormal step 2^-24 */
        float v = u2f(a) * 16777216.0f;                  /* exact scaling */
        float r = rintf(v);                              /* RNE */
        return sign | (uint16_t)r;
    }
    uint32_t e = (a >> 23) - 112;                        /* rebias 127 -> 15 */
    uint32_t m = a & 0x7fffffu;
    uint32_t q = m >> 13, rem = m & 0x1fffu;
    uint32_t h = (e << 10) | q;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) h += 1;  /* carry may bump e */
    return sign | (uint16_t)h;
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = ldexpf((float)m, -24);
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

uint8_t oracle_f32_to_e4m3(float x) {
    uint32_t bits = f2u(x);
    uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
    float a = fabsf(x);
    if (a != a) return sign | 0x7fu;
    if (a >= 448.0f) return sign | 0x7eu;
    if (a < 0.015625f) return sign | (uint8_t)rintf(a * 512.0f);  /* 2^-9 grid */
    uint32_t ab = f2u(a);
    int e = (int)(ab >> 23) - 127;
    uint32_t mant = ab & 0x7fffffu, q = mant >> 20, rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ++q;
    if (q == 8) { q = 0; ++e; }
    uint32_t code = ((uint32_t)(e + 7) << 3) | q;
    if (code > 0x7eu) code = 0x7eu;
    return sign | (uint8_t)code;
}

float oracle_e4m3_to_f32(uint8_t b) {
    int s = b & 0x80, e = (b >> 3) & 0xf, m = b & 7;
    float v;
    if (e == 0xf && m == 7) return NAN;
    if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return s ? -v : v;
}

void oracle_encode_array(int dtype, const float *src, void *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        switch (dtype) {
            case 0: ((uint16_t *)dst)[i] = oracle_f32_to_f16(src[i]); break;
            case 1: ((uint16_t *)dst)[i] = oracle_f32_to_bf16(src[i]); break;
            case 2: ((uint8_t *)dst)[i] = oracle_f32_to_e4m3(src[i]); break;
            default: ((float *)dst)[i] = src[i]; break;
        }
    }
}

void oracle_decode_array(int dtype, const void *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        switch (dtype) {
            case 0: dst[i] = oracle_f16_to_f32(((const uint16_t *)src)[i]); break;
            case 1: dst[i] = oracle_bf16_to_f32(((const uint16_t *)src)[i]); break;
            case 2: dst[i] = oracle_e4m3_to_f32(((const uint8_t *)src)[i]); break;
            default: dst[i] = ((const float *)src)[i]; break;
        }
    }
}

static size_t esize_of(int dtype) { return dtype == 2 ? 1 : (dtype == 3 ? 4 : 2); }

/* ======================================================================
 * Page allocator, restated from the reference's structure: one free stack of
 * (superblock, index) handles per layer and per K/V (ref superblock.rs:40-142,
 * LayerKvPool :151-171), moved in lockstep (ref pool.rs:364-410); logical
 * block ids with a recycled-id stack (ref pool.rs:412-454); sequences
 * (ref pool.rs:551-572).  Reference counts are this build's CoW extension.
 * ====================================================================== */

typedef struct { uint32_t sb, idx; } Handle;

typedef struct {
    Handle *free;    /* LIFO stack */
    size_t nfree;
    size_t sb_count;
} LayerPool;

typedef struct {
    uint64_t va;
    uint32_t sb, idx;
    uint32_t refcount;
    int in_use;
    int loc;            /* 0 GPU, 1 CPU swap, 3 evicting, 4 restoring (kcmm.h:63-68) */
    uint64_t cpu_off;   /* swap offset while loc == 1 */
} OBlock;

typedef struct OTier OTier;

typedef struct {
    uint32_t *table;
    size_t n, cap;
    uint32_t seq_len;
} OSeq;

struct OPool {
    size_t block_size, num_layers, kv_heads, head_dim;
    size_t elem_per_block, block_bytes, bps, max_blocks_per_seq, max_blocks_total;
    size_t max_physical, region_bytes;
    int rollback;
    LayerPool *pools;        /* 2*L: K pools then V pools */
    OBlock *blocks;
    size_t nblocks, cap_blocks;
    uint32_t *free_ids;
    size_t nfree_ids, cap_free_ids;
    OSeq *seqs;
    size_t nseqs, cap_seqs;
    OTier *tier;             /* NULL: tiering disabled */
};

static void tier_on_allocate(OTier *t, Handle h);
static void tier_free_slot(OTier *t, uint64_t off);
static void tier_delete(OTier *t);

static void *grow(void *p, size_t *cap, size_t need, size_t elem) {
    if (need <= *cap) return p;
    size_t c = *cap ? *cap : 16;
    while (c < need) c *= 2;
    *cap = c;
    return realloc(p, c * elem);
}

OPool *opool_new(size_t block_size, size_t num_layers, size_t kv_heads, size_t head_dim,
                 size_t max_batch, size_t max_seq_len, int dtype, int rollback) {
    OPool *p = (OPool *)calloc(1, sizeof(OPool));
    p->block_size = block_size ? block_size : 16;              /* ref ffi.rs:477 */
    p->num_layers = num_layers;
    p->kv_heads = kv_heads;
    p->head_dim = head_dim;
    p->elem_per_block = kv_heads * p->block_size * head_dim;   /* ref pool.rs:202 */
    size_t data = p->elem_per_block * esize_of(dtype);
    p->block_bytes = dtype == 2 ? (data + kv_heads * 4 + 255) / 256 * 256 : data;
    p->bps = SB_BYTES / p->block_bytes;                        /* ref superblock.rs:78 */
    p->max_blocks_per_seq = (max_seq_len + p->block_size - 1) / p->block_size;
    p->max_blocks_total = max_batch * p->max_blocks_per_seq;  /* ref pool.rs:206-207 */
    size_t sbs = (p->max_blocks_total + p->bps - 1) / p->bps;
    p->max_physical = sbs * p->bps;                            /* ref pool.rs:1145-1152 */
    size_t ref_va = (p->max_blocks_total * p->block_bytes + SB_BYTES - 1) / SB_BYTES * SB_BYTES;
    p->region_bytes = ref_va > sbs * SB_BYTES ? ref_va : sbs * SB_BYTES;
    p->rollback = rollback;
    p->pools = (LayerPool *)calloc(2 * num_layers, sizeof(LayerPool));
    for (size_t l = 0; l < 2 * num_layers; ++l)
        p->pools[l].free = (Handle *)malloc((p->max_physical + 1) * sizeof(Handle));
    return p;
}

void opool_delete(OPool *p) {
    if (!p) return;
    for (size_t l = 0; l < 2 * p->num_layers; ++l) free(p->pools[l].free);
    for (size_t s = 0; s < p->nseqs; ++s) free(p->seqs[s].table);
    free(p->pools); free(p->blocks); free(p->free_ids); free(p->seqs);
    if (p->tier) tier_delete(p->tier);
    free(p);
}

/* ref pool.rs:323-362 */
static int ensure_capacity(OPool *p) {
    if (p->pools[0].nfree > 0) return 0;
    if (p->pools[0].sb_count * p->bps >= p->max_physical) return -1;
    for (size_t l = 0; l < 2 * p->num_layers; ++l) {
        LayerPool *lp = &p->pools[l];
        uint32_t sb = (uint32_t)lp->sb_count++;              /* ref superblock.rs:103-116 */
        for (size_t i = 0; i < p->bps; ++i) {
            lp->free[lp->nfree].sb = sb;
            lp->free[lp->nfree].idx = (uint32_t)i;
            lp->nfree++;
        }
    }
    return 0;
}

/* ref pool.rs:364-454 */
static int alloc_one(OPool *p, uint32_t *id_out) {
    if (ensure_capacity(p)) return -1;
    Handle h = {0, 0};
    for (size_t l = 0; l < 2 * p->num_layers; ++l) {
        LayerPool *lp = &p->pools[l];
        Handle x = lp->free[--lp->nfree];
        if (l == 0) h = x;
        else if (x.sb != h.sb || x.idx != h.idx) abort();  /* lockstep broken */
    }
    OBlock b;
    b.va = (uint64_t)h.sb * SB_BYTES + (uint64_t)h.idx * p->block_bytes;
    b.sb = h.sb; b.idx = h.idx; b.refcount = 1; b.in_use = 1;
    b.loc = 0; b.cpu_off = 0;
    uint32_t id;
    if (p->nfree_ids > 0) {
        id = p->free_ids[--p->nfree_ids];
        p->blocks[id] = b;
    } else {
        p->blocks = (OBlock *)grow(p->blocks, &p->cap_blocks, p->nblocks + 1, sizeof(OBlock));
        id = (uint32_t)p->nblocks++;
        p->blocks[id] = b;
    }
    *id_out = id;
    if (p->tier) tier_on_allocate(p->tier, h);   /* ref pool.rs:446-449 */
    return 0;
}

static void push_handle(OPool *p, uint32_t sb, uint32_t idx) {
    for (size_t l = 0; l < 2 * p->num_layers; ++l) {
        LayerPool *lp = &p->pools[l];
        lp->free[lp->nfree].sb = sb;
        lp->free[lp->nfree].idx = idx;
        lp->nfree++;
    }
}

int opool_alloc(OPool *p, uint32_t n, uint32_t *out) {
    size_t before = p->nblocks;
    for (uint32_t i = 0; i < n; ++i) {
        if (alloc_one(p, &out[i])) {
            if (p->rollback) {
                for (uint32_t j = i; j-- > 0;) {
                    OBlock *b = &p->blocks[out[j]];
                    push_handle(p, b->sb, b->idx);
                    if (out[j] >= before) {
                        p->nblocks--;
                    } else {
                        memset(b, 0, sizeof(*b));
                        p->free_ids = (uint32_t *)grow(p->free_ids, &p->cap_free_ids,
                                                       p->nfree_ids + 1, sizeof(uint32_t));
                        p->free_ids[p->nfree_ids++] = out[j];
                    }
                }
            }
            return -1;
        }
    }
    return 0;
}

/* ref pool.rs:478-549 (+ reference counts) */
void opool_release(OPool *p, const uint32_t *ids, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t id = ids[i];
        if (id >= p->nblocks) continue;
        OBlock *b = &p->blocks[id];
        if (!b->in_use) continue;
        if (b->refcount > 1) { b->refcount--; continue; }
        b->in_use = 0;
        b->refcount = 0;
        /* ref pool.rs:491-545: a swapped-out block gives back its swap slot */
        if (b->loc == 1) {
            if (p->tier) tier_free_slot(p->tier, b->cpu_off);
        } else {
            push_handle(p, b->sb, b->idx);
        }
        p->free_ids = (uint32_t *)grow(p->free_ids, &p->cap_free_ids, p->nfree_ids + 1,
                                       sizeof(uint32_t));
        p->free_ids[p->nfree_ids++] = id;
    }
}

static OSeq *new_seq(OPool *p) {
    p->seqs = (OSeq *)grow(p->seqs, &p->cap_seqs, p->nseqs + 1, sizeof(OSeq));
    OSeq *s = &p->seqs[p->nseqs++];
    memset(s, 0, sizeof(*s));
    return s;
}

static void seq_push(OSeq *s, uint32_t v) {
    s->table = (uint32_t *)grow(s->table, &s->cap, s->n + 1, sizeof(uint32_t));
    s->table[s->n++] = v;
}

uint32_t opool_register(OPool *p, const uint32_t *table, uint32_t n) {
    OSeq *s = new_seq(p);
    for (uint32_t i = 0; i < n; ++i) seq_push(s, table[i]);
    return (uint32_t)(p->nseqs - 1);
}

void opool_unregister(OPool *p, uint32_t seq) {
    if (seq >= p->nseqs) return;
    OSeq *s = &p->seqs[seq];
    uint32_t *t = s->table;
    size_t n = s->n;
    s->table = NULL; s->n = 0; s->cap = 0; s->seq_len = 0;
    if (n) opool_release(p, t, (uint32_t)n);
    free(t);
}

int opool_append_block(OPool *p, uint32_t seq, uint32_t blk) {
    if (seq >= p->nseqs) return -1;
    seq_push(&p->seqs[seq], blk);
    return 0;
}

void opool_update_seq_len(OPool *p, uint32_t seq, uint32_t len) {
    if (seq < p->nseqs) p->seqs[seq].seq_len = len;
}

int opool_block_table(OPool *p, uint32_t seq, uint32_t *out, uint32_t max, uint32_t *count) {
    if (seq >= p->nseqs) { *count = 0; return -1; }
    uint32_t n = (uint32_t)(p->seqs[seq].n < max ? p->seqs[seq].n : max);
    memcpy(out, p->seqs[seq].table, n * sizeof(uint32_t));
    *count = n;
    return 0;
}

int opool_block_offset(OPool *p, uint32_t blk, uint64_t *out) {
    if (blk >= p->nblocks || !p->blocks[blk].in_use) return -1;
    *out = p->blocks[blk].va;
    return 0;
}

/* ref pool.rs:724-748 */
uint32_t opool_offsets_f16(OPool *p, uint64_t *out, uint32_t max) {
    uint32_t n = (uint32_t)(p->nblocks < max ? p->nblocks : max);
    for (uint32_t i = 0; i < n; ++i) out[i] = p->blocks[i].in_use ? p->blocks[i].va / 2 : 0;
    return n;
}

uint32_t opool_valid_flags(OPool *p, uint8_t *out, uint32_t max) {
    uint32_t n = (uint32_t)(p->nblocks < max ? p->nblocks : max);
    for (uint32_t i = 0; i < n; ++i) out[i] = p->blocks[i].in_use ? 1 : 0;
    return n;
}

int opool_table_offsets(OPool *p, uint32_t seq, uint64_t *out, uint32_t max, uint32_t *count) {
    *count = 0;
    if (seq >= p->nseqs) return -1;
    OSeq *s = &p->seqs[seq];
    for (size_t i = 0; i < s->n; ++i) {
        uint32_t id = s->table[i];
        if (id >= p->nblocks || !p->blocks[id].in_use) return -1;
    }
    uint32_t n = (uint32_t)(s->n < max ? s->n : max);
    for (uint32_t i = 0; i < n; ++i) out[i] = p->blocks[s->table[i]].va;
    *count = n;
    return 0;
}

/* Copy-on-write extension (vLLM fork / clear_copy_on_writes semantics,
 * ref patch_vllm.py:1083-1101, shadow_allocator.py:63-118). */
int opool_fork(OPool *p, uint32_t src, uint32_t *out_seq) {
    if (src >= p->nseqs) return -1;
    OSeq *d = new_seq(p);
    OSeq *s = &p->seqs[src];
    for (size_t i = 0; i < s->n; ++i) {
        uint32_t id = s->table[i];
        seq_push(d, id);
        if (id < p->nblocks && p->blocks[id].in_use) p->blocks[id].refcount++;
    }
    d->seq_len = s->seq_len;
    *out_seq = (uint32_t)(p->nseqs - 1);
    return 0;
}

int opool_share_prefix(OPool *p, uint32_t src, uint32_t dst, uint32_t n, uint32_t *out) {
    if (src >= p->nseqs || dst >= p->nseqs || p->seqs[src].n < n) return -1;
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t id = p->seqs[src].table[i];
        if (id >= p->nblocks || !p->blocks[id].in_use) return -1;
    }
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t id = p->seqs[src].table[i];
        p->blocks[id].refcount++;
        seq_push(&p->seqs[dst], id);
        out[i] = id;
    }
    return 0;
}

int opool_cow(OPool *p, uint32_t seq, uint32_t logical, uint32_t *src, uint32_t *dst) {
    if (seq >= p->nseqs || logical >= p->seqs[seq].n) return -1;
    uint32_t old = p->seqs[seq].table[logical];
    if (old >= p->nblocks || !p->blocks[old].in_use) return -1;
    if (p->blocks[old].refcount <= 1) return 0;
    if (p->blocks[old].loc != 0) return -1;   /* page data must be in HBM to copy */
    uint32_t nid;
    if (alloc_one(p, &nid)) return -1;
    p->seqs[seq].table[logical] = nid;
    p->blocks[old].refcount--;
    *src = old;
    *dst = nid;
    return 1;
}

/* One more reference on an in-use block (the prefix cache's hold); -1 if the
 * block is not in use. */
int opool_incref(OPool *p, uint32_t blk) {
    if (blk >= p->nblocks || !p->blocks[blk].in_use) return -1;
    p->blocks[blk].refcount++;
    return 0;
}

uint32_t opool_seq_len(OPool *p, uint32_t seq) {
    return seq < p->nseqs ? p->seqs[seq].seq_len : 0;
}

uint32_t opool_refcount(OPool *p, uint32_t blk) {
    if (blk >= p->nblocks || !p->blocks[blk].in_use) return 0;
    return p->blocks[blk].refcount;
}

static uint64_t in_use_count(OPool *p) {
    uint64_t n = 0;
    for (size_t i = 0; i < p->nblocks; ++i) n += p->blocks[i].in_use ? 1 : 0;
    return n;
}

void opool_stats(OPool *p, uint64_t *st) {
    uint64_t in_use = in_use_count(p);
    size_t sbc = p->pools[0].sb_count;
    st[0] = in_use;
    st[1] = p->nblocks;
    st[2] = sbc * p->bps;
    st[3] = p->pools[0].nfree;
    st[4] = p->nseqs;
    st[5] = p->num_layers;
    st[6] = p->bps;
    st[7] = sbc;
    st[8] = p->block_size;
    st[9] = p->max_blocks_per_seq;
    st[10] = p->block_bytes;
    /* ref pool.rs:1160-1172 */
    float idle = 0.0f;
    if (sbc > 0) {
        uint64_t total = (uint64_t)sbc * SB_BYTES * p->num_layers * 2;
        uint64_t used = in_use * p->block_bytes * p->num_layers * 2;
        if (used < total) idle = (float)(total - used) / (float)total;
    }
    uint32_t ib;
    memcpy(&ib, &idle, 4);
    st[11] = ib;
    st[12] = p->max_physical;
    st[13] = p->region_bytes / SB_BYTES;
}

/* ref pool.rs:1179-1240, metrics.rs:142-162 (all f32) */
void opool_metrics(OPool *p, float *m) {
    uint64_t total_physical = p->pools[0].sb_count * p->bps;
    uint64_t in_use = in_use_count(p);
    uint64_t used = 0, tokens = 0;
    for (size_t s = 0; s < p->nseqs; ++s) { used += p->seqs[s].n; tokens += p->seqs[s].seq_len; }
    uint64_t L2 = p->num_layers * 2;
    uint64_t actual = p->pools[0].sb_count * SB_BYTES * L2;
    uint64_t slots = used * p->block_size;
    m[0] = slots ? (float)((int64_t)slots - (int64_t)tokens) / (float)slots : 0.0f;
    uint64_t ideal = tokens * (p->elem_per_block / p->block_size * L2);
    m[1] = actual ? (float)ideal / (float)actual : 1.0f;
    m[2] = total_physical ? (float)in_use / (float)total_physical : 0.0f;
    uint64_t act_sb = (in_use + p->bps - 1) / p->bps;
    uint64_t act_bytes = act_sb * SB_BYTES * L2;
    m[3] = act_bytes ? 1.0f - (float)ideal / (float)act_bytes : 0.0f;
}

int opool_below_low_watermark(OPool *p, float threshold) {
    uint64_t total = p->pools[0].sb_count * p->bps;
    if (!total) return 0;
    return (float)p->pools[0].nfree / (float)total < threshold;
}

/* ======================================================================
 * Tiering: HBM <-> host swap of whole blocks (all layers' K and V).
 * Restates ref tiering.rs: the eviction policies (:25-545), the swap-slot
 * allocator (:547-643), evict (:937-1406) and restore (:1476-1935), and the
 * pool side (pool.rs:412-454 on_allocate, :478-549 free, :824-936 restore,
 * :983-1002 physical release; ffi.rs:1900-2008 the C entry points).
 * Time stamps are a logical clock (one tick per policy event) instead of
 * Instant::now(): the same order, without ties.
 * Deviation: a victim handle maps to the GPU-resident block that owns it
 * (ref find_block_idx, pool.rs:769-779, takes the first in-use block with
 * that handle, which can be a swapped-out block whose stale handle was
 * reissued).
 * ====================================================================== */

enum { POL_LRU = 0, POL_LFU = 1, POL_FIFO = 2, POL_ARC = 3, POL_SINK = 4 };

typedef struct { Handle h; uint64_t v; } PolEntry;
typedef struct { Handle *a; size_t n, cap; } HList;
typedef struct { uint64_t start, end; } ORange;

struct OTier {
    int policy;
    uint64_t clock;
    PolEntry *map; size_t nmap, cap_map;      /* lru/fifo/sink: time; lfu: count */
    HList t1, t2, b1, b2;                     /* arc (index 0 = MRU end) */
    size_t arc_p, arc_cap;
    ORange *fr; size_t nfr, cap_fr;           /* free swap ranges, sorted by start */
    uint64_t swap_size, per_block;
    size_t max_batch;
};

static int heq(Handle a, Handle b) { return a.sb == b.sb && a.idx == b.idx; }

static PolEntry *map_find(OTier *t, Handle h) {
    for (size_t i = 0; i < t->nmap; ++i) if (heq(t->map[i].h, h)) return &t->map[i];
    return NULL;
}
static void map_set(OTier *t, Handle h, uint64_t v) {
    PolEntry *e = map_find(t, h);
    if (e) { e->v = v; return; }
    t->map = (PolEntry *)grow(t->map, &t->cap_map, t->nmap + 1, sizeof(PolEntry));
    t->map[t->nmap].h = h;
    t->map[t->nmap].v = v;
    t->nmap++;
}
static void map_remove(OTier *t, Handle h) {
    for (size_t i = 0; i < t->nmap; ++i)
        if (heq(t->map[i].h, h)) { t->map[i] = t->map[--t->nmap]; return; }
}

static long hl_find(HList *l, Handle h) {
    for (size_t i = 0; i < l->n; ++i) if (heq(l->a[i], h)) return (long)i;
    return -1;
}
static void hl_insert(HList *l, size_t at, Handle h) {
    l->a = (Handle *)grow(l->a, &l->cap, l->n + 1, sizeof(Handle));
    memmove(l->a + at + 1, l->a + at, (l->n - at) * sizeof(Handle));
    l->a[at] = h;
    l->n++;
}
static void hl_remove_at(HList *l, size_t at) {
    memmove(l->a + at, l->a + at + 1, (l->n - at - 1) * sizeof(Handle));
    l->n--;
}
static void hl_push_bounded(HList *l, Handle h, size_t cap) {
    hl_insert(l, l->n, h);
    while (l->n > cap) hl_remove_at(l, 0);
}

/* ARC replace(): ref tiering.rs:269-296 */
static void arc_replace(OTier *t) {
    if (t->t1.n > 0 && (t->t1.n > t->arc_p || t->t2.n == 0)) {
        Handle v = t->t1.a[t->t1.n - 1];
        t->t1.n--;
        hl_push_bounded(&t->b1, v, t->arc_cap);
    } else if (t->t2.n > 0) {
        Handle v = t->t2.a[t->t2.n - 1];
        t->t2.n--;
        hl_push_bounded(&t->b2, v, t->arc_cap);
    }
}

/* on_allocate: ref tiering.rs:75-77 (lru), :128-130 (lfu), :184-186 (fifo),
 * :299-337 (arc), :492-494 (sink_window) */
static void tier_on_allocate(OTier *t, Handle h) {
    switch (t->policy) {
    case POL_LFU: map_set(t, h, 1); break;
    case POL_ARC: {
        long i1 = hl_find(&t->b1, h);
        if (i1 >= 0) hl_remove_at(&t->b1, (size_t)i1);
        long i2 = hl_find(&t->b2, h);
        if (i2 >= 0) hl_remove_at(&t->b2, (size_t)i2);
        if (i1 >= 0) {
            size_t nb2 = t->b2.n ? t->b2.n : 1, nb1 = t->b1.n ? t->b1.n : 1;
            size_t d = nb2 / nb1; if (d < 1) d = 1;
            t->arc_p = t->arc_p + d < t->arc_cap ? t->arc_p + d : t->arc_cap;
            hl_insert(&t->t2, 0, h);
        } else if (i2 >= 0) {
            size_t nb1 = t->b1.n ? t->b1.n : 1, nb2 = t->b2.n ? t->b2.n : 1;
            size_t d = nb1 / nb2; if (d < 1) d = 1;
            t->arc_p = t->arc_p > d ? t->arc_p - d : 0;
            hl_insert(&t->t2, 0, h);
        } else {
            hl_insert(&t->t1, 0, h);
        }
        while (t->t1.n + t->t2.n > t->arc_cap) arc_replace(t);
        break;
    }
    default: map_set(t, h, ++t->clock); break;
    }
}

/* on_access: ref tiering.rs:94-96, :147-150, :203-206 (fifo: none),
 * :376-393 (arc), :526-528 */
static void tier_on_access(OTier *t, Handle h) {
    switch (t->policy) {
    case POL_FIFO: break;
    case POL_LFU: {
        PolEntry *e = map_find(t, h);
        if (e) e->v++; else map_set(t, h, 1);
        break;
    }
    case POL_ARC: {
        long i = hl_find(&t->t1, h);
        if (i >= 0) { hl_remove_at(&t->t1, (size_t)i); hl_insert(&t->t2, 0, h); break; }
        i = hl_find(&t->t2, h);
        if (i >= 0) { hl_remove_at(&t->t2, (size_t)i); hl_insert(&t->t2, 0, h); }
        break;
    }
    default: map_set(t, h, ++t->clock); break;
    }
}

/* on_evict: ref tiering.rs:98-100, :152-154, :208-210, :395-424, :530-533 */
static void tier_on_evict(OTier *t, Handle h) {
    if (t->policy != POL_ARC) { map_remove(t, h); return; }
    long i = hl_find(&t->t1, h);
    if (i >= 0) {
        hl_remove_at(&t->t1, (size_t)i);
        if (hl_find(&t->b1, h) < 0) hl_push_bounded(&t->b1, h, t->arc_cap);
        return;
    }
    i = hl_find(&t->t2, h);
    if (i >= 0) {
        hl_remove_at(&t->t2, (size_t)i);
        if (hl_find(&t->b2, h) < 0) hl_push_bounded(&t->b2, h, t->arc_cap);
    }
}

/* select_victims: candidates in order, keyed, stable sort ascending,
 * truncated (ref tiering.rs:79-92, :132-145, :188-201, :339-374, :497-524).
 * Untracked candidates are dropped except under ARC (score |T1|+|T2|+1). */
static size_t tier_select(OTier *t, const Handle *cand, size_t n, size_t count, Handle *out) {
    if (n == 0 || count == 0) return 0;
    PolEntry *k = (PolEntry *)malloc(n * sizeof(PolEntry));
    size_t m = 0;
    for (size_t i = 0; i < n; ++i) {
        if (t->policy == POL_ARC) {
            long p1 = -1, p2 = -1;
            for (size_t j = t->t1.n; j-- > 0;) if (heq(t->t1.a[j], cand[i])) { p1 = (long)(t->t1.n - 1 - j); break; }
            if (p1 < 0)
                for (size_t j = t->t2.n; j-- > 0;) if (heq(t->t2.a[j], cand[i])) { p2 = (long)(t->t2.n - 1 - j); break; }
            k[m].h = cand[i];
            k[m].v = p1 >= 0 ? (uint64_t)p1 : p2 >= 0 ? t->t1.n + (uint64_t)p2 : t->t1.n + t->t2.n + 1;
            m++;
        } else {
            PolEntry *e = map_find(t, cand[i]);
            if (!e) continue;
            k[m].h = cand[i];
            k[m].v = e->v;
            m++;
        }
    }
    /* stable insertion sort by key */
    for (size_t i = 1; i < m; ++i) {
        PolEntry x = k[i];
        size_t j = i;
        while (j > 0 && k[j - 1].v > x.v) { k[j] = k[j - 1]; --j; }
        k[j] = x;
    }
    size_t r = m < count ? m : count;
    for (size_t i = 0; i < r; ++i) out[i] = k[i].h;
    free(k);
    return r;
}

/* swap-slot allocator: best fit, shrink from the left; free merges
 * (ref tiering.rs:578-643) */
static int tier_alloc_slot(OTier *t, uint64_t size, uint64_t *off) {
    if (size == 0 || t->nfr == 0) return -1;
    size_t best = (size_t)-1;
    uint64_t best_len = UINT64_MAX;
    for (size_t i = 0; i < t->nfr; ++i) {
        uint64_t len = t->fr[i].end - t->fr[i].start;
        if (len >= size && len < best_len) { best_len = len; best = i; }
    }
    if (best == (size_t)-1) return -1;
    *off = t->fr[best].start;
    if (best_len == size) {
        memmove(t->fr + best, t->fr + best + 1, (t->nfr - best - 1) * sizeof(ORange));
        t->nfr--;
    } else {
        t->fr[best].start += size;
    }
    return 0;
}
static void tier_free_range(OTier *t, uint64_t off, uint64_t size) {
    if (size == 0) return;
    uint64_t end = off + size;
    size_t at = 0;
    while (at < t->nfr && !(t->fr[at].start > off)) ++at;
    int mp = at > 0 && t->fr[at - 1].end == off;
    int mn = at < t->nfr && t->fr[at].start == end;
    if (mp && mn) {
        t->fr[at - 1].end = t->fr[at].end;
        memmove(t->fr + at, t->fr + at + 1, (t->nfr - at - 1) * sizeof(ORange));
        t->nfr--;
    } else if (mp) {
        t->fr[at - 1].end = end;
    } else if (mn) {
        t->fr[at].start = off;
    } else {
        t->fr = (ORange *)grow(t->fr, &t->cap_fr, t->nfr + 1, sizeof(ORange));
        memmove(t->fr + at + 1, t->fr + at, (t->nfr - at) * sizeof(ORange));
        t->fr[at].start = off;
        t->fr[at].end = end;
        t->nfr++;
    }
}
static void tier_free_slot(OTier *t, uint64_t off) { tier_free_range(t, off, t->per_block); }

static void tier_reset_policy(OTier *t, int policy, size_t arc_cap) {
    t->policy = policy;
    t->nmap = 0;
    t->t1.n = t->t2.n = t->b1.n = t->b2.n = 0;
    t->arc_p = 0;
    t->arc_cap = arc_cap ? arc_cap : 1;
}

static void tier_delete(OTier *t) {
    free(t->map); free(t->t1.a); free(t->t2.a); free(t->b1.a); free(t->b2.a); free(t->fr);
    free(t);
}

/* ref ffi.rs:480-497 (defaults), tiering.rs:723-826 (sizing, policy) */
int opool_enable_tiering(OPool *p, int policy, size_t max_blocks, size_t max_batch_blocks) {
    if (p->tier) return -1;
    OTier *t = (OTier *)calloc(1, sizeof(OTier));
    if (!max_blocks) max_blocks = 16384;
    if (!max_batch_blocks) max_batch_blocks = 64;
    t->per_block = (uint64_t)p->num_layers * 2 * p->block_bytes;
    t->swap_size = (uint64_t)max_blocks * t->per_block;
    t->max_batch = max_batch_blocks;
    /* ffi.rs:425-432: only 0/1/2 name a policy, anything else is LRU */
    tier_reset_policy(t, policy == 1 ? POL_LFU : policy == 2 ? POL_FIFO : POL_LRU, max_blocks);
    if (t->swap_size) {
        t->fr = (ORange *)malloc(sizeof(ORange));
        t->fr[0].start = 0;
        t->fr[0].end = t->swap_size;
        t->nfr = 1;
        t->cap_fr = 1;
    }
    p->tier = t;
    return 0;
}

/* ref tiering.rs:851-875: a fresh policy (no history); arc sized from the
 * swap buffer, sink_window (1, 4) */
int opool_set_policy(OPool *p, const char *name) {
    if (!p->tier) return -1;
    OTier *t = p->tier;
    if (!strcmp(name, "lru")) tier_reset_policy(t, POL_LRU, 0);
    else if (!strcmp(name, "lfu")) tier_reset_policy(t, POL_LFU, 0);
    else if (!strcmp(name, "fifo")) tier_reset_policy(t, POL_FIFO, 0);
    else if (!strcmp(name, "arc")) {
        size_t cap = (size_t)(t->swap_size / (t->max_batch ? t->max_batch : 1));
        tier_reset_policy(t, POL_ARC, cap ? cap : 1);
    } else if (!strcmp(name, "sink_window")) tier_reset_policy(t, POL_SINK, 0);
    else return -1;
    return 0;
}

const char *opool_policy_name(OPool *p) {
    static const char *names[] = {"lru", "lfu", "fifo", "arc", "sink_window"};
    return p->tier ? names[p->tier->policy] : "";
}

int opool_location(OPool *p, uint32_t blk) {
    if (blk >= p->nblocks || !p->blocks[blk].in_use) return -1;
    return p->blocks[blk].loc;
}

uint64_t opool_cpu_offset(OPool *p, uint32_t blk) {
    if (blk >= p->nblocks || !p->blocks[blk].in_use || p->blocks[blk].loc != 1) return UINT64_MAX;
    return p->blocks[blk].cpu_off;
}

/* the hint / protect path: on_access of an in-use block's handle
 * (ref ffi.rs:2326-2336, 2404-2421) */
int opool_access(OPool *p, uint32_t blk) {
    if (!p->tier) return 0;
    if (blk >= p->nblocks || !p->blocks[blk].in_use) return -1;
    Handle h = {p->blocks[blk].sb, p->blocks[blk].idx};
    tier_on_access(p->tier, h);
    return 0;
}

/* kcmm_evict_blocks (ref ffi.rs:1900-1945, tiering.rs:1064-1111 and the
 * unbatched / batched paths :1113-1406, which agree on the state they leave):
 * candidates = handles of in-use GPU-resident blocks in id order; victims by
 * the policy; per victim a swap slot (skipped when none is left); then each
 * victim's handle returns to the free list, the block becomes CPU-resident
 * and the policy forgets the handle.  Returns the number evicted; out gets
 * their block ids in victim order. */
uint32_t opool_evict(OPool *p, uint32_t count, uint32_t *out) {
    OTier *t = p->tier;
    if (!t || count == 0) return 0;
    Handle *cand = (Handle *)malloc((p->nblocks + 1) * sizeof(Handle));
    size_t nc = 0;
    for (size_t i = 0; i < p->nblocks; ++i)
        if (p->blocks[i].in_use && p->blocks[i].loc == 0) {
            cand[nc].sb = p->blocks[i].sb;
            cand[nc].idx = p->blocks[i].idx;
            nc++;
        }
    Handle *vic = (Handle *)malloc((nc + 1) * sizeof(Handle));
    size_t nv = tier_select(t, cand, nc, count, vic);
    uint32_t done = 0;
    for (size_t v = 0; v < nv; ++v) {
        uint32_t id = UINT32_MAX;
        for (size_t i = 0; i < p->nblocks; ++i)
            if (p->blocks[i].in_use && p->blocks[i].loc == 0 && p->blocks[i].sb == vic[v].sb &&
                p->blocks[i].idx == vic[v].idx) { id = (uint32_t)i; break; }
        if (id == UINT32_MAX) continue;
        uint64_t off;
        if (tier_alloc_slot(t, t->per_block, &off)) continue;
        p->blocks[id].loc = 3;
        p->blocks[id].cpu_off = off;
        out[done++] = id;
    }
    for (uint32_t j = 0; j < done; ++j) {
        OBlock *b = &p->blocks[out[j]];
        Handle h = {b->sb, b->idx};
        push_handle(p, b->sb, b->idx);
        b->loc = 1;
        tier_on_evict(t, h);
    }
    free(cand);
    free(vic);
    return done;
}

/* restore of one block (ref tiering.rs:1801-1935): new handle by the
 * allocation rule (growth included), block re-pointed, swap slot freed,
 * on_access(new handle). */
static int restore_one(OPool *p, uint32_t id) {
    OTier *t = p->tier;
    OBlock *b = &p->blocks[id];
    if (ensure_capacity(p)) return -1;
    Handle h = {0, 0};
    for (size_t l = 0; l < 2 * p->num_layers; ++l) {
        LayerPool *lp = &p->pools[l];
        Handle x = lp->free[--lp->nfree];
        if (l == 0) h = x;
    }
    b = &p->blocks[id];
    b->sb = h.sb;
    b->idx = h.idx;
    b->va = (uint64_t)h.sb * SB_BYTES + (uint64_t)h.idx * p->block_bytes;
    tier_free_slot(t, b->cpu_off);
    b->loc = 0;
    b->cpu_off = 0;
    tier_on_access(t, h);
    return 0;
}

/* kcmm_restore_evicted_block (ref pool.rs:833-884): 0 and an error when
 * tiering is off, the block is not in use or in transit; a GPU-resident
 * block returns its offset. */
int opool_restore_one(OPool *p, uint32_t blk, uint64_t *va) {
    if (!p->tier || blk >= p->nblocks || !p->blocks[blk].in_use) return -1;
    OBlock *b = &p->blocks[blk];
    if (b->loc == 0) { *va = b->va; return 0; }
    if (b->loc != 1) return -1;
    if (restore_one(p, blk)) return -1;
    *va = p->blocks[blk].va;
    return 0;
}

/* kcmm_restore_evicted_blocks (ref pool.rs:895-936, tiering.rs:1711-1745):
 * every id validated first (out of bounds / not in use / in transit: error,
 * nothing done); GPU-resident ids skipped; a repeated id restores once.
 * Fewer than 8 blocks: one at a time, stopping at the first failure; 8 or
 * more: a failed block stays swapped out and the call reports an error. */
int opool_restore(OPool *p, const uint32_t *ids, uint32_t n) {
    if (!p->tier) return -1;
    for (uint32_t i = 0; i < n; ++i) {
        if (ids[i] >= p->nblocks || !p->blocks[ids[i]].in_use) return -1;
        int l = p->blocks[ids[i]].loc;
        if (l == 3 || l == 4) return -1;
    }
    uint32_t *todo = (uint32_t *)malloc((n + 1) * sizeof(uint32_t));
    uint32_t m = 0;
    for (uint32_t i = 0; i < n; ++i) {
        if (p->blocks[ids[i]].loc != 1) continue;
        int dup = 0;
        for (uint32_t j = 0; j < m; ++j) dup |= todo[j] == ids[i];
        if (!dup) todo[m++] = ids[i];
    }
    int rc = 0;
    for (uint32_t i = 0; i < m; ++i) {
        if (restore_one(p, todo[i])) {
            rc = -1;
            if (m < 8) break;
        }
    }
    free(todo);
    return rc;
}

/* Standalone policy / swap-slot objects, for pinning them to the
 * reference's own unit tests (ref tiering.rs:2106-2740, 3796-4030). */
OTier *otier_new(int policy, size_t arc_cap, uint64_t swap_size, uint64_t per_block) {
    OTier *t = (OTier *)calloc(1, sizeof(OTier));
    tier_reset_policy(t, policy, arc_cap);
    t->per_block = per_block;
    t->swap_size = swap_size;
    if (swap_size) {
        t->fr = (ORange *)malloc(sizeof(ORange));
        t->fr[0].start = 0;
        t->fr[0].end = swap_size;
        t->nfr = 1;
        t->cap_fr = 1;
    }
    return t;
}
void otier_free(OTier *t) { tier_delete(t); }
void otier_event(OTier *t, int kind, uint32_t sb, uint32_t idx) {
    Handle h = {sb, idx};
    if (kind == 0) tier_on_allocate(t, h);
    else if (kind == 1) tier_on_access(t, h);
    else tier_on_evict(t, h);
}
size_t otier_select(OTier *t, const uint32_t *hs, size_t n, size_t count, uint32_t *out) {
    Handle *c = (Handle *)malloc((n + 1) * sizeof(Handle));
    Handle *o = (Handle *)malloc((n + 1) * sizeof(Handle));
    for (size_t i = 0; i < n; ++i) { c[i].sb = hs[2 * i]; c[i].idx = hs[2 * i + 1]; }
    size_t r = tier_select(t, c, n, count, o);
    for (size_t i = 0; i < r; ++i) { out[2 * i] = o[i].sb; out[2 * i + 1] = o[i].idx; }
    free(c);
    free(o);
    return r;
}
int otier_slot_alloc(OTier *t, uint64_t size, uint64_t *off) { return tier_alloc_slot(t, size, off); }
void otier_slot_free(OTier *t, uint64_t off, uint64_t size) { tier_free_range(t, off, size); }
size_t otier_ranges(OTier *t, uint64_t *out, size_t max) {
    size_t n = t->nfr < max ? t->nfr : max;
    for (size_t i = 0; i < n; ++i) { out[2 * i] = t->fr[i].start; out[2 * i + 1] = t->fr[i].end; }
    return n;
}
size_t otier_arc_list(OTier *t, int which, uint32_t *out, size_t max) {
    HList *l = which == 0 ? &t->t1 : which == 1 ? &t->t2 : which == 2 ? &t->b1 : &t->b2;
    size_t n = l->n < max ? l->n : max;
    for (size_t i = 0; i < n; ++i) { out[2 * i] = l->a[i].sb; out[2 * i + 1] = l->a[i].idx; }
    return n;
}
size_t otier_arc_p(OTier *t) { return t->arc_p; }

/* ======================================================================
 * KV write
 * ====================================================================== */

/* fp8 page write (this build's fp8 contract, stated in include/kcmm_mi355x.h
 * at kcmm_pool_create_typed; the reference has no fp8 pages).  The rows one
 * call writes into a page act as one set: row_of[slot] is the source row the
 * call writes at that slot (its last one for the slot), or -1.  Per kv head:
 * amax over the written rows; writing slot 0, or a footer scale that is not a
 * finite positive number, starts the page (scale amax/448, 1 if 0, unwritten
 * slots left as they are); otherwise the scale grows to amax/448 when
 * amax > 448*old and every unwritten slot is re-encoded from old to new.
 * Written rows are stored as e4m3(x/scale). */
static void fp8_write_page(uint8_t *page, const int32_t *row_of, uint32_t bs,
                           const uint16_t *src, uint32_t kv_heads, uint32_t D,
                           uint32_t row_bytes, uint32_t data_bytes) {
    for (uint32_t g = 0; g < kv_heads; ++g) {
        float amax = 0.0f;
        for (uint32_t u = 0; u < bs; ++u) {
            if (row_of[u] < 0) continue;
            const uint16_t *x = src + ((uint64_t)row_of[u] * kv_heads + g) * D;
            for (uint32_t d = 0; d < D; ++d) {
                float a = fabsf(oracle_bf16_to_f32(x[d]));
                if (a > amax) amax = a;
            }
        }
        uint8_t *sp = page + data_bytes + g * 4;
        float old;
        memcpy(&old, sp, 4);
        const int fresh = row_of[0] >= 0 || !(old > 0.0f && old <= 3.40282347e38f);
        float scale;
        if (fresh) {
            scale = amax > 0.0f ? amax / 448.0f : 1.0f;
        } else {
            scale = old;
            if (amax > 448.0f * old) {
                scale = amax / 448.0f;
                for (uint32_t u = 0; u < bs; ++u) {
                    if (row_of[u] >= 0) continue;
                    uint8_t *row = page + (uint64_t)u * row_bytes + g * D;
                    for (uint32_t d = 0; d < D; ++d) {
                        float y = oracle_e4m3_to_f32(row[d]) * old;
                        row[d] = oracle_f32_to_e4m3(y / scale);
                    }
                }
            }
        }
        for (uint32_t u = 0; u < bs; ++u) {
            if (row_of[u] < 0) continue;
            const uint16_t *x = src + ((uint64_t)row_of[u] * kv_heads + g) * D;
            uint8_t *row = page + (uint64_t)u * row_bytes + g * D;
            for (uint32_t d = 0; d < D; ++d) row[d] = oracle_f32_to_e4m3(oracle_bf16_to_f32(x[d]) / scale);
        }
        memcpy(sp, &scale, 4);
    }
}

/* ref pool.rs:1073-1091: dst = region + va_offset + off*step*2, one row copy
 * per row in call order (a repeated slot keeps the last row). */
static void copy_row(uint8_t *k_region, uint8_t *v_region, const uint8_t *k_src,
                     const uint8_t *v_src, uint64_t page, uint32_t slot, uint32_t src_row,
                     uint32_t row_bytes) {
    uint64_t dst = page + (uint64_t)slot * row_bytes;
    memcpy(k_region + dst, k_src + (uint64_t)src_row * row_bytes, row_bytes);
    memcpy(v_region + dst, v_src + (uint64_t)src_row * row_bytes, row_bytes);
}

int oracle_kv_write_rows(int dtype, uint8_t *k_region, uint8_t *v_region, const uint8_t *k_src,
                         const uint8_t *v_src, const uint64_t *page_offsets,
                         const uint32_t *slots, const uint32_t *src_rows, uint32_t n,
                         uint32_t kv_heads, uint32_t head_dim, uint32_t row_bytes,
                         uint32_t data_bytes) {
    if (dtype != 2) {
        for (uint32_t i = 0; i < n; ++i)
            copy_row(k_region, v_region, k_src, v_src, page_offsets[i], slots[i], src_rows[i],
                     row_bytes);
        return 0;
    }
    const uint32_t bs = data_bytes / row_bytes;
    int32_t *row_of = (int32_t *)malloc(bs * sizeof(int32_t));
    uint8_t *done = (uint8_t *)calloc(n ? n : 1, 1);
    for (uint32_t i = 0; i < n; ++i) {
        if (done[i]) continue;
        for (uint32_t u = 0; u < bs; ++u) row_of[u] = -1;
        for (uint32_t j = i; j < n; ++j)
            if (page_offsets[j] == page_offsets[i]) {
                row_of[slots[j]] = (int32_t)src_rows[j];
                done[j] = 1;
            }
        fp8_write_page(k_region + page_offsets[i], row_of, bs, (const uint16_t *)k_src, kv_heads,
                       head_dim, row_bytes, data_bytes);
        fp8_write_page(v_region + page_offsets[i], row_of, bs, (const uint16_t *)v_src, kv_heads,
                       head_dim, row_bytes, data_bytes);
    }
    free(done);
    free(row_of);
    return 0;
}

/* ref kcmm_vllm_kv_write.cu:8-66: padding skipped, id >= len -> status 1,
 * inactive id -> status 2, first error wins. */
int oracle_kv_write_device_slots(int dtype, uint8_t *k_region, uint8_t *v_region,
                                 const uint8_t *k_src, const uint8_t *v_src, const int64_t *slots,
                                 uint32_t batch, const uint64_t *offsets_f16,
                                 const uint8_t *valid, uint32_t offsets_len, uint32_t block_size,
                                 uint32_t kv_heads, uint32_t head_dim, uint32_t row_bytes,
                                 uint32_t data_bytes, int32_t *status) {
    int32_t *row_of = (int32_t *)malloc(block_size * sizeof(int32_t));
    uint8_t *done = (uint8_t *)calloc(batch ? batch : 1, 1);
    for (uint32_t r = 0; r < batch; ++r) {
        int64_t slot = slots[r];
        if (slot < 0 || done[r]) continue;
        int64_t id = slot / block_size;
        if (id >= (int64_t)offsets_len) { if (status && *status == 0) *status = 1; continue; }
        if (valid && valid[id] == 0) { if (status && *status == 0) *status = 2; continue; }
        const uint64_t page = offsets_f16[id] * 2;
        if (dtype != 2) {
            copy_row(k_region, v_region, k_src, v_src, page, (uint32_t)(slot % block_size), r,
                     row_bytes);
            continue;
        }
        /* fp8: all rows of this page in the call, as one set */
        for (uint32_t u = 0; u < block_size; ++u) row_of[u] = -1;
        for (uint32_t j = r; j < batch; ++j)
            if (slots[j] >= 0 && slots[j] / block_size == id) {
                row_of[slots[j] % block_size] = (int32_t)j;
                done[j] = 1;
            }
        fp8_write_page(k_region + page, row_of, block_size, (const uint16_t *)k_src, kv_heads,
                       head_dim, row_bytes, data_bytes);
        fp8_write_page(v_region + page, row_of, block_size, (const uint16_t *)v_src, kv_heads,
                       head_dim, row_bytes, data_bytes);
    }
    free(done);
    free(row_of);
    return 0;
}

void oracle_copy_pages(uint8_t *const *regions, uint32_t n_regions, const uint64_t *pairs,
                       uint32_t n_pairs, uint32_t block_bytes) {
    for (uint32_t p = 0; p < n_pairs; ++p)
        for (uint32_t r = 0; r < n_regions; ++r)
            memmove(regions[r] + pairs[2 * p + 1], regions[r] + pairs[2 * p], block_bytes);
}

/* ======================================================================
 * Paged decode attention
 * ====================================================================== */

static double q_elem(int dtype, const void *q, size_t i) {
    if (dtype == 0) return oracle_f16_to_f32(((const uint16_t *)q)[i]);
    if (dtype == 3) return ((const float *)q)[i];
    return oracle_bf16_to_f32(((const uint16_t *)q)[i]);  /* bf16 and fp8 pools */
}

static double kv_elem(int dtype, const uint8_t *page, uint64_t off, uint32_t d,
                      uint32_t data_bytes, uint32_t kvh) {
    switch (dtype) {
        case 0: { uint16_t h; memcpy(&h, page + off + 2 * d, 2); return oracle_f16_to_f32(h); }
        case 1: { uint16_t h; memcpy(&h, page + off + 2 * d, 2); return oracle_bf16_to_f32(h); }
        case 2: {
            float s;
            memcpy(&s, page + data_bytes + 4 * kvh, 4);
            return (double)oracle_e4m3_to_f32(page[off + d]) * (double)s;
        }
        default: { float f; memcpy(&f, page + off + 4 * d, 4); return f; }
    }
}

int oracle_attn_decode_f64(int dtype, const void *q, double *out, const uint8_t *k_region,
                           const uint8_t *v_region, const int32_t *block_tables,
                           const int32_t *seq_lens, const uint64_t *offsets_f16, uint32_t batch,
                           uint32_t hq, uint32_t hkv, uint32_t D, uint32_t bs, uint32_t mbps,
                           uint32_t row_bytes, uint32_t data_bytes, double scale) {
    size_t es = esize_of(dtype);
    #pragma omp parallel for schedule(dynamic)
    for (long long task = 0; task < (long long)batch * hq; ++task) {
        uint32_t b = (uint32_t)(task / hq), h = (uint32_t)(task % hq);
        uint32_t kvh = h * hkv / hq;                       /* ref kcmm_vllm_paged_attn.cu:40 */
        int64_t L = seq_lens[b];
        if (L > (int64_t)mbps * bs) L = (int64_t)mbps * bs;
        double *o = out + ((size_t)b * hq + h) * D;
        if (L <= 0) { for (uint32_t d = 0; d < D; ++d) o[d] = 0.0; continue; }
        double *s = (double *)malloc((size_t)L * sizeof(double));
        const size_t qi = ((size_t)b * hq + h) * D;
        double mx = -INFINITY;
        for (int64_t t = 0; t < L; ++t) {
            int32_t blk = block_tables[(size_t)b * mbps + t / bs];
            uint64_t page = offsets_f16[blk] * 2;
            uint64_t off = (uint64_t)(t % bs) * row_bytes + (uint64_t)kvh * D * es;
            double acc = 0.0;
            for (uint32_t d = 0; d < D; ++d)
                acc += q_elem(dtype, q, qi + d) * kv_elem(dtype, k_region + page, off, d, data_bytes, kvh);
            s[t] = acc * scale;
            if (s[t] > mx) mx = s[t];
        }
        double z = 0.0;
        for (int64_t t = 0; t < L; ++t) { s[t] = exp(s[t] - mx); z += s[t]; }
        for (uint32_t d = 0; d < D; ++d) o[d] = 0.0;
        for (int64_t t = 0; t < L; ++t) {
            int32_t blk = block_tables[(size_t)b * mbps + t / bs];
            uint64_t page = offsets_f16[blk] * 2;
            uint64_t off = (uint64_t)(t % bs) * row_bytes + (uint64_t)kvh * D * es;
            double w = s[t] / z;
            for (uint32_t d = 0; d < D; ++d)
                o[d] += w * kv_elem(dtype, v_region + page, off, d, data_bytes, kvh);
        }
        free(s);
    }
    return 0;
}

/* Causal chunked-prefill attention over paged K/V.  The reference has no
 * chunked prefill (prefill is one token per decode step, ref
 * transformer.rs:50-65); this is the north star's extension, restated as the
 * textbook definition: sequence b holds seq_lens[b] tokens in the cache, the
 * last len_b = qsl[b+1] - qsl[b] of which are this chunk's queries (their K/V
 * already appended).  Query i of b sits at position p = seq_lens[b] - len_b + i
 * and attends to keys 0..p; GQA head map as in decode.  Two-pass softmax in
 * fp64.  q/out rows are [qsl[b] + i][hq][D]. */
int oracle_attn_prefill_f64(int dtype, const void *q, double *out, const uint8_t *k_region,
                            const uint8_t *v_region, const int32_t *block_tables,
                            const int32_t *seq_lens, const int32_t *qsl,
                            const uint64_t *offsets_f16, uint32_t batch, uint32_t hq,
                            uint32_t hkv, uint32_t D, uint32_t bs, uint32_t mbps,
                            uint32_t row_bytes, uint32_t data_bytes, double scale) {
    size_t es = esize_of(dtype);
    const int64_t total = qsl[batch];
    #pragma omp parallel for schedule(dynamic)
    for (long long task = 0; task < (long long)total * hq; ++task) {
        const int64_t row = task / hq;
        const uint32_t h = (uint32_t)(task % hq);
        uint32_t b = 0;
        while ((int64_t)qsl[b + 1] <= row) ++b;
        const int64_t len = qsl[b + 1] - qsl[b];
        const int64_t pos = (int64_t)seq_lens[b] - len + (row - qsl[b]);
        const uint32_t kvh = h * hkv / hq;
        double *o = out + ((size_t)row * hq + h) * D;
        for (uint32_t d = 0; d < D; ++d) o[d] = 0.0;
        if (pos < 0 || pos >= (int64_t)mbps * bs) continue;
        const int64_t L = pos + 1;
        double *s = (double *)malloc((size_t)L * sizeof(double));
        const size_t qi = ((size_t)row * hq + h) * D;
        double mx = -INFINITY;
        for (int64_t t = 0; t < L; ++t) {
            int32_t blk = block_tables[(size_t)b * mbps + t / bs];
            uint64_t page = offsets_f16[blk] * 2;
            uint64_t off = (uint64_t)(t % bs) * row_bytes + (uint64_t)kvh * D * es;
            double acc = 0.0;
            for (uint32_t d = 0; d < D; ++d)
                acc += q_elem(dtype, q, qi + d) * kv_elem(dtype, k_region + page, off, d, data_bytes, kvh);
            s[t] = acc * scale;
            if (s[t] > mx) mx = s[t];
        }
        double z = 0.0;
        for (int64_t t = 0; t < L; ++t) { s[t] = exp(s[t] - mx); z += s[t]; }
        for (int64_t t = 0; t < L; ++t) {
            int32_t blk = block_tables[(size_t)b * mbps + t / bs];
            uint64_t page = offsets_f16[blk] * 2;
            uint64_t off = (uint64_t)(t % bs) * row_bytes + (uint64_t)kvh * D * es;
            double w = s[t] / z;
            for (uint32_t d = 0; d < D; ++d)
                o[d] += w * kv_elem(dtype, v_region + page, off, d, data_bytes, kvh);
        }
        free(s);
    }
    return 0;
}

/* The reference kernel's loop (ref kcmm_vllm_paged_attn.cu:38-101): m starts
 * at -1e30, per token dot*scale, m=max, e=exp(dot-m), corr=exp(old_m-m),
 * s=s*corr+e, acc=acc*corr+e*v; out=acc/s.  16-bit K/V only. */
int oracle_attn_decode_ref_f32(int dtype, const void *q, float *out, const uint8_t *k_region,
                               const uint8_t *v_region, const int32_t *block_tables,
                               const int32_t *seq_lens, const uint64_t *offsets_f16,
                               uint32_t batch, uint32_t hq, uint32_t hkv, uint32_t D,
                               uint32_t bs, uint32_t mbps, uint32_t row_bytes, float scale,
                               int threads) {
    if (D > 256 || (dtype != 0 && dtype != 1 && dtype != 3)) return -1;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#endif
    #pragma omp parallel for schedule(dynamic, 4)
    for (long long task = 0; task < (long long)batch * hq; ++task) {
        uint32_t b = (uint32_t)(task / hq), h = (uint32_t)(task % hq);
        uint32_t kvh = h * hkv / hq;
        int32_t L = seq_lens[b];
        float *o = out + ((size_t)b * hq + h) * D;
        if (L <= 0) { for (uint32_t d = 0; d < D; ++d) o[d] = 0.0f; continue; }
        float qv[256], acc[256];
        for (uint32_t d = 0; d < D; ++d) {
            if (dtype == 3) {
                qv[d] = ((const float *)q)[((size_t)b * hq + h) * D + d];
            } else {
                uint16_t x = ((const uint16_t *)q)[((size_t)b * hq + h) * D + d];
                qv[d] = dtype == 0 ? oracle_f16_to_f32(x) : oracle_bf16_to_f32(x);
            }
            acc[d] = 0.0f;
        }
        const uint32_t es = dtype == 3 ? 4 : 2;
        float m = -1e30f, s = 0.0f;
        for (int32_t pos = 0; pos < L; ++pos) {
            int32_t blk = block_tables[(size_t)b * mbps + pos / bs];
            uint64_t base = offsets_f16[blk] * 2 + (uint64_t)(pos % bs) * row_bytes +
                            (uint64_t)kvh * D * es;
            const uint16_t *kr = (const uint16_t *)(k_region + base);
            const uint16_t *vr = (const uint16_t *)(v_region + base);
            const float *kf = (const float *)(k_region + base);
            const float *vf = (const float *)(v_region + base);
            float dot = 0.0f;
            if (dtype == 3) {
                for (uint32_t d = 0; d < D; ++d) dot += qv[d] * kf[d];
            } else if (dtype == 1) {
                for (uint32_t d = 0; d < D; ++d) dot += qv[d] * u2f((uint32_t)kr[d] << 16);
            } else {
                for (uint32_t d = 0; d < D; ++d) dot += qv[d] * oracle_f16_to_f32(kr[d]);
            }
            dot *= scale;
            float old_m = m;
            m = fmaxf(m, dot);
            float e = expf(dot - m);
            float corr = expf(old_m - m);
            s = s * corr + e;
            if (dtype == 3) {
                for (uint32_t d = 0; d < D; ++d) acc[d] = acc[d] * corr + e * vf[d];
            } else if (dtype == 1) {
                for (uint32_t d = 0; d < D; ++d) acc[d] = acc[d] * corr + e * u2f((uint32_t)vr[d] << 16);
            } else {
                for (uint32_t d = 0; d < D; ++d) acc[d] = acc[d] * corr + e * oracle_f16_to_f32(vr[d]);
            }
        }
        float inv = 1.0f / s;
        for (uint32_t d = 0; d < D; ++d) o[d] = acc[d] * inv;
    }
    return 0;
}

/* ======================================================================
 * GEMM: Y = X W^T (the HF Linear product ref llama_transformer.rs:115-120
 * intends; ref runtime.rs:17-41 delegates it to cuBLAS).
 * ====================================================================== */
/* Y = X (W8 diag(s))^T with e4m3 weights and an fp32 scale per weight row:
 * the fp64 sum of x * decode(w8) times the row's scale. */
void oracle_gemm_fp8w_f64(const uint16_t *x, const uint8_t *w8, const float *s, double *y,
                          uint32_t m, uint32_t n, uint32_t k) {
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)m; ++i) {
        double *xr = (double *)malloc(k * sizeof(double));
        for (uint32_t t = 0; t < k; ++t) xr[t] = oracle_bf16_to_f32(x[(size_t)i * k + t]);
        for (uint32_t j = 0; j < n; ++j) {
            const uint8_t *wr = w8 + (size_t)j * k;
            double acc = 0.0;
            for (uint32_t t = 0; t < k; ++t) acc += xr[t] * (double)oracle_e4m3_to_f32(wr[t]);
            y[(size_t)i * n + j] = acc * (double)s[j];
        }
        free(xr);
    }
}

void oracle_gemm_bf16_f64(const uint16_t *x, const uint16_t *w, double *y, uint32_t m,
                          uint32_t n, uint32_t k) {
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)m; ++i) {
        double *xr = (double *)malloc(k * sizeof(double));
        for (uint32_t t = 0; t < k; ++t) xr[t] = oracle_bf16_to_f32(x[(size_t)i * k + t]);
        for (uint32_t j = 0; j < n; ++j) {
            const uint16_t *wr = w + (size_t)j * k;
            double acc = 0.0;
            for (uint32_t t = 0; t < k; ++t) acc += xr[t] * (double)oracle_bf16_to_f32(wr[t]);
            y[(size_t)i * n + j] = acc;
        }
        free(xr);
    }
}
