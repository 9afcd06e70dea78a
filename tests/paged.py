"""Test-side construction of paged K/V regions from dense per-sequence
tensors (numpy only), independent of the product's workload builder."""
from __future__ import annotations

import numpy as np

import oracle as O


def layout(batch, ctx, kv_heads, head_dim, block_size, dtype, seed, shuffle=True,
           mbps=None):
    """Dense K/V per sequence, scattered over a shuffled set of page slots.

    Returns dict with block_tables [B][mbps] int32, offsets_f16 uint64 (one
    entry per block id; id i lives at byte i*block_bytes), host regions
    k_region / v_region, the dense float K/V actually stored (after the dtype
    round trip) and geometry."""
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, dtype=np.int64)
    esize = 1 if dtype == O.FP8 else (4 if dtype == O.F32 else 2)
    row_bytes = kv_heads * head_dim * esize
    data_bytes = row_bytes * block_size
    block_bytes = ((data_bytes + 4 * kv_heads + 255) // 256) * 256 if dtype == O.FP8 else data_bytes
    pages = [max(1, -(-int(L) // block_size)) for L in ctx]
    n_ids = sum(pages) + 3                      # a few ids no sequence uses
    mbps = mbps or max(pages)
    perm = rng.permutation(n_ids)                # drawn either way: same K/V for both layouts
    ids = perm if shuffle else np.arange(n_ids)
    bt = np.zeros((batch, mbps), np.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = ids[pos:pos + n]
        pos += n
    offsets = (np.arange(n_ids, dtype=np.uint64) * block_bytes) // 2
    kreg = np.zeros(n_ids * block_bytes, np.uint8)
    vreg = np.zeros_like(kreg)
    dense_k, dense_v = [], []
    for b in range(batch):
        n = pages[b]
        for reg, dense in ((kreg, dense_k), (vreg, dense_v)):
            x = rng.standard_normal((n * block_size, kv_heads, head_dim)).astype(np.float32)
            stored = np.zeros(x.shape, dtype=np.float64)
            for pi in range(n):
                page = int(bt[b, pi]) * block_bytes
                blk = x[pi * block_size:(pi + 1) * block_size]
                if dtype == O.FP8:
                    amax = np.abs(blk).max(axis=(0, 2))
                    sc = np.where(amax > 0, amax / np.float32(448), np.float32(1)).astype(np.float32)
                    enc = O.encode(O.FP8, blk / sc[None, :, None])
                    reg[page:page + data_bytes] = enc.reshape(-1)
                    reg[page + data_bytes:page + data_bytes + 4 * kv_heads] = sc.view(np.uint8)
                    stored[pi * block_size:(pi + 1) * block_size] = \
                        O.decode(O.FP8, enc).astype(np.float64) * sc[None, :, None]
                else:
                    enc = O.encode(dtype, blk)
                    reg[page:page + data_bytes] = enc.view(np.uint8).reshape(-1)
                    stored[pi * block_size:(pi + 1) * block_size] = O.decode(dtype, enc)
            dense.append(stored[: max(int(ctx[b]), 0)])
    return dict(block_tables=bt, offsets=offsets, k_region=kreg, v_region=vreg, dense_k=dense_k,
                dense_v=dense_v, row_bytes=row_bytes, data_bytes=data_bytes,
                block_bytes=block_bytes, seq_lens=ctx.astype(np.int32))


def dense_reference(q, dense_k, dense_v, num_q_heads, kv_heads, scale):
    """softmax(scale q K^T) V per (b, h) with numpy in float64 (two-pass)."""
    B = len(dense_k)
    D = q.shape[-1]
    out = np.zeros((B, num_q_heads, D))
    for b in range(B):
        K, V = dense_k[b].astype(np.float64), dense_v[b].astype(np.float64)
        if K.shape[0] == 0:
            continue
        for h in range(num_q_heads):
            g = h * kv_heads // num_q_heads
            s = K[:, g, :] @ q[b, h].astype(np.float64) * scale
            w = np.exp(s - s.max())
            out[b, h] = (w / w.sum()) @ V[:, g, :]
    return out
