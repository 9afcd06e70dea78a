"""Synthetic decode-step workloads built through the KCMM C ABI.

Used by bench.py, __graft_entry__.smoke() and the GPU tests to lay out a
paged KV cache the way a serving engine would: pages are allocated from the
pool, shuffled with a seeded permutation, handed to sequences as block
tables, and filled with N(0,1) values.  PRNG: numpy PCG64
(np.random.default_rng(seed)); fixed seeds per configuration.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from .bindings import (KV_BF16, KV_F16, KV_F32, KV_FP8, KcmmLibrary, KcmmPool, make_config,
                       memcpy_htod)

SB = 2 * 1024 * 1024


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (vectorised)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def encode16(dtype: int, x: np.ndarray) -> np.ndarray:
    """Element bits of a 16-bit pool type (or the fp32 values of an fp32 pool)."""
    if dtype == KV_F32:
        return np.ascontiguousarray(x, dtype=np.float32)
    return f32_to_f16_bits(x) if dtype == KV_F16 else f32_to_bf16_bits(x)


def elem_bytes(dtype: int) -> int:
    """Bytes of one K/V element of a pool type."""
    return {KV_FP8: 1, KV_F32: 4}.get(dtype, 2)


def io_dtype(dtype: int) -> int:
    """Element type of q/out rows: f16 for f16 pools, fp32 for fp32 pools, bf16 otherwise."""
    return dtype if dtype in (KV_F16, KV_F32) else KV_BF16


def torch_io_dtype(dtype: int):
    return {KV_F16: torch.float16, KV_F32: torch.float32}.get(dtype, torch.bfloat16)


def encode_fp8_page(blk: np.ndarray):
    """A whole page [bs][Hkv][D] at once (prefill-style): scale per kv head =
    amax/448 (1 for an all-zero head), e4m3fn RNE via torch's cast."""
    amax = np.abs(blk).max(axis=(0, 2)).astype(np.float32)
    scales = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    y = torch.from_numpy((blk / scales[None, :, None]).astype(np.float32))
    data = y.to(torch.float8_e4m3fn).view(torch.uint8).numpy().reshape(-1)
    return data, scales


@dataclass
class DecodeCase:
    lib: KcmmLibrary
    pool: KcmmPool
    dtype: int
    batch: int
    num_q_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    num_layers: int
    seq_lens: np.ndarray            # int32 [B], tokens attended (incl. the appended one)
    block_tables: np.ndarray        # int32 [B][mbps]
    offsets_f16: np.ndarray         # uint64 [n_ids]
    q_bits: np.ndarray              # uint16 [B][Hq][D]
    k_mirror: list = field(default_factory=list)   # per layer host copy of the K region
    v_mirror: list = field(default_factory=list)
    dev: dict = field(default_factory=dict)        # torch device tensors

    @property
    def mbps(self) -> int:
        return self.block_tables.shape[1]

    @property
    def geometry(self) -> dict:
        st = self.pool.stats()
        elem = elem_bytes(self.dtype)
        row_bytes = self.kv_heads * self.head_dim * elem
        return dict(block_bytes=st["block_bytes"], row_bytes=row_bytes,
                    data_bytes=row_bytes * self.block_size,
                    mapped_bytes=st["superblock_count"] * SB)

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes one decode attention step reads (one layer)."""
        elem = elem_bytes(self.dtype)
        return int(self.seq_lens.astype(np.int64).sum()) * 2 * self.kv_heads * self.head_dim * elem

    def run_attention(self, layer: int = 0, stream_ptr: int | None = None, scale=None) -> None:
        scale = 1.0 / math.sqrt(self.head_dim) if scale is None else scale
        d = self.dev
        self.pool.paged_attn_decode(
            layer_idx=layer, query_ptr=d["q"].data_ptr(), out_ptr=d["out"].data_ptr(),
            block_tables_ptr=d["bt"].data_ptr(), seq_lens_ptr=d["sl"].data_ptr(),
            block_offsets_f16_ptr=d["offs"].data_ptr(), batch=self.batch,
            num_q_heads=self.num_q_heads, kv_heads=self.kv_heads, head_dim=self.head_dim,
            block_size=self.block_size, max_blocks_per_seq=self.mbps, scale=scale,
            stream_ptr=stream_ptr)

    def out_bits(self) -> np.ndarray:
        """Output element bits (fp32 values for an fp32 pool)."""
        if self.dtype == KV_F32:
            return self.dev["out"].cpu().numpy()
        return self.dev["out"].cpu().view(torch.int16).numpy().view(np.uint16)


def _fill_pages_host(case: DecodeCase, rng: np.random.Generator, layer_tokens) -> None:
    """Write N(0,1) K/V for every attended token into host mirrors of the
    regions, then upload the mapped part of each region."""
    g = case.geometry
    hk, d, bs = case.kv_heads, case.head_dim, case.block_size
    for layer in range(case.num_layers):
        mk = np.zeros(g["mapped_bytes"], dtype=np.uint8)
        mv = np.zeros(g["mapped_bytes"], dtype=np.uint8)
        for b in range(case.batch):
            L = int(layer_tokens[b])
            if L <= 0:
                continue
            n_pages = -(-L // bs)
            for which, mirror in ((0, mk), (1, mv)):
                x = rng.standard_normal((n_pages * bs, hk, d)).astype(np.float32)
                x[L:] = 0.0
                for pi in range(n_pages):
                    page = int(case.offsets_f16[case.block_tables[b, pi]]) * 2
                    blk = x[pi * bs:(pi + 1) * bs]
                    if case.dtype == KV_FP8:
                        data, scales = encode_fp8_page(blk)
                        mirror[page:page + data.size] = data
                        mirror[page + g["data_bytes"]:page + g["data_bytes"] + 4 * hk] = \
                            scales.view(np.uint8)
                    else:
                        data = encode16(case.dtype, blk).view(np.uint8).reshape(-1)
                        mirror[page:page + data.size] = data
        memcpy_htod(case.pool.va_k(layer), mk)
        memcpy_htod(case.pool.va_v(layer), mv)
        case.k_mirror.append(mk)
        case.v_mirror.append(mv)


def build_decode_case(lib: KcmmLibrary, *, batch: int, num_q_heads: int, kv_heads: int,
                      head_dim: int, block_size: int, ctx_lens, dtype: int = KV_BF16,
                      num_layers: int = 1, seed: int = 0, host_mirror: bool = True,
                      extra_seq_len: int = 0, device: str = "cuda",
                      shuffle: bool = True, tiering: bool = False) -> DecodeCase:
    """Allocate pages for `ctx_lens` tokens per sequence (+ `extra_seq_len`
    page headroom), shuffle them over the pool, fill them and upload q."""
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx_lens, dtype=np.int64)
    max_len = int(max(1, ctx.max() + extra_seq_len))
    cfg = make_config(num_layers=num_layers, kv_heads=kv_heads, head_dim=head_dim,
                      max_batch=batch, max_seq_len=max_len, block_size=block_size,
                      tiering=tiering)
    pool = lib.create_pool(cfg, dtype)
    pages = [max(1, -(-int(L + extra_seq_len) // block_size)) for L in ctx]
    ids = []
    total = sum(pages)
    for start in range(0, total, 4096):
        ids += pool.alloc_blocks(min(4096, total - start))
    perm = rng.permutation(np.asarray(ids, dtype=np.int64))
    if not shuffle:   # pages of a sequence contiguous in allocation order
        perm = np.asarray(ids, dtype=np.int64)
    mbps = -(-max_len // block_size)
    bt = np.zeros((batch, mbps), dtype=np.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
        s = pool.register_sequence(bt[b, :n].tolist())
        pool.update_seq_len(s, int(ctx[b]))
    offs = np.asarray(pool.all_block_offsets_f16(), dtype=np.uint64)
    qdt = io_dtype(dtype)   # fp8 pools take bf16 queries
    q = encode16(qdt, rng.standard_normal((batch, num_q_heads, head_dim)).astype(np.float32))
    case = DecodeCase(lib=lib, pool=pool, dtype=dtype, batch=batch, num_q_heads=num_q_heads,
                      kv_heads=kv_heads, head_dim=head_dim, block_size=block_size,
                      num_layers=num_layers, seq_lens=ctx.astype(np.int32), block_tables=bt,
                      offsets_f16=offs, q_bits=q)
    if host_mirror:
        _fill_pages_host(case, rng, ctx)
    else:
        fill_regions_on_device(case, seed)
    tdt = torch_io_dtype(dtype)
    qt = torch.from_numpy(q.copy()) if dtype == KV_F32 else torch.from_numpy(q.view(np.int16)).view(tdt)
    case.dev = {
        "q": qt.to(device),
        "out": torch.zeros((batch, num_q_heads, head_dim), dtype=tdt, device=device),
        "bt": torch.from_numpy(bt).to(device),
        "sl": torch.from_numpy(case.seq_lens.copy()).to(device),
        "offs": torch.from_numpy(offs.view(np.int64)).to(device),
    }
    return case


def _region_copy(dst: int, src, nbytes: int) -> None:
    import ctypes
    from .bindings import hip
    h = hip()
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    rc = h.hipMemcpy(ctypes.c_void_p(dst), ctypes.c_void_p(src.data_ptr()), nbytes, 3)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy D2D failed ({rc})")


def fill_regions_on_device(case: DecodeCase, seed: int) -> None:
    """Fill the regions on the GPU (torch), for workloads too large for a host
    mirror: every mapped byte of a 16-bit pool with N(0,1) values; every
    allocated page of an fp8 pool with N(0,1) rows quantized per (page, kv
    head) exactly as encode_fp8_page does (scale = amax/448, e4m3fn RNE),
    scales in the page footer."""
    g = case.geometry
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    if case.dtype == KV_FP8:
        _fill_fp8_on_device(case, gen)
        torch.cuda.synchronize()
        return
    es = elem_bytes(case.dtype)
    n = g["mapped_bytes"] // es
    tdt = torch_io_dtype(case.dtype)
    for layer in range(case.num_layers):
        for base in (case.pool.va_k(layer), case.pool.va_v(layer)):
            chunk = 64 << 20
            for off in range(0, n, chunk):
                m = min(chunk, n - off)
                t = torch.randn(m, generator=gen, device="cuda", dtype=torch.float32).to(tdt)
                _region_copy(base + es * off, t, es * m)
    torch.cuda.synchronize()


def _fill_fp8_on_device(case: DecodeCase, gen) -> None:
    g = case.geometry
    bb, data_bytes = g["block_bytes"], g["data_bytes"]
    hk, d, bs = case.kv_heads, case.head_dim, case.block_size
    bps = SB // bb
    ids = np.asarray([i for b in range(case.batch)
                      for i in case.block_tables[b, :max(1, -(-int(case.seq_lens[b]) // bs))]],
                     dtype=np.int64)
    ids = np.unique(ids)
    off = case.offsets_f16[ids].astype(np.int64) * 2
    sb = torch.from_numpy(off // SB).cuda()
    idx = torch.from_numpy((off % SB) // bb).cuda()
    n_sb = g["mapped_bytes"] // SB
    for layer in range(case.num_layers):
        for base in (case.pool.va_k(layer), case.pool.va_v(layer)):
            image = torch.zeros(g["mapped_bytes"], dtype=torch.uint8, device="cuda")
            view = image.view(n_sb, SB)[:, :bps * bb].view(n_sb, bps, bb)
            for c0 in range(0, len(ids), 4096):
                c1 = min(len(ids), c0 + 4096)
                x = torch.randn((c1 - c0, bs, hk, d), generator=gen, device="cuda")
                amax = x.abs().amax(dim=(1, 3))
                scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
                q8 = (x / scale[:, None, :, None]).to(torch.float8_e4m3fn).view(torch.uint8)
                page = torch.zeros((c1 - c0, bb), dtype=torch.uint8, device="cuda")
                page[:, :data_bytes] = q8.reshape(c1 - c0, -1)
                page[:, data_bytes:data_bytes + 4 * hk] = scale.contiguous().view(torch.uint8).reshape(c1 - c0, -1)
                view[sb[c0:c1], idx[c0:c1]] = page
            _region_copy(base, image, g["mapped_bytes"])
            del image


@dataclass
class PrefillCase:
    """Chunked-prefill workload: sequences' pages (some shared), the chunk's
    queries and the device tensors the prefill entry point takes."""
    pool: KcmmPool
    dtype: int
    num_q_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    block_tables: np.ndarray        # int32 [B][mbps]
    seq_lens: np.ndarray            # int32 [B], cached tokens incl. the chunk
    qsl: np.ndarray                 # int32 [B+1]
    offsets_f16: np.ndarray
    q_bits: np.ndarray              # uint16 [T][Hq][D]
    dev: dict = field(default_factory=dict)

    @property
    def mbps(self) -> int:
        return self.block_tables.shape[1]

    def flops(self) -> float:
        """Algorithmic FLOPs: QK^T and PV over keys 0..p for every query."""
        hq, d = self.num_q_heads, self.head_dim
        total = 0
        for b in range(len(self.seq_lens)):
            n = int(self.qsl[b + 1] - self.qsl[b])
            first = int(self.seq_lens[b]) - n
            total += sum(first + i + 1 for i in range(n))
        return 4.0 * hq * d * total

    def run(self, layer: int = 0, stream_ptr: int = 0, scale=None) -> None:
        scale = 1.0 / math.sqrt(self.head_dim) if scale is None else scale
        d = self.dev
        self.pool.paged_attn_prefill(
            layer_idx=layer, query_ptr=d["q"].data_ptr(), out_ptr=d["out"].data_ptr(),
            block_tables_ptr=d["bt"].data_ptr(), seq_lens_ptr=d["sl"].data_ptr(),
            query_start_loc_ptr=d["qsl"].data_ptr(), block_offsets_f16_ptr=d["offs"].data_ptr(),
            batch=len(self.seq_lens), total_query_tokens=int(self.qsl[-1]),
            num_q_heads=self.num_q_heads, kv_heads=self.kv_heads, head_dim=self.head_dim,
            block_size=self.block_size, max_blocks_per_seq=self.mbps, scale=scale,
            stream_ptr=stream_ptr)


def build_prefix_shared_case(lib: KcmmLibrary, *, batch: int, prefix_tokens: int,
                             suffix_tokens: int, chunk: int, num_q_heads: int, kv_heads: int,
                             head_dim: int, block_size: int, dtype: int = KV_BF16,
                             num_layers: int = 1, seed: int = 0,
                             device: str = "cuda") -> PrefillCase:
    """`batch` sequences share `prefix_tokens` of refcounted pages (sequence 0
    owns them, the others take them with kcmm_share_prefix) and own
    `suffix_tokens` each; the chunk is the last `chunk` tokens of every
    sequence.  Regions are filled on the device."""
    assert prefix_tokens % block_size == 0
    rng = np.random.default_rng(seed)
    total = prefix_tokens + suffix_tokens
    cfg = make_config(num_layers=num_layers, kv_heads=kv_heads, head_dim=head_dim,
                      max_batch=batch, max_seq_len=total, block_size=block_size)
    pool = lib.create_pool(cfg, dtype)
    npre = prefix_tokens // block_size
    nsuf = -(-suffix_tokens // block_size)
    mbps = npre + nsuf
    bt = np.zeros((batch, mbps), dtype=np.int32)
    pre = pool.alloc_blocks(npre) if npre else []
    for b in range(batch):
        own = pool.alloc_blocks(nsuf)
        if b == 0:
            s = pool.register_sequence(pre + own)
        else:
            s = pool.register_sequence([])
            pool.share_prefix(0, s, npre)
            for blk in own:
                pool.append_block_to_sequence(s, blk)
        pool.update_seq_len(s, total)
        bt[b] = pool.block_table(s)
    offs = np.asarray(pool.all_block_offsets_f16(), dtype=np.uint64)
    sl = np.full(batch, total, dtype=np.int32)
    qsl = (np.arange(batch + 1) * chunk).astype(np.int32)
    q = encode16(io_dtype(dtype),
                 rng.standard_normal((batch * chunk, num_q_heads, head_dim)).astype(np.float32))
    case = PrefillCase(pool=pool, dtype=dtype, num_q_heads=num_q_heads, kv_heads=kv_heads,
                       head_dim=head_dim, block_size=block_size, block_tables=bt, seq_lens=sl,
                       qsl=qsl, offsets_f16=offs, q_bits=q)
    shim = DecodeCase(lib=lib, pool=pool, dtype=dtype, batch=batch, num_q_heads=num_q_heads,
                      kv_heads=kv_heads, head_dim=head_dim, block_size=block_size,
                      num_layers=num_layers, seq_lens=sl, block_tables=bt, offsets_f16=offs,
                      q_bits=q)
    fill_regions_on_device(shim, seed + 1)
    tdt = torch_io_dtype(dtype)
    qt = torch.from_numpy(q.copy()) if dtype == KV_F32 else torch.from_numpy(q.view(np.int16)).view(tdt)
    case.dev = {
        "q": qt.to(device),
        "out": torch.zeros((batch * chunk, num_q_heads, head_dim), dtype=tdt, device=device),
        "bt": torch.from_numpy(bt).to(device),
        "sl": torch.from_numpy(sl.copy()).to(device),
        "qsl": torch.from_numpy(qsl.copy()).to(device),
        "offs": torch.from_numpy(offs.view(np.int64)).to(device),
    }
    return case


def rope_inv_freq(theta: float, head_dim: int) -> np.ndarray:
    """Default (unscaled) RoPE frequencies, fp32: theta^(-2i/head_dim) for
    i < head_dim/2, the rotate-half pairing (i, i + head_dim/2)."""
    return (1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))).astype(np.float32)
