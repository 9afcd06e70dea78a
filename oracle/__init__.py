"""Python access to the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker used by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg.  Nothing in the
lattice_amd package imports this module, and no product code path may fall
back to it.  oracle.h says which reference lines each function restates;
tests/test_oracle_*.py pin each one to the reference's own expectations.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

F16, BF16, FP8, F32 = 0, 1, 2, 3
_NP_STORAGE = {F16: np.uint16, BF16: np.uint16, FP8: np.uint8, F32: np.float32}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle` (or __graft_entry__.build())")
        _lib = C.CDLL(str(LIB_PATH))
        _bind(_lib)
    return _lib


REF_C_CALLER = Path("/root/reference/examples/kcmm_c_integration.c")


def build() -> None:
    """Compiles liboracle.so and, where the reference tree is present (this
    container; the GPU box only has the built files), the reference's own C
    caller of the ABI into _ref/ (see the Makefile)."""
    import subprocess
    subprocess.run(["make", "-s", "-B", "-C", str(HERE), "liboracle.so"], check=True)
    if REF_C_CALLER.exists():
        subprocess.run(["make", "-s", "-B", "-C", str(HERE), "ref"], check=True)


P = C.c_void_p
U32, U64, I32, F = C.c_uint32, C.c_uint64, C.c_int32, C.c_float


def _bind(l: C.CDLL) -> None:
    sig = {
        "oracle_f32_to_bf16": ([F], C.c_uint16), "oracle_bf16_to_f32": ([C.c_uint16], F),
        "oracle_f32_to_f16": ([F], C.c_uint16), "oracle_f16_to_f32": ([C.c_uint16], F),
        "oracle_f32_to_e4m3": ([F], C.c_uint8), "oracle_e4m3_to_f32": ([C.c_uint8], F),
        "oracle_encode_array": ([C.c_int, P, P, C.c_size_t], None),
        "oracle_decode_array": ([C.c_int, P, P, C.c_size_t], None),
        "opool_new": ([C.c_size_t] * 6 + [C.c_int, C.c_int], P),
        "opool_delete": ([P], None),
        "opool_alloc": ([P, U32, P], C.c_int),
        "opool_release": ([P, P, U32], None),
        "opool_register": ([P, P, U32], U32),
        "opool_unregister": ([P, U32], None),
        "opool_append_block": ([P, U32, U32], C.c_int),
        "opool_update_seq_len": ([P, U32, U32], None),
        "opool_block_table": ([P, U32, P, U32, P], C.c_int),
        "opool_block_offset": ([P, U32, P], C.c_int),
        "opool_offsets_f16": ([P, P, U32], U32),
        "opool_valid_flags": ([P, P, U32], U32),
        "opool_table_offsets": ([P, U32, P, U32, P], C.c_int),
        "opool_fork": ([P, U32, P], C.c_int),
        "opool_share_prefix": ([P, U32, U32, U32, P], C.c_int),
        "opool_cow": ([P, U32, U32, P, P], C.c_int),
        "opool_refcount": ([P, U32], U32),
        "opool_incref": ([P, U32], C.c_int),
        "opool_seq_len": ([P, U32], U32),
        "opool_stats": ([P, P], None),
        "opool_metrics": ([P, P], None),
        "opool_below_low_watermark": ([P, F], C.c_int),
        "opool_enable_tiering": ([P, C.c_int, C.c_size_t, C.c_size_t], C.c_int),
        "opool_set_policy": ([P, C.c_char_p], C.c_int),
        "opool_policy_name": ([P], C.c_char_p),
        "opool_location": ([P, U32], C.c_int),
        "opool_cpu_offset": ([P, U32], C.c_uint64),
        "opool_access": ([P, U32], C.c_int),
        "opool_evict": ([P, U32, P], U32),
        "opool_restore_one": ([P, U32, P], C.c_int),
        "opool_restore": ([P, P, U32], C.c_int),
        "otier_new": ([C.c_int, C.c_size_t, C.c_uint64, C.c_uint64], P),
        "otier_free": ([P], None),
        "otier_event": ([P, C.c_int, U32, U32], None),
        "otier_select": ([P, P, C.c_size_t, C.c_size_t, P], C.c_size_t),
        "otier_slot_alloc": ([P, C.c_uint64, P], C.c_int),
        "otier_slot_free": ([P, C.c_uint64, C.c_uint64], None),
        "otier_ranges": ([P, P, C.c_size_t], C.c_size_t),
        "otier_arc_list": ([P, C.c_int, P, C.c_size_t], C.c_size_t),
        "otier_arc_p": ([P], C.c_size_t),
        "oracle_kv_write_rows": ([C.c_int, P, P, P, P, P, P, P, U32, U32, U32, U32, U32], C.c_int),
        "oracle_kv_write_device_slots": ([C.c_int, P, P, P, P, P, U32, P, P, U32, U32, U32, U32,
                                          U32, U32, P], C.c_int),
        "oracle_copy_pages": ([P, U32, P, U32, U32], None),
        "oracle_attn_decode_f64": ([C.c_int, P, P, P, P, P, P, P] + [U32] * 8 + [C.c_double],
                                   C.c_int),
        "oracle_attn_decode_ref_f32": ([C.c_int, P, P, P, P, P, P, P] + [U32] * 7 + [F, C.c_int],
                                       C.c_int),
        "oracle_attn_prefill_f64": ([C.c_int, P, P, P, P, P, P, P, P] + [U32] * 8 + [C.c_double],
                                    C.c_int),
        "oracle_gemm_bf16_f64": ([P, P, P, U32, U32, U32], None),
        "oracle_gemm_fp8w_f64": ([P, P, P, P, U32, U32, U32], None),
    }
    for name, (args, res) in sig.items():
        fn = getattr(l, name)
        fn.argtypes = args
        fn.restype = res


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---- numeric formats -------------------------------------------------------

def encode(dtype: int, x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=_NP_STORAGE[dtype])
    lib().oracle_encode_array(dtype, _p(x), _p(out), x.size)
    return out


def decode(dtype: int, x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=_NP_STORAGE[dtype])
    out = np.empty(x.shape, dtype=np.float32)
    lib().oracle_decode_array(dtype, _p(x), _p(out), x.size)
    return out


# ---- page allocator ----------------------------------------------------------

class OraclePool:
    """Restatement of the reference allocator (ref superblock.rs, pool.rs)."""

    def __init__(self, block_size, num_layers, kv_heads, head_dim, max_batch, max_seq_len,
                 dtype=F16, rollback_on_failure=True):
        self._h = lib().opool_new(block_size, num_layers, kv_heads, head_dim, max_batch,
                                  max_seq_len, dtype, int(rollback_on_failure))
        self.block_size = block_size

    def __del__(self):
        if getattr(self, "_h", None):
            lib().opool_delete(self._h)
            self._h = None

    def alloc(self, n: int) -> list[int] | None:
        out = np.zeros(max(n, 1), dtype=np.uint32)
        return None if lib().opool_alloc(self._h, n, _p(out)) else out[:n].tolist()

    def release(self, ids):
        a = np.asarray(ids, dtype=np.uint32)
        lib().opool_release(self._h, _p(a), a.size)

    def register(self, table) -> int:
        a = np.asarray(table, dtype=np.uint32)
        return lib().opool_register(self._h, _p(a) if a.size else None, a.size)

    def unregister(self, seq):
        lib().opool_unregister(self._h, seq)

    def append_block(self, seq, blk) -> int:
        return lib().opool_append_block(self._h, seq, blk)

    def update_seq_len(self, seq, n):
        lib().opool_update_seq_len(self._h, seq, n)

    def block_table(self, seq, max_blocks=1 << 16):
        out = np.zeros(max_blocks, dtype=np.uint32)
        cnt = C.c_uint32(0)
        rc = lib().opool_block_table(self._h, seq, _p(out), max_blocks, C.byref(cnt))
        return None if rc else out[: cnt.value].tolist()

    def block_offset(self, blk):
        v = C.c_uint64(0)
        return None if lib().opool_block_offset(self._h, blk, C.byref(v)) else v.value

    def offsets_f16(self, max_blocks=1 << 20):
        out = np.zeros(max_blocks, dtype=np.uint64)
        n = lib().opool_offsets_f16(self._h, _p(out), max_blocks)
        return out[:n]

    def valid_flags(self, max_blocks=1 << 20):
        out = np.zeros(max_blocks, dtype=np.uint8)
        n = lib().opool_valid_flags(self._h, _p(out), max_blocks)
        return out[:n]

    def table_offsets(self, seq, max_blocks=1 << 16):
        out = np.zeros(max_blocks, dtype=np.uint64)
        cnt = C.c_uint32(0)
        rc = lib().opool_table_offsets(self._h, seq, _p(out), max_blocks, C.byref(cnt))
        return None if rc else out[: cnt.value].tolist()

    def fork(self, src):
        v = C.c_uint32(0)
        return None if lib().opool_fork(self._h, src, C.byref(v)) else v.value

    def share_prefix(self, src, dst, n):
        out = np.zeros(max(n, 1), dtype=np.uint32)
        return None if lib().opool_share_prefix(self._h, src, dst, n, _p(out)) else out[:n].tolist()

    def cow(self, seq, logical):
        s, d = C.c_uint32(0), C.c_uint32(0)
        rc = lib().opool_cow(self._h, seq, logical, C.byref(s), C.byref(d))
        return rc, (s.value, d.value)

    def refcount(self, blk) -> int:
        return lib().opool_refcount(self._h, blk)

    def incref(self, blk) -> bool:
        return lib().opool_incref(self._h, blk) == 0

    def seq_len(self, seq) -> int:
        return lib().opool_seq_len(self._h, seq)

    def stats(self) -> dict:
        st = np.zeros(14, dtype=np.uint64)
        lib().opool_stats(self._h, _p(st))
        keys = ["blocks_in_use", "total_blocks", "total_physical_blocks", "free_physical_blocks",
                "active_sequences", "num_layers", "blocks_per_superblock", "superblock_count",
                "block_size", "max_blocks_per_seq", "block_bytes"]
        d = {k: int(st[i]) for i, k in enumerate(keys)}
        d["physical_idle_ratio"] = float(np.array([st[11]], dtype=np.uint32).view(np.float32)[0])
        d["max_physical_blocks"] = int(st[12])
        d["region_superblocks"] = int(st[13])
        return d

    def metrics(self) -> dict:
        m = np.zeros(4, dtype=np.float32)
        lib().opool_metrics(self._h, _p(m))
        return dict(zip(["ifr", "pme", "bu", "rfi"], m.tolist()))

    def below_low_watermark(self, t) -> bool:
        return bool(lib().opool_below_low_watermark(self._h, t))

    # tiering (ref tiering.rs, pool.rs:824-1002, ffi.rs:1900-2008)
    def enable_tiering(self, policy=0, max_blocks=0, max_batch_blocks=0):
        return lib().opool_enable_tiering(self._h, policy, max_blocks, max_batch_blocks) == 0

    def set_policy(self, name: str) -> bool:
        return lib().opool_set_policy(self._h, name.encode()) == 0

    def policy_name(self) -> str:
        return lib().opool_policy_name(self._h).decode()

    def location(self, blk) -> int | None:
        v = lib().opool_location(self._h, blk)
        return None if v < 0 else v

    def cpu_offset(self, blk):
        v = lib().opool_cpu_offset(self._h, blk)
        return None if v == 2**64 - 1 else v

    def access(self, blk) -> bool:
        return lib().opool_access(self._h, blk) == 0

    def evict(self, count) -> list[int]:
        out = np.zeros(max(self.stats()["total_blocks"], 1), dtype=np.uint32)
        n = lib().opool_evict(self._h, count, _p(out))
        return out[:n].tolist()

    def restore_one(self, blk):
        v = C.c_uint64(0)
        return None if lib().opool_restore_one(self._h, blk, C.byref(v)) else v.value

    def restore(self, ids) -> bool:
        a = np.asarray(ids, dtype=np.uint32)
        return lib().opool_restore(self._h, _p(a) if a.size else None, a.size) == 0


class OracleTier:
    """One eviction policy + swap-slot allocator (ref tiering.rs:25-643),
    with handles as (superblock, index) tuples."""
    POLICIES = {"lru": 0, "lfu": 1, "fifo": 2, "arc": 3, "sink_window": 4}

    def __init__(self, policy="lru", arc_capacity=1, swap_size=0, per_block=0):
        self._h = lib().otier_new(self.POLICIES[policy], arc_capacity, swap_size, per_block)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().otier_free(self._h)
            self._h = None

    def on_allocate(self, h):
        lib().otier_event(self._h, 0, h[0], h[1])

    def on_access(self, h):
        lib().otier_event(self._h, 1, h[0], h[1])

    def on_evict(self, h):
        lib().otier_event(self._h, 2, h[0], h[1])

    def select_victims(self, cands, count):
        a = np.asarray(cands, dtype=np.uint32).reshape(-1)
        out = np.zeros(max(a.size, 2), dtype=np.uint32)
        n = lib().otier_select(self._h, _p(a) if a.size else None, a.size // 2, count, _p(out))
        return [tuple(int(v) for v in out[2 * i:2 * i + 2]) for i in range(n)]

    def allocate(self, size):
        v = C.c_uint64(0)
        return None if lib().otier_slot_alloc(self._h, size, C.byref(v)) else v.value

    def free(self, off, size):
        lib().otier_slot_free(self._h, off, size)

    def free_ranges(self):
        out = np.zeros(2 * 4096, dtype=np.uint64)
        n = lib().otier_ranges(self._h, _p(out), 4096)
        return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(n)]

    def arc_list(self, which):
        out = np.zeros(2 * 4096, dtype=np.uint32)
        n = lib().otier_arc_list(self._h, {"t1": 0, "t2": 1, "b1": 2, "b2": 3}[which], _p(out), 4096)
        return [tuple(int(v) for v in out[2 * i:2 * i + 2]) for i in range(n)]

    def arc_p(self):
        return lib().otier_arc_p(self._h)


# ---- prefix cache ------------------------------------------------------------------
# The reference's prefix-sharing manager contract (src/kcmm/sharing.rs:9-65:
# content hash -> prefix blocks, reference counted; a placeholder there),
# restated over OraclePool.

FNV64_OFFSET, FNV64_PRIME = 0xCBF29CE484222325, 0x100000001B3


def fnv1a64(data: bytes, h: int = FNV64_OFFSET) -> int:
    """FNV-1a, 64-bit (the published algorithm: xor each byte, multiply by
    the FNV prime, modulo 2^64)."""
    for b in data:
        h = ((h ^ b) * FNV64_PRIME) & 0xFFFFFFFFFFFFFFFF
    return h


def prefix_hash_blocks(tokens, block_size: int, seed: int = 0) -> list[int]:
    """Chained hashes of the full blocks of a token sequence: hash i is
    FNV-1a-64 of (hash i-1 as 8 LE bytes, seed for block 0) + the block's
    token ids as int32 LE."""
    t = np.asarray(tokens, dtype=np.int32)
    out, prev = [], seed & 0xFFFFFFFFFFFFFFFF
    for i in range(len(t) // block_size):
        prev = fnv1a64(prev.to_bytes(8, "little") +
                       t[i * block_size:(i + 1) * block_size].astype("<i4").tobytes())
        out.append(prev)
    return out


class OraclePrefixCache:
    """Prefix cache over an OraclePool: key -> (block, depth, last_use); each
    entry holds one reference on its block."""

    def __init__(self, pool: OraclePool):
        self.pool, self.entries, self.tick = pool, {}, 0

    def register(self, seq, hashes) -> int | None:
        table = self.pool.block_table(seq)
        n = len(hashes)
        if table is None or n > len(table):
            return None
        if n * self.pool.block_size > self.pool.seq_len(seq):
            return None
        if any(self.pool.refcount(b) == 0 for b in table[:n]):
            return None
        added = 0
        for i, h in enumerate(hashes):
            if h in self.entries:
                continue
            self.tick += 1
            self.entries[h] = [table[i], i, self.tick]
            self.pool.incref(table[i])
            added += 1
        return added

    def match(self, hashes) -> list[int]:
        self.tick += 1
        out = []
        for h in hashes:
            e = self.entries.get(h)
            if e is None:
                break
            e[2] = self.tick
            out.append(e[0])
        return out

    def attach(self, dst, hashes) -> list[int] | None:
        if self.pool.block_table(dst) is None:
            return None
        blocks = self.match(hashes)
        for b in blocks:
            self.pool.incref(b)
            self.pool.append_block(dst, b)
        return blocks

    def evict(self, n) -> int:
        order = sorted(self.entries.items(), key=lambda kv: (kv[1][2], -kv[1][1]))[:n]
        for h, _ in order:
            del self.entries[h]
        if order:
            self.pool.release([e[0] for _, e in order])
        return len(order)


# ---- KV write / page copy ------------------------------------------------------

def _check_page_end(regions, page_end: int, what: str) -> None:
    """The C oracle trusts its offsets: refuse writes past a host region."""
    if any(r.nbytes < page_end for r in regions):
        raise ValueError(f"{what}: a write ends at byte {page_end}, past a region of "
                         f"{min(r.nbytes for r in regions)} bytes")


def _page_bytes(dtype, kv_heads, data_bytes):
    return data_bytes + (4 * kv_heads if dtype == FP8 else 0)


def kv_write_rows(dtype, k_region, v_region, k_src, v_src, page_offsets, slots, src_rows,
                  kv_heads, head_dim, row_bytes, data_bytes):
    po = np.ascontiguousarray(page_offsets, dtype=np.uint64)
    sl = np.ascontiguousarray(slots, dtype=np.uint32)
    if po.size:
        _check_page_end((k_region, v_region),
                        int(po.max()) + _page_bytes(dtype, kv_heads, data_bytes), "kv_write_rows")
    sr = np.ascontiguousarray(src_rows, dtype=np.uint32)
    lib().oracle_kv_write_rows(dtype, _p(k_region), _p(v_region), _p(k_src), _p(v_src), _p(po),
                               _p(sl), _p(sr), po.size, kv_heads, head_dim, row_bytes, data_bytes)


def kv_write_device_slots(dtype, k_region, v_region, k_src, v_src, slots, offsets_f16, valid,
                          block_size, kv_heads, head_dim, row_bytes, data_bytes) -> int:
    s = np.ascontiguousarray(slots, dtype=np.int64)
    o = np.ascontiguousarray(offsets_f16, dtype=np.uint64)
    ids = s[s >= 0] // block_size
    ids = ids[ids < o.size]
    if ids.size:
        _check_page_end((k_region, v_region),
                        int(o[ids].max()) * 2 + _page_bytes(dtype, kv_heads, data_bytes),
                        "kv_write_device_slots")
    v = None if valid is None else np.ascontiguousarray(valid, dtype=np.uint8)
    status = np.zeros(1, dtype=np.int32)
    lib().oracle_kv_write_device_slots(dtype, _p(k_region), _p(v_region), _p(k_src), _p(v_src),
                                       _p(s), s.size, _p(o), _p(v), o.size, block_size, kv_heads,
                                       head_dim, row_bytes, data_bytes, _p(status))
    return int(status[0])


def copy_pages(regions: list[np.ndarray], pairs, block_bytes: int) -> None:
    ptrs = (C.c_void_p * len(regions))(*[r.ctypes.data for r in regions])
    pr = np.ascontiguousarray(pairs, dtype=np.uint64).reshape(-1)
    if pr.size:
        end = int(pr.max()) + block_bytes
        if any(r.nbytes < end for r in regions):
            raise ValueError(f"copy_pages: a page ends at byte {end}, past a region of "
                             f"{min(r.nbytes for r in regions)} bytes")
    lib().oracle_copy_pages(C.cast(ptrs, C.c_void_p), len(regions), _p(pr), pr.size // 2,
                            block_bytes)


# ---- attention / GEMM ------------------------------------------------------------

def attn_decode_f64(dtype, q, k_region, v_region, block_tables, seq_lens, offsets_f16,
                    num_q_heads, kv_heads, head_dim, block_size, row_bytes, data_bytes, scale):
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    of = np.ascontiguousarray(offsets_f16, dtype=np.uint64)
    q = np.ascontiguousarray(q)
    batch, mbps = bt.shape
    out = np.zeros((batch, num_q_heads, head_dim), dtype=np.float64)
    lib().oracle_attn_decode_f64(dtype, _p(q), _p(out), _p(k_region), _p(v_region), _p(bt),
                                 _p(sl), _p(of), batch, num_q_heads, kv_heads, head_dim,
                                 block_size, mbps, row_bytes, data_bytes, scale)
    return out


def attn_prefill_f64(dtype, q, k_region, v_region, block_tables, seq_lens, query_start_loc,
                     offsets_f16, num_q_heads, kv_heads, head_dim, block_size, row_bytes,
                     data_bytes, scale):
    """Causal chunked prefill (fp64): q/out [total_rows][Hq][D]."""
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    qsl = np.ascontiguousarray(query_start_loc, dtype=np.int32)
    of = np.ascontiguousarray(offsets_f16, dtype=np.uint64)
    q = np.ascontiguousarray(q)
    batch, mbps = bt.shape
    out = np.zeros((int(qsl[-1]), num_q_heads, head_dim), dtype=np.float64)
    lib().oracle_attn_prefill_f64(dtype, _p(q), _p(out), _p(k_region), _p(v_region), _p(bt),
                                  _p(sl), _p(qsl), _p(of), batch, num_q_heads, kv_heads,
                                  head_dim, block_size, mbps, row_bytes, data_bytes, scale)
    return out


def attn_decode_ref_f32(dtype, q, k_region, v_region, block_tables, seq_lens, offsets_f16,
                        num_q_heads, kv_heads, head_dim, block_size, row_bytes, scale,
                        threads=0, out=None):
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    of = np.ascontiguousarray(offsets_f16, dtype=np.uint64)
    q = np.ascontiguousarray(q)
    batch, mbps = bt.shape
    if out is None:
        out = np.zeros((batch, num_q_heads, head_dim), dtype=np.float32)
    rc = lib().oracle_attn_decode_ref_f32(dtype, _p(q), _p(out), _p(k_region), _p(v_region),
                                          _p(bt), _p(sl), _p(of), batch, num_q_heads, kv_heads,
                                          head_dim, block_size, mbps, row_bytes, scale, threads)
    if rc:
        raise ValueError("oracle_attn_decode_ref_f32: unsupported dtype/head_dim")
    return out


def gemm_bf16_f64(x_bits: np.ndarray, w_bits: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    m, k = x.shape
    n, k2 = w.shape
    assert k == k2
    y = np.zeros((m, n), dtype=np.float64)
    lib().oracle_gemm_bf16_f64(_p(x), _p(w), _p(y), m, n, k)
    return y


def gemm_fp8w_f64(x_bits: np.ndarray, w8: np.ndarray, wscale: np.ndarray) -> np.ndarray:
    """Y = X (decode(W8) diag(wscale))^T in fp64 (bf16 X, e4m3 W8, fp32 scale per row)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w = np.ascontiguousarray(w8, dtype=np.uint8)
    s = np.ascontiguousarray(wscale, dtype=np.float32)
    m, k = x.shape
    n, k2 = w.shape
    assert k == k2 and s.shape == (n,)
    y = np.zeros((m, n), dtype=np.float64)
    lib().oracle_gemm_fp8w_f64(_p(x), _p(w), _p(s), _p(y), m, n, k)
    return y


def quantize_fp8_rows(w: np.ndarray):
    """Per-row e4m3 weights: scale = amax/448 (1 for an all-zero row), codes =
    RNE of w/scale with saturation (the page writer's rule, applied per row)."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.abs(w).max(axis=1)
    scale = np.where(amax > 0, amax / np.float32(448.0), np.float32(1.0)).astype(np.float32)
    return encode(FP8, w / scale[:, None]), scale


# ---- decode-step glue and one decoder layer ----------------------------------
# Restatement of one layer of ref LlamaTransformer::forward_step_paged
# (src/model/llama_transformer.rs:262-391) with Hugging Face Llama semantics
# (the reference's own rope.cu pairs and theta are not HF's): fp64 arithmetic,
# activations rounded to bf16 wherever a bf16 model stores them.

def bf16_round(x) -> np.ndarray:
    return decode(BF16, encode(BF16, np.asarray(x, dtype=np.float64))).astype(np.float64)


def rmsnorm_f64(x, w, eps, round_bf16=True):
    """HF LlamaRMSNorm: w * (x * rsqrt(mean(x^2) + eps)), the normalised row
    rounded to bf16 before the weight multiply when round_bf16."""
    x = np.asarray(x, dtype=np.float64)
    t = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    if round_bf16:
        return bf16_round(np.asarray(w, dtype=np.float64) * bf16_round(t))
    return np.asarray(w, dtype=np.float64) * t


def default_inv_freq(theta: float, head_dim: int) -> np.ndarray:
    """HF default rope: inv_freq[i] = theta^(-2i/head_dim), i < head_dim/2."""
    return 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))


def rope_f64(x, pos, inv_freq):
    """HF apply_rotary_pos_emb on the last axis: x*cos + rotate_half(x)*sin,
    angle pos * inv_freq[i] for the pair (i, i + D/2).  pos broadcasts
    against x's leading axes (x.shape[:-1])."""
    x = np.asarray(x, dtype=np.float64)
    d2 = x.shape[-1] // 2
    ang = np.asarray(pos, dtype=np.float64)[..., None] * np.asarray(inv_freq, dtype=np.float64)
    c = np.concatenate([np.cos(ang), np.cos(ang)], axis=-1)
    s = np.concatenate([np.sin(ang), np.sin(ang)], axis=-1)
    rot = np.concatenate([-x[..., d2:], x[..., :d2]], axis=-1)
    return x * c + rot * s


def silu_mul_f64(gate, up):
    g = np.asarray(gate, dtype=np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(up, dtype=np.float64)


def fp8_page_rows(region, page_byte, slots, kv_heads, head_dim, row_bytes, data_bytes):
    """Dequantized rows [len(slots)][Hkv][D] of an fp8 page: e4m3 codes times
    the page's per-kv-head scale (footer at data_bytes)."""
    sc = region[page_byte + data_bytes:page_byte + data_bytes + 4 * kv_heads].view(np.float32)
    out = np.empty((len(slots), kv_heads, head_dim), dtype=np.float64)
    for i, s in enumerate(slots):
        a = page_byte + s * row_bytes
        codes = region[a:a + kv_heads * head_dim].reshape(kv_heads, head_dim)
        out[i] = decode(FP8, codes).astype(np.float64) * sc[:, None]
    return out


def layer_weight_f64(w, name):
    """Layer weight `name` of dict w in fp64: bf16 bits, or, for fp8-weight
    projections, a (e4m3 codes [out][in], fp32 scale [out]) pair whose
    weight is code * scale row by row."""
    v = w[name]
    if isinstance(v, tuple):
        codes, scale = v
        return decode(FP8, codes).astype(np.float64) * np.asarray(scale, np.float64)[:, None]
    return decode(BF16, v).astype(np.float64)


def decode_layer_step_f64(hidden_bits, w, k_region, v_region, block_tables, seq_lens,
                          offsets_f16, inv_freq, num_q_heads, kv_heads, head_dim,
                          intermediate, block_size, row_bytes, eps, round_bf16=True,
                          dtype=BF16, data_bytes=0):
    """One decoder layer of a decode step for a bf16 pool (dtype FP8: an
    fp8-e4m3 pool, the new k / v rows written by kv_write_rows and every row
    read back dequantized).

    hidden_bits [B][H] uint16 (bf16); w: dict of bf16-bit arrays attn_norm [H],
    qkv [(Hq+2Hkv)D][H], o [H][Hq D], mlp_norm [H], gate_up [2I][H], down [H][I]
    (a projection may instead be an fp8 (codes, row scales) pair, see
    layer_weight_f64).
    Sequence b's new token is at position seq_lens[b] - 1; its rotated k and v
    are written (as bf16) into k_region / v_region (uint8 copies of the
    layer's regions) and attention runs over rows 0..pos of its pages (the
    new row at full precision when not round_bf16).  round_bf16 rounds every
    stored activation to bf16 as a bf16 model does; without it the layer is
    computed in fp64 throughout.  Returns the new hidden state (float64)."""
    rnd = bf16_round if round_bf16 else (lambda a: np.asarray(a, dtype=np.float64))
    f = lambda name: layer_weight_f64(w, name)
    hq, hkv, d = num_q_heads, kv_heads, head_dim
    grp = hq // hkv
    x = decode(BF16, hidden_bits).astype(np.float64)
    bsz = x.shape[0]
    pos = np.asarray(seq_lens, dtype=np.int64) - 1
    bt = np.asarray(block_tables)
    n1 = rmsnorm_f64(x, f("attn_norm"), eps, round_bf16)
    qkv = rnd(n1 @ f("qkv").T)
    q = qkv[:, :hq * d].reshape(bsz, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].reshape(bsz, hkv, d)
    v = qkv[:, (hq + hkv) * d:].reshape(bsz, hkv, d)
    pe = np.maximum(pos, 0)[:, None].astype(np.float64)
    q_r = rnd(rope_f64(q, pe, inv_freq))
    k_r = rnd(rope_f64(k, pe, inv_freq))
    att = np.zeros((bsz, hq, d), dtype=np.float64)
    for b in range(bsz):
        p = int(pos[b])
        if p < 0 or p >= bt.shape[1] * block_size:
            continue
        rows_k, rows_v = [], []
        if dtype == FP8:
            pb = int(offsets_f16[bt[b, p // block_size]]) * 2
            kv_write_rows(FP8, k_region, v_region,
                          encode(BF16, k_r[b].ravel()).reshape(1, -1),
                          encode(BF16, v[b].ravel()).reshape(1, -1), [pb], [p % block_size],
                          [0], hkv, d, row_bytes, data_bytes)
            for t in range(p + 1):
                pg = int(offsets_f16[bt[b, t // block_size]]) * 2
                rows_k.append(fp8_page_rows(k_region, pg, [t % block_size], hkv, d, row_bytes,
                                            data_bytes)[0])
                rows_v.append(fp8_page_rows(v_region, pg, [t % block_size], hkv, d, row_bytes,
                                            data_bytes)[0])
        for t in range(p + 1 if dtype != FP8 else 0):
            base = int(offsets_f16[bt[b, t // block_size]]) * 2 + (t % block_size) * row_bytes
            if t == p:
                k_region[base:base + hkv * d * 2] = encode(BF16, k_r[b].ravel()).view(np.uint8)
                v_region[base:base + hkv * d * 2] = encode(BF16, v[b].ravel()).view(np.uint8)
                rows_k.append(k_r[b])
                rows_v.append(v[b])
                continue
            rows_k.append(decode(BF16, k_region[base:base + hkv * d * 2].view(np.uint16))
                          .astype(np.float64).reshape(hkv, d))
            rows_v.append(decode(BF16, v_region[base:base + hkv * d * 2].view(np.uint16))
                          .astype(np.float64).reshape(hkv, d))
        kk, vv = np.stack(rows_k), np.stack(rows_v)            # [p+1][Hkv][D]
        for h in range(hq):
            sc = kk[:, h // grp, :] @ q_r[b, h] / np.sqrt(d)
            e = np.exp(sc - sc.max())
            att[b, h] = (e / e.sum()) @ vv[:, h // grp, :]
    att = rnd(att).reshape(bsz, hq * d)
    h1 = rnd(x + rnd(att @ f("o").T))
    n2 = rmsnorm_f64(h1, f("mlp_norm"), eps, round_bf16)
    gu = rnd(n2 @ f("gate_up").T)
    g = gu[:, :intermediate]
    act = rnd(rnd(g / (1.0 + np.exp(-g))) * gu[:, intermediate:])   # F.silu rounds, then * up
    return rnd(h1 + rnd(act @ f("down").T))
