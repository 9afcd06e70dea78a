"""The reference's KV-write known-answer test (ref
scripts/kcmm/kv_write_ffi_smoke.py:189-516), as a scenario that runs against
either the oracle (CPU) or libkcmm.so (GPU) and records region bytes and
status codes after each step."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

import oracle as O

KAT = json.loads((Path(__file__).parent / "golden" / "kv_write_kat.json").read_text())


def f16_rows(n, step, offset):
    """torch.arange(n*step, dtype=float16) + offset, as raw f16 bits."""
    return (np.arange(n * step, dtype=np.float32) + offset).astype(np.float16).view(
        np.uint16).reshape(n, step)


def resolve_slots(spec, blocks, block_size):
    out = []
    for s in spec:
        out.append(-1 if s[0] == -1 else blocks[int(s[0][1])] * block_size + s[1])
    return out


def run_oracle():
    """Replay the KAT on the oracle; returns the recorded observations."""
    c = KAT["config"]
    bs, step = c["block_size"], c["kv_heads"] * c["head_dim"]
    pool = O.OraclePool(bs, c["num_layers"], c["kv_heads"], c["head_dim"], c["max_batch"],
                        c["max_seq_len"], O.F16)
    ids = pool.alloc(KAT["setup"]["alloc"])
    inactive = ids[KAT["setup"]["free_index"]]
    pool.release([inactive])
    blocks = ids[: KAT["setup"]["register_first"]]
    seq = pool.register(blocks)
    region = pool.stats()["superblock_count"] * 2 * 1024 * 1024
    kreg = np.zeros(region, np.uint8)
    vreg = np.zeros(region, np.uint8)
    row_bytes = step * 2
    obs = {"blocks": blocks, "inactive": inactive, "seq": seq, "steps": [],
           "block_offset": {b: pool.block_offset(b) for b in blocks}}

    pw = KAT["position_write"]
    k = f16_rows(2, step, pw["k_offset"])
    v = f16_rows(2, step, pw["v_offset"])
    tbl = pool.block_table(seq)
    pages = [pool.block_offset(tbl[p // bs]) for p in pw["positions"]]
    O.kv_write_rows(O.F16, kreg, vreg, k, v, pages, [p % bs for p in pw["positions"]], [0, 1],
                    c["kv_heads"], c["head_dim"], row_bytes, row_bytes * bs)
    obs["steps"].append(("position", kreg.copy(), vreg.copy()))

    hs = KAT["host_slot_write"]
    slots = resolve_slots(hs["slots"], blocks, bs)
    k = f16_rows(3, step, hs["k_offset"])
    v = f16_rows(3, step, hs["v_offset"])
    rows = [(pool.block_offset(s // bs), s % bs, r) for r, s in enumerate(slots) if s >= 0]
    O.kv_write_rows(O.F16, kreg, vreg, k, v, [r[0] for r in rows], [r[1] for r in rows],
                    [r[2] for r in rows], c["kv_heads"], c["head_dim"], row_bytes, row_bytes * bs)
    obs["steps"].append(("host_slots", kreg.copy(), vreg.copy()))

    ds = KAT["device_slot_write"]
    slots = resolve_slots(ds["slots"], blocks, bs)
    k = f16_rows(3, step, ds["k_offset"])
    v = f16_rows(3, step, ds["v_offset"])
    offs = pool.offsets_f16()
    valid = pool.valid_flags()
    st = O.kv_write_device_slots(O.F16, kreg, vreg, k, v, slots, offs, valid, bs, c["kv_heads"],
                                 c["head_dim"], row_bytes, row_bytes * bs)
    obs["steps"].append(("device_slots", kreg.copy(), vreg.copy(), st))
    obs["offsets"] = offs.tolist()
    obs["valid"] = valid.tolist()

    invalid_slot = c["max_blocks"] * bs
    inactive_slot = inactive * bs
    obs["inactive_status"] = O.kv_write_device_slots(
        O.F16, kreg, vreg, k[:1], v[:1], [inactive_slot], offs, valid, bs, c["kv_heads"],
        c["head_dim"], row_bytes, row_bytes * bs)
    obs["invalid_status"] = O.kv_write_device_slots(
        O.F16, kreg, vreg, k[:1], v[:1], [invalid_slot], offs, valid, bs, c["kv_heads"],
        c["head_dim"], row_bytes, row_bytes * bs)
    obs["final"] = (kreg.copy(), vreg.copy())
    pool.unregister(seq)
    obs["blocks_in_use_after"] = pool.stats()["blocks_in_use"]
    return obs


def expected_rows(obs):
    """The KAT's own expectations: (step name, region, byte offset, bytes)."""
    c = KAT["config"]
    bs, step = c["block_size"], c["kv_heads"] * c["head_dim"]
    row_bytes = step * 2
    boff = obs["block_offset"]
    blocks = obs["blocks"]
    exp = []
    pw = KAT["position_write"]
    k = f16_rows(2, step, pw["k_offset"])
    v = f16_rows(2, step, pw["v_offset"])
    for r, p in enumerate(pw["positions"]):
        at = boff[blocks[p // bs]] + (p % bs) * row_bytes
        exp += [("position", "k", at, k[r].tobytes()), ("position", "v", at, v[r].tobytes())]
    for name, key, n in (("host_slots", "host_slot_write", 3), ("device_slots", "device_slot_write", 3)):
        spec = KAT[key]
        k = f16_rows(n, step, spec["k_offset"])
        v = f16_rows(n, step, spec["v_offset"])
        for r, s in enumerate(resolve_slots(spec["slots"], blocks, bs)):
            if s < 0:
                continue
            at = boff[s // bs] + (s % bs) * row_bytes
            exp += [(name, "k", at, k[r].tobytes()), (name, "v", at, v[r].tobytes())]
    return exp
