"""KV append: the oracle replays the reference's KV-write KAT (ref
scripts/kcmm/kv_write_ffi_smoke.py) and the address formulas of ref
paged_kv.rs:826-867; the fp8 write contract is pinned by closed forms."""
import numpy as np
import pytest

import oracle as O
from tests import kat_kv_write as K


def test_kat_rows_land_where_the_reference_says(oracle_lib):
    obs = K.run_oracle()
    regions = {s[0]: (s[1], s[2]) for s in obs["steps"]}
    for step, which, at, data in K.expected_rows(obs):
        reg = regions[step][0 if which == "k" else 1]
        assert reg[at:at + len(data)].tobytes() == data, (step, which, at)
    assert obs["steps"][2][3] == 0                 # device slots: status 0
    assert obs["valid"][obs["inactive"]] == 0
    assert obs["inactive_status"] == 2             # ref kv_write_ffi_smoke.py:452-478
    assert obs["invalid_status"] != 0              # ref :480-505
    assert obs["blocks_in_use_after"] == 0         # ref :507-516


def test_kat_touches_nothing_else(oracle_lib):
    obs = K.run_oracle()
    k, v = obs["final"]
    written = np.zeros(k.size, bool)
    for _, _, at, data in K.expected_rows(obs):
        written[at:at + len(data)] = True
    assert not k[~written].any() and not v[~written].any()


def test_address_formulas(oracle_lib):
    # ref paged_kv.rs:829-867: pos 47 of physical block 7 -> 7*16*512 + 15*512
    # elements; pos 25 through table [3, 7, 1] -> 7*16*512 + 9*512.
    bs, hk, d = 16, 4, 128
    step = hk * d
    row_bytes, block_bytes = step * 2, step * bs * 2
    reg_k = np.zeros(8 * block_bytes, np.uint8)
    reg_v = np.zeros_like(reg_k)
    src = np.arange(2 * step, dtype=np.uint16).reshape(2, step) + 1
    table = [3, 7, 1]
    for row, (blk, pos) in enumerate([(7, 47), (table[25 // bs], 25)]):
        reg_k[:] = 0
        O.kv_write_rows(O.F16, reg_k, reg_v, src, src, [blk * block_bytes], [pos % bs], [row],
                        hk, d, row_bytes, block_bytes)
        elems = np.nonzero(reg_k.view(np.uint16))[0]
        expect = 7 * 16 * 512 + (15 if row == 0 else 9) * 512
        assert elems[0] == expect and elems.size == step


def test_fp8_write_scale_and_regrowth(oracle_lib):
    # Closed forms of the fp8 page contract: slot 0 sets scale = amax/448;
    # a larger row raises it and re-encodes earlier rows with the new scale.
    hk, d, bs = 2, 64, 16
    row_bytes, data_bytes = hk * d, hk * d * bs
    block_bytes = ((data_bytes + 4 * hk + 255) // 256) * 256
    kreg = np.zeros(block_bytes, np.uint8)
    vreg = np.zeros(block_bytes, np.uint8)
    rng = np.random.default_rng(0)
    x0 = rng.standard_normal((1, hk, d)).astype(np.float32)
    b0 = O.encode(O.BF16, x0)
    O.kv_write_rows(O.FP8, kreg, vreg, b0, b0, [0], [0], [0], hk, d, row_bytes, data_bytes)
    sc = kreg[data_bytes:data_bytes + 4 * hk].view(np.float32)
    amax0 = np.abs(O.decode(O.BF16, b0)).max(axis=2)[0]
    assert np.array_equal(sc, (amax0 / np.float32(448.0)).astype(np.float32))
    row0 = kreg[:hk * d].reshape(hk, d)
    assert (np.abs(O.decode(O.FP8, row0)).max(axis=1) == 448).all()   # amax maps to 448
    deq0 = O.decode(O.FP8, row0) * sc[:, None]
    assert np.allclose(deq0, O.decode(O.BF16, b0)[0], rtol=2 ** -3, atol=0)

    x1 = x0 * 4  # every head grows: forces re-encoding of slot 0
    b1 = O.encode(O.BF16, x1)
    O.kv_write_rows(O.FP8, kreg, vreg, b1, b1, [0], [1], [0], hk, d, row_bytes, data_bytes)
    sc1 = kreg[data_bytes:data_bytes + 4 * hk].view(np.float32)
    amax1 = np.abs(O.decode(O.BF16, b1)).max(axis=2)[0]
    assert np.array_equal(sc1, (amax1 / np.float32(448.0)).astype(np.float32))
    re0 = O.encode(O.FP8, (O.decode(O.FP8, row0) * sc[:, None]) / sc1[:, None])
    assert np.array_equal(kreg[:hk * d].reshape(hk, d), re0)

    x2 = x0 * 0.5  # smaller row: scale unchanged, earlier rows untouched
    before = kreg.copy()
    b2 = O.encode(O.BF16, x2)
    O.kv_write_rows(O.FP8, kreg, vreg, b2, b2, [0], [2], [0], hk, d, row_bytes, data_bytes)
    assert np.array_equal(kreg[:2 * row_bytes], before[:2 * row_bytes])
    assert np.array_equal(kreg[data_bytes:data_bytes + 8], before[data_bytes:data_bytes + 8])


def test_copy_pages_moves_whole_pages(oracle_lib):
    regs = [np.arange(4 * 64, dtype=np.uint8).copy() for _ in range(3)]
    O.copy_pages(regs, [[0, 128], [64, 192]], 64)
    for r in regs:
        assert np.array_equal(r[128:192], np.arange(64, dtype=np.uint8))
        assert np.array_equal(r[192:256], np.arange(64, 128, dtype=np.uint8))
