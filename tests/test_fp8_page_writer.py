"""fp8 page writer: properties that do not restate the writer's formula.

The contract (include/kcmm_mi355x.h, kcmm_pool_create_typed) says the rows one
call writes into a page act as one set, so the page bytes must not depend on
the order of the rows, and every live row must decode -- e4m3 code times the
page's per-kv-head footer scale -- to its bf16 input within the e4m3 grid:
at most one e4m3 step (2^-3 relative for normals, 2^-9 * scale below 2^-6 *
scale) per rounding, and a row is rounded at most twice here (written, then
re-encoded once when a later call raises the scale).  The decoder and the
bf16 encoder used to check this are torch's float8_e4m3fn / bfloat16 casts,
independent of the oracle's codecs.  The rows of the cases that used to fail
(order [3, 0] with slot 3 at 8x; [0, 5, 2] with slot 2 at 8x; a first write
at slot > 0 on a zero footer) are included by name.
"""
import numpy as np
import pytest
import torch

import oracle as O

HK, D, BS = 2, 64, 16
ROW = HK * D                      # fp8 row bytes
DATA = ROW * BS                   # page data bytes; footer follows
PAGE = ((DATA + 4 * HK + 255) // 256) * 256


def bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16) \
        .view(torch.int16).numpy().view(np.uint16)


def bf16_value(bits):
    return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()


def e4m3_value(codes):
    return torch.from_numpy(np.ascontiguousarray(codes)).view(torch.float8_e4m3fn).float().numpy()


def scales(region, page):
    return region[page * PAGE + DATA:page * PAGE + DATA + 4 * HK].view(np.float32).copy()


def row_value(region, page, slot):
    a = page * PAGE + slot * ROW
    return e4m3_value(region[a:a + ROW].reshape(HK, D)) * scales(region, page)[:, None]


def write(path, kreg, vreg, pages, slots, bits):
    """One call: row i goes to (pages[i], slots[i]); bits [2][n][HK*D]."""
    n = len(pages)
    if path == "host":
        O.kv_write_rows(O.FP8, kreg, vreg, bits[0], bits[1], [p * PAGE for p in pages], slots,
                        list(range(n)), HK, D, ROW, DATA)
    else:
        offs = np.arange(kreg.size // PAGE, dtype=np.uint64) * (PAGE // 2)
        st = O.kv_write_device_slots(O.FP8, kreg, vreg, bits[0], bits[1],
                                     [p * BS + s for p, s in zip(pages, slots)], offs, None, BS,
                                     HK, D, ROW, DATA)
        assert st == 0


def check_rows(kreg, live):
    """live: {(page, slot): bf16 input [HK][D] as float}."""
    for (page, slot), x in live.items():
        s = scales(kreg, page)
        got = row_value(kreg, page, slot)
        bound = 2.0 ** -3 * np.abs(x) + 2.0 ** -9 * s[:, None]
        assert np.all(np.abs(got - x) <= bound * (1 + 1e-6)), (page, slot)
        # no value clipped: every live element fits the e4m3 range at this scale
        assert np.all(np.abs(x) <= 448.0 * s[:, None] * (1 + 1e-6)), (page, slot)
    for page in {p for p, _ in live}:
        assert np.all(np.isfinite(scales(kreg, page))) and np.all(scales(kreg, page) > 0)


@pytest.mark.parametrize("path", ["host", "device"])
def test_named_cases(oracle_lib, path):
    rng = np.random.default_rng(1)
    cases = [([3, 0], {3: 8.0}), ([0, 5, 2], {2: 8.0}), ([7], {}), ([4, 9], {4: 0.0})]
    for order, mag in cases:
        kreg = np.zeros(2 * PAGE, np.uint8)
        vreg = np.zeros_like(kreg)
        x = rng.standard_normal((2, len(order), ROW)).astype(np.float32)
        for i, s in enumerate(order):
            x[:, i] *= mag.get(s, 1.0)
        bits = bf16_bits(x)
        if order == [0, 5, 2]:
            # slot 0 and 5 in one call, slot 2 in the next: the scale grows
            # and slot 5 (after slot 2) must be re-encoded too
            write(path, kreg, vreg, [1, 1], [0, 5], bits[:, :2])
            write(path, kreg, vreg, [1], [2], bits[:, 2:])
        else:
            write(path, kreg, vreg, [1] * len(order), order, bits)
        live = {(1, s): bf16_value(bits[0, i]).reshape(HK, D) for i, s in enumerate(order)}
        check_rows(kreg, live)
        livev = {(1, s): bf16_value(bits[1, i]).reshape(HK, D) for i, s in enumerate(order)}
        check_rows(vreg, livev)


def _call_rows(rng, n_pages, order, start_slot=0, count=BS):
    rows = [(p, s) for p in range(n_pages) for s in range(start_slot, start_slot + count)]
    if order == "interleaved":
        rows = [(p, s) for s in range(start_slot, start_slot + count) for p in range(n_pages)]
    elif order == "reversed":
        rows = rows[::-1]
    elif order == "shuffled":
        rows = [rows[i] for i in rng.permutation(len(rows))]
    return rows


@pytest.mark.parametrize("path", ["host", "device"])
def test_bytes_do_not_depend_on_row_order(oracle_lib, path):
    """The same set of rows, in four orders, over two calls (the second one
    continues the pages from slot 6 and grows some scales): identical bytes,
    and every live row decodes within the grid bound."""
    rng = np.random.default_rng(7)
    n_pages = 4
    first = {(p, s): None for p in range(n_pages) for s in range(6)}
    second = {(p, s): None for p in range(n_pages) for s in range(6, BS)}
    vals = {}
    for key in list(first) + list(second):
        m = 8.0 if rng.random() < 0.2 else 1.0
        vals[key] = (rng.standard_normal((2, ROW)) * m).astype(np.float32)
    results = []
    for order in ["seq", "interleaved", "reversed", "shuffled"]:
        kreg = np.zeros(n_pages * PAGE, np.uint8)
        vreg = np.zeros_like(kreg)
        for start, count in [(0, 6), (6, BS - 6)]:
            rows = _call_rows(rng, n_pages, order, start, count)
            bits = bf16_bits(np.stack([vals[r] for r in rows], axis=1))
            write(path, kreg, vreg, [p for p, _ in rows], [s for _, s in rows], bits)
        results.append((kreg, vreg))
        live = {key: bf16_value(bf16_bits(v[0])).reshape(HK, D) for key, v in vals.items()}
        check_rows(kreg, live)
    for kreg, vreg in results[1:]:
        assert np.array_equal(kreg, results[0][0]) and np.array_equal(vreg, results[0][1])


@pytest.mark.parametrize("path", ["host", "device"])
def test_repeated_slot_keeps_the_last_row(oracle_lib, path):
    rng = np.random.default_rng(3)
    kreg = np.zeros(PAGE, np.uint8)
    vreg = np.zeros_like(kreg)
    slots = [0, 4, 2, 4, 9, 0]
    x = rng.standard_normal((2, len(slots), ROW)).astype(np.float32)
    x[:, 1] *= 8.0                       # the superseded row of slot 4 is large
    bits = bf16_bits(x)
    write(path, kreg, vreg, [0] * len(slots), slots, bits)
    last = {s: i for i, s in enumerate(slots)}
    live = {(0, s): bf16_value(bits[0, i]).reshape(HK, D) for s, i in last.items()}
    check_rows(kreg, live)
    # the superseded row takes no part in the scale
    amax = np.max([np.abs(v).max(axis=1) for v in live.values()], axis=0)
    assert np.allclose(scales(kreg, 0), amax / 448.0, rtol=1e-6)


@pytest.mark.parametrize("path", ["host", "device"])
def test_slot0_restarts_and_zero_rows(oracle_lib, path):
    """A call that writes slot 0 starts the page: the scale comes from that
    call's rows only, even when the old scale was far larger; an all-zero
    first row gives scale 1 and zero codes."""
    rng = np.random.default_rng(11)
    kreg = np.zeros(PAGE, np.uint8)
    vreg = np.zeros_like(kreg)
    big = bf16_bits((rng.standard_normal((2, 3, ROW)) * 100).astype(np.float32))
    write(path, kreg, vreg, [0, 0, 0], [0, 1, 2], big)
    small = bf16_bits((rng.standard_normal((2, 2, ROW)) * 0.01).astype(np.float32))
    write(path, kreg, vreg, [0, 0], [1, 0], small)
    live = {(0, 1): bf16_value(small[0, 0]).reshape(HK, D),
            (0, 0): bf16_value(small[0, 1]).reshape(HK, D)}
    check_rows(kreg, live)
    assert np.all(scales(kreg, 0) < 1e-3)
    zero = np.zeros((2, 1, ROW), np.uint16)
    write(path, kreg, vreg, [0], [0], zero)
    assert np.all(scales(kreg, 0) == 1.0)
    assert not kreg[:ROW].any()
