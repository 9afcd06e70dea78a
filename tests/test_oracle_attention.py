"""Pins the oracle's paged decode attention.

* against an independent dense two-pass softmax in numpy (no pages, no
  online recurrence): catches addressing, GQA-map, scale and softmax errors;
* the reference's KAT: seq_len 1 returns the mapped V row exactly (ref
  scripts/kcmm/non_default_stream_ffi_smoke.py:172-179,334-343);
* closed forms: q = 0 gives the mean of V; a dominant key selects its V;
  permuting the page placement changes nothing; seq_len <= 0 gives zeros;
* the reference kernel's own fp32 loop (the CPU baseline) within the fp32
  tolerance of 1e-5 relative.
"""
import numpy as np
import pytest

import oracle as O
from tests.paged import dense_reference, layout


def run_oracle(lay, q, hq, hkv, d, bs, dtype, scale):
    return O.attn_decode_f64(dtype, q, lay["k_region"], lay["v_region"], lay["block_tables"],
                             lay["seq_lens"], lay["offsets"], hq, hkv, d, bs, lay["row_bytes"],
                             lay["data_bytes"], scale)


def qbits(dtype, x):
    return O.encode(O.F16 if dtype == O.F16 else (O.F32 if dtype == O.F32 else O.BF16), x)


@pytest.mark.parametrize("dtype", [O.F16, O.BF16, O.FP8, O.F32])
@pytest.mark.parametrize("hq,hkv,d,bs", [(8, 8, 64, 16), (32, 8, 128, 16), (6, 4, 80, 8),
                                         (4, 1, 256, 32)])
def test_matches_dense_softmax(oracle_lib, dtype, hq, hkv, d, bs):
    ctx = [1, 17, 40, 0, 95]
    lay = layout(len(ctx), ctx, hkv, d, bs, dtype, seed=hq + d + dtype)
    rng = np.random.default_rng(7)
    qf = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    q = qbits(dtype, qf)
    qd = O.decode(O.F16 if dtype == O.F16 else (O.F32 if dtype == O.F32 else O.BF16), q)
    scale = 1 / np.sqrt(d)
    got = run_oracle(lay, q, hq, hkv, d, bs, dtype, scale)
    ref = dense_reference(qd, lay["dense_k"], lay["dense_v"], hq, hkv, scale)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    assert not got[3].any()                               # seq_len 0 -> zeros


def test_seq_len_one_returns_v_row_exactly(oracle_lib):
    # ref non_default_stream_ffi_smoke.py: q = 0, v = arange + 1000, torch.equal
    hq, hkv, d, bs = 4, 2, 8, 4
    lay = layout(1, [1], hkv, d, bs, O.F16, seed=3)
    page = int(lay["block_tables"][0, 0]) * lay["block_bytes"]
    v = (np.arange(hkv * d, dtype=np.float32) + 1000).astype(np.float16)
    lay["v_region"][page:page + v.nbytes] = v.view(np.uint8)
    q = np.zeros((1, hq, d), np.uint16)
    got = run_oracle(lay, q, hq, hkv, d, bs, O.F16, 1.0)
    expect = np.stack([v.reshape(hkv, d)[h * hkv // hq] for h in range(hq)]).astype(np.float64)
    assert np.array_equal(got[0], expect)


def test_zero_query_gives_mean_of_values_per_kv_head(oracle_lib):
    hq, hkv, d, bs = 8, 2, 16, 16
    ctx = [33, 5]
    lay = layout(2, ctx, hkv, d, bs, O.BF16, seed=4)
    got = run_oracle(lay, np.zeros((2, hq, d), np.uint16), hq, hkv, d, bs, O.BF16, 0.3)
    for b in range(2):
        for h in range(hq):
            assert np.allclose(got[b, h], lay["dense_v"][b][:, h // 4, :].mean(axis=0),
                               rtol=1e-12, atol=1e-12)


def test_dominant_key_selects_its_value(oracle_lib):
    hq, hkv, d, bs = 2, 1, 32, 16
    lay = layout(1, [50], hkv, d, bs, O.F32, seed=5)
    k = lay["dense_k"][0][:, 0, :]
    q = (k[37] * 1e4).astype(np.float32)[None, None, :].repeat(2, axis=1)
    got = run_oracle(lay, q, hq, hkv, d, bs, O.F32, 1.0)
    assert np.allclose(got[0, 0], lay["dense_v"][0][37, 0], rtol=0, atol=1e-9)


def test_page_placement_does_not_matter(oracle_lib):
    hq, hkv, d, bs = 8, 4, 64, 16
    ctx = [70, 16, 3]
    a = layout(3, ctx, hkv, d, bs, O.BF16, seed=9, shuffle=True)
    b = layout(3, ctx, hkv, d, bs, O.BF16, seed=9, shuffle=False)
    q = O.encode(O.BF16, np.random.default_rng(1).standard_normal((3, hq, d)))
    ra = run_oracle(a, q, hq, hkv, d, bs, O.BF16, 0.125)
    rb = run_oracle(b, q, hq, hkv, d, bs, O.BF16, 0.125)
    assert not np.array_equal(a["block_tables"], b["block_tables"])
    assert np.array_equal(ra, rb)


@pytest.mark.parametrize("dtype", [O.F16, O.BF16, O.F32])
def test_reference_loop_within_fp32_tolerance(oracle_lib, dtype):
    hq, hkv, d, bs = 8, 8, 64, 16                         # BASELINE configs[0] shape
    rng = np.random.default_rng(11)
    ctx = rng.integers(1, 513, size=4) + 1
    lay = layout(4, ctx, hkv, d, bs, dtype, seed=12)
    q = qbits(dtype, rng.standard_normal((4, hq, d)))
    scale = 1 / np.sqrt(d)
    ref = run_oracle(lay, q, hq, hkv, d, bs, dtype, scale)
    got = O.attn_decode_ref_f32(dtype, q, lay["k_region"], lay["v_region"], lay["block_tables"],
                                lay["seq_lens"], lay["offsets"], hq, hkv, d, bs,
                                lay["row_bytes"], scale, threads=4)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err <= 1e-5, err
