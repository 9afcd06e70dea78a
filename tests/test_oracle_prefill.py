"""Pins the oracle's causal chunked-prefill attention (the north star's
extension; the reference prefills one token per decode step, ref
src/model/transformer.rs:50-65, so there is no reference value to match):

* against an independent dense causal softmax in numpy over the stored K/V;
* a chunk of one token is exactly the decode oracle at the same length;
* q = 0 gives, for each query, the mean of V over keys 0..p (closed form);
* page placement does not change the result.
"""
import numpy as np
import pytest

import oracle as O
from tests.paged import layout


def chunk_setup(ctx, lens, hkv, d, bs, dtype, seed):
    lay = layout(len(ctx), ctx, hkv, d, bs, dtype, seed=seed)
    qsl = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    return lay, qsl


def run(lay, qsl, q, hq, hkv, d, bs, dtype, scale):
    return O.attn_prefill_f64(dtype, q, lay["k_region"], lay["v_region"], lay["block_tables"],
                              lay["seq_lens"], qsl, lay["offsets"], hq, hkv, d, bs,
                              lay["row_bytes"], lay["data_bytes"], scale)


def dense_causal(qd, lay, qsl, hq, hkv, scale):
    out = np.zeros(qd.shape)
    for b in range(len(lay["dense_k"])):
        K, V = lay["dense_k"][b], lay["dense_v"][b]
        n = qsl[b + 1] - qsl[b]
        for i in range(n):
            p = K.shape[0] - n + i
            for h in range(hq):
                g = h * hkv // hq
                s = K[:p + 1, g, :] @ qd[qsl[b] + i, h].astype(np.float64) * scale
                w = np.exp(s - s.max())
                out[qsl[b] + i, h] = (w / w.sum()) @ V[:p + 1, g, :]
    return out


@pytest.mark.parametrize("dtype", [O.BF16, O.F16, O.FP8, O.F32])
@pytest.mark.parametrize("hq,hkv,d,bs", [(8, 2, 64, 16), (32, 8, 128, 16), (4, 4, 32, 8)])
def test_matches_dense_causal_softmax(oracle_lib, dtype, hq, hkv, d, bs):
    ctx = [40, 17, 70, 1]
    lens = [13, 17, 32, 1]           # a chunk may be the whole sequence
    lay, qsl = chunk_setup(ctx, lens, hkv, d, bs, dtype, seed=hq + d + dtype)
    rng = np.random.default_rng(11)
    qdt = dtype if dtype in (O.F16, O.F32) else O.BF16
    q = O.encode(qdt, rng.standard_normal((qsl[-1], hq, d)).astype(np.float32))
    scale = 1 / np.sqrt(d)
    got = run(lay, qsl, q, hq, hkv, d, bs, dtype, scale)
    ref = dense_causal(O.decode(qdt, q), lay, qsl, hq, hkv, scale)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_chunk_of_one_is_decode(oracle_lib):
    hq, hkv, d, bs = 16, 4, 64, 16
    ctx = [33, 5, 100]
    lay, qsl = chunk_setup(ctx, [1, 1, 1], hkv, d, bs, O.BF16, seed=12)
    rng = np.random.default_rng(12)
    q = O.encode(O.BF16, rng.standard_normal((3, hq, d)).astype(np.float32))
    got = run(lay, qsl, q, hq, hkv, d, bs, O.BF16, 0.2)
    dec = O.attn_decode_f64(O.BF16, q, lay["k_region"], lay["v_region"], lay["block_tables"],
                            lay["seq_lens"], lay["offsets"], hq, hkv, d, bs, lay["row_bytes"],
                            lay["data_bytes"], 0.2)
    assert np.array_equal(got, dec)


def test_zero_query_gives_prefix_means(oracle_lib):
    hq, hkv, d, bs = 4, 2, 16, 8
    ctx, lens = [20], [20]
    lay, qsl = chunk_setup(ctx, lens, hkv, d, bs, O.F32, seed=13)
    got = run(lay, qsl, np.zeros((20, hq, d), np.float32), hq, hkv, d, bs, O.F32, 1.0)
    V = lay["dense_v"][0]
    for i in range(20):
        for h in range(hq):
            assert np.allclose(got[i, h], V[:i + 1, h * hkv // hq].mean(axis=0), rtol=1e-12, atol=1e-12)


def test_page_placement_does_not_matter(oracle_lib):
    hq, hkv, d, bs = 8, 2, 32, 16
    ctx, lens = [50, 31], [20, 31]
    qsl = np.array([0, 20, 51], np.int32)
    a = layout(2, ctx, hkv, d, bs, O.BF16, seed=14, shuffle=True)
    b = layout(2, ctx, hkv, d, bs, O.BF16, seed=14, shuffle=False)
    q = O.encode(O.BF16, np.random.default_rng(14).standard_normal((51, hq, d)).astype(np.float32))
    assert np.array_equal(run(a, qsl, q, hq, hkv, d, bs, O.BF16, 0.3),
                          run(b, qsl, q, hq, hkv, d, bs, O.BF16, 0.3))
