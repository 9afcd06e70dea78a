"""Pins the oracle's numeric formats against library routines.

bf16 and float8_e4m3fn against torch's dtype casts, IEEE half against numpy's
float16 cast -- independent implementations of the same published formats.
A dropped rounding bit, a wrong exponent bias or a mishandled subnormal fails
one of these exhaustive or tie-targeted checks.
"""
import numpy as np
import pytest
import torch

import oracle as O


def _ties_and_randoms(seed=0, n=200_000):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32) * np.float32(4.0)
    # exact ties for bf16 (low 16 bits = 0x8000) and f16 (low 13 bits = 0x1000)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    bf_ties = ((bits & np.uint32(0xFFFF0000)) | np.uint32(0x8000)).view(np.float32)
    f16_ties = ((bits & np.uint32(0xFFFFE000)) | np.uint32(0x1000)).view(np.float32)
    return np.concatenate([x, bf_ties, f16_ties])


def test_bf16_decode_all_codes(oracle_lib):
    codes = np.arange(65536, dtype=np.uint16)
    ours = O.decode(O.BF16, codes)
    ref = torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32)[~np.isnan(ref)], ref.view(np.uint32)[~np.isnan(ref)])
    assert np.isnan(ours[np.isnan(ref)]).all()


def test_bf16_encode_matches_torch(oracle_lib):
    x = _ties_and_randoms()
    x = x[np.isfinite(x)]
    ours = O.encode(O.BF16, x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite = np.isfinite(torch.from_numpy(x).to(torch.bfloat16).float().numpy())
    assert np.array_equal(ours[finite], ref[finite])


def test_f16_decode_all_codes(oracle_lib):
    codes = np.arange(65536, dtype=np.uint16)
    ours = O.decode(O.F16, codes)
    ref = codes.view(np.float16).astype(np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.isnan(ours[~ok]).all()


def test_f16_encode_matches_numpy(oracle_lib):
    x = _ties_and_randoms(1)
    # subnormal range and overflow boundary
    extra = np.array([6e-8, 5.96e-8, 2.98e-8, 2.99e-8, 6.1e-5, 6.09e-5, 65504, 65519.9, 65520,
                      70000, -0.0, 1e-30], dtype=np.float32)
    with np.errstate(invalid="ignore"):
        x = np.concatenate([x, extra, x * np.float32(1e-5)])
    nan = np.isnan(x)
    ours = O.encode(O.F16, x)
    with np.errstate(over="ignore"):
        ref = x[~nan].astype(np.float16).view(np.uint16)
    assert np.array_equal(ours[~nan], ref)
    # NaN stays NaN (payloads are not part of the contract)
    assert ((ours[nan] & 0x7C00) == 0x7C00).all() and ((ours[nan] & 0x3FF) != 0).all()


def test_e4m3_decode_all_codes(oracle_lib):
    codes = np.arange(256, dtype=np.uint8)
    ours = O.decode(O.FP8, codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok], ref[ok])
    assert np.isnan(ours[~ok]).all() and (~ok).sum() == 2  # 0x7f and 0xff only


def test_e4m3_encode_matches_torch_in_range(oracle_lib):
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(100_000) * 100, rng.standard_normal(50_000) * 0.01,
                        # midpoints between consecutive codes -> RNE ties
                        (O.decode(O.FP8, np.arange(0, 126, dtype=np.uint8))[:-1] +
                         O.decode(O.FP8, np.arange(1, 126, dtype=np.uint8))) / 2]).astype(np.float32)
    x = x[np.abs(x) < 464]  # torch turns values past the max-finite rounding point into NaN
    ours = O.encode(O.FP8, x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)


def test_e4m3_saturates(oracle_lib):
    x = np.array([448, 460, 464, 1000, 1e30, -500, -1e30], dtype=np.float32)
    assert O.encode(O.FP8, x).tolist() == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE]
    assert O.encode(O.FP8, np.array([np.nan], np.float32))[0] & 0x7F == 0x7F


@pytest.mark.parametrize("dt", [O.F16, O.BF16, O.FP8])
def test_roundtrip_of_representable_values_is_identity(oracle_lib, dt):
    n = {O.F16: 65536, O.BF16: 65536, O.FP8: 256}[dt]
    codes = np.arange(n, dtype=np.uint16 if dt != O.FP8 else np.uint8)
    vals = O.decode(dt, codes)
    ok = np.isfinite(vals) & ~((vals == 0) & (codes != 0))  # skip NaN/inf and -0
    assert np.array_equal(O.encode(dt, vals[ok]), codes[ok])
