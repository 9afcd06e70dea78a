"""Pins the oracle GEMM (Y = X W^T, ref llama_transformer.rs:115-120) against
numpy's BLAS matmul in float64, plus identity / transposition closed forms.
(The reference's own arithmetic sits in cuBLAS via cudarc 0.11.9 and has no
value-level test at that boundary; see the parity notes.)"""
import numpy as np

import oracle as O


def test_matches_numpy(oracle_lib):
    rng = np.random.default_rng(0)
    x = O.encode(O.BF16, rng.standard_normal((37, 192)))
    w = O.encode(O.BF16, rng.standard_normal((70, 192)) * 0.02)
    got = O.gemm_bf16_f64(x, w)
    ref = O.decode(O.BF16, x).astype(np.float64) @ O.decode(O.BF16, w).astype(np.float64).T
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


def test_identity_weight_copies_input(oracle_lib):
    rng = np.random.default_rng(1)
    x = O.encode(O.BF16, rng.standard_normal((5, 64)))
    eye = O.encode(O.BF16, np.eye(64))
    assert np.array_equal(O.gemm_bf16_f64(x, eye), O.decode(O.BF16, x).astype(np.float64))


def test_operand_order_is_x_times_w_transposed(oracle_lib):
    # a transposed operand would give W X^T; with a non-square W it must not
    x = O.encode(O.BF16, np.array([[1, 2, 3, 4]], np.float32))
    w = O.encode(O.BF16, np.array([[1, 0, 0, 0], [0, 0, 0, 1]], np.float32))
    assert O.gemm_bf16_f64(x, w).tolist() == [[1.0, 4.0]]


def test_fp8_weights_match_numpy_over_torch_decode(oracle_lib):
    """The fp8-weight oracle against numpy fp64 over torch's float8_e4m3fn
    decode of the codes, with the row scales applied after the sum."""
    import torch
    rng = np.random.default_rng(3)
    x = O.encode(O.BF16, rng.standard_normal((19, 256)))
    w8, s = O.quantize_fp8_rows(rng.standard_normal((48, 256)) * 0.02)
    wd = torch.from_numpy(w8).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    ref = (O.decode(O.BF16, x).astype(np.float64) @ wd.T) * s.astype(np.float64)[None, :]
    assert np.allclose(O.gemm_fp8w_f64(x, w8, s), ref, rtol=1e-12, atol=1e-12)


def test_fp8_weights_equal_bf16_oracle_on_exact_values(oracle_lib):
    """Every e4m3 value is a bf16 value: with unit scales the fp8-weight
    product equals the (pinned) bf16 product of the same weights exactly;
    a scale of 2 doubles it exactly; a planted swap of two codes fails."""
    rng = np.random.default_rng(4)
    x = O.encode(O.BF16, rng.standard_normal((8, 128)))
    w8 = rng.integers(0, 256, size=(32, 128), dtype=np.uint8)
    w8[(w8 & 0x7F) == 0x7F] = 0x00                    # no NaN codes
    wb = O.encode(O.BF16, O.decode(O.FP8, w8))
    one = np.ones(32, np.float32)
    y8 = O.gemm_fp8w_f64(x, w8, one)
    assert np.array_equal(y8, O.gemm_bf16_f64(x, wb))
    assert np.array_equal(O.gemm_fp8w_f64(x, w8, one * 2), 2 * y8)
    w_bad = w8.copy()
    w_bad[:, [0, 1]] = w_bad[:, [1, 0]]
    assert not np.array_equal(O.gemm_fp8w_f64(x, w_bad, one), y8)


def test_row_quantizer_round_trip(oracle_lib):
    """quantize_fp8_rows: the row's amax maps to 448 exactly; dequantized
    values stay within half an e4m3 step (2^-4 relative) of the input."""
    rng = np.random.default_rng(5)
    w = rng.standard_normal((16, 64)).astype(np.float32) * 0.05
    w8, s = O.quantize_fp8_rows(w)
    deq = O.decode(O.FP8, w8).astype(np.float64) * s[:, None]
    assert np.all(np.abs(O.decode(O.FP8, w8)).max(axis=1) == 448.0)
    assert np.all(np.abs(deq - w) <= np.abs(w) * 2 ** -4 + s[:, None] * 2 ** -9)
