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
