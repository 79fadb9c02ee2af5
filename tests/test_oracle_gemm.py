"""Pins the GEMM and epilogue parts of the CPU oracle without the GPU.

  * int32 accumulators against numpy's int64 matmul (brute force, exact);
  * the epilogue against the fp64 closed form ((acc * as) * ws) + bias within
    the bf16 output rounding (w4a8.cu:480-525, bindings.cpp:379-383), and with
    the bias term, the per-row and per-column scales each perturbed to show the
    check notices a dropped or transposed term;
  * the scalar weight-scale form of dequantize_int8_bf16 (bf16_epilogue.cu:105-119).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (7, 13, 48), (64, 96, 1536), (5, 8, 13824)])
def test_int_gemm_matches_numpy(m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    ref = a.astype(np.int64) @ w.astype(np.int64).T
    np.testing.assert_array_equal(oracle.int8_gemm_i32(a, w), ref.astype(np.int32))


def test_int_gemm_extreme_accumulator():
    a = np.full((2, 13824), -128, np.int8)
    assert int(oracle.int8_gemm_i32(a, a).max()) == 16384 * 13824


def _bf16_to_f64(bits):
    return oracle.bf16_bits_to_f32(bits).astype(np.float64).reshape(bits.shape)


@pytest.mark.parametrize("with_bias", [True, False])
def test_epilogue_closed_form(with_bias):
    rng = np.random.default_rng(5)
    m, n = 33, 40
    acc = rng.integers(-(2 ** 28), 2 ** 28, (m, n)).astype(np.int32)
    as_ = rng.uniform(1e-4, 1e-2, m).astype(np.float32)
    ws = rng.uniform(1e-3, 5e-3, n).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.02).astype(np.float32) if with_bias else None
    out = _bf16_to_f64(oracle.epilogue_bf16(acc, as_, ws, bias))
    exact = acc.astype(np.float64) * as_[:, None] * ws[None, :] + (0 if bias is None else bias[None, :])
    tol = np.abs(exact) * 2.0 ** -8 + 1e-30
    assert np.all(np.abs(out - exact) <= tol)
    # perturbations the check must notice
    wrong = [acc.astype(np.float64) * as_[:, None] * ws[None, :] * 1.01]
    if bias is not None:
        wrong.append(acc.astype(np.float64) * as_[:, None] * ws[None, :])
    for w_ in wrong:
        assert np.any(np.abs(out - w_) > np.abs(w_) * 2.0 ** -8 + 1e-30)


def test_epilogue_scalar_weight_scale_and_column_slice():
    rng = np.random.default_rng(6)
    acc = rng.integers(-(2 ** 20), 2 ** 20, (9, 24)).astype(np.int32)
    as_ = rng.uniform(1e-3, 1e-2, 9).astype(np.float32)
    ws = np.array([3e-3], np.float32)
    out = _bf16_to_f64(oracle.epilogue_bf16(acc, as_, ws, None, cols=17))
    exact = acc[:, :17].astype(np.float64) * as_[:, None] * 3e-3
    assert out.shape == (9, 17)
    assert np.all(np.abs(out - exact) <= np.abs(exact) * 2.0 ** -8 + 1e-30)
