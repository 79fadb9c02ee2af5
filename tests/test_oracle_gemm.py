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


def _bf16_rne(x64: np.ndarray) -> np.ndarray:
    """fp64 -> fp32 (one rounding) -> bf16 bits by round-to-nearest-even on the fp32 pattern."""
    u = np.asarray(x64, np.float64).astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("gate_rows,gated", [(1, True), (37, True), (1, False)])
def test_residual_gate_closed_form(gate_rows, gated):
    """bf16 y * g is exact in fp64 and fp32, so fma(y, g, r) in fp32 is the fp64
    sum rounded once to fp32, then to bf16; a gate indexed by i % rows, a dropped
    gate or a dropped residual must all show."""
    rng = np.random.default_rng(gate_rows + 7 * gated)
    m, n = 131, 48
    y = oracle.f32_to_bf16_bits(rng.standard_normal((m, n)).astype(np.float32)).reshape(m, n)
    r = oracle.f32_to_bf16_bits((rng.standard_normal((m, n)) * 4).astype(np.float32)).reshape(m, n)
    rows = (m + gate_rows - 1) // gate_rows
    g = oracle.f32_to_bf16_bits(rng.uniform(-2, 2, (rows, n)).astype(np.float32)).reshape(rows, n) if gated else None
    out = oracle.residual_gate_bf16(y, r, g, gate_rows)
    yf, rf = _bf16_to_f64(y), _bf16_to_f64(r)
    gf = np.ones((m, n)) if g is None else _bf16_to_f64(g)[np.arange(m) // gate_rows]
    np.testing.assert_array_equal(out, _bf16_rne(yf * gf + rf))
    wrong = [_bf16_rne(yf * gf), _bf16_rne(rf)]
    if g is not None:
        wrong.append(_bf16_rne(yf + rf))
    if g is not None and gate_rows > 1:
        wrong.append(_bf16_rne(yf * _bf16_to_f64(g)[np.arange(m) % rows] + rf))
    for w_ in wrong:
        assert np.any(out != w_)


def _edge_epilogue_inputs():
    """Accumulators, scales and bias that reach every fp16 class: ordinary
    values, results past 65504 (overflow to +-inf, and the 65504 / 65520
    rounding boundary), fp16 subnormals and underflow to +-0, plus inf and NaN
    scales and bias (NaN results)."""
    rng = np.random.default_rng(17)
    m, n = 40, 64
    acc = rng.integers(-(2 ** 24), 2 ** 24, (m, n)).astype(np.int32)
    acc[:, 0] = 1
    acc[:, 1] = -1
    acc[:, 2] = 0
    as_ = rng.uniform(1e-4, 1e-2, m).astype(np.float32)
    as_[3] = 1.0          # acc * ws straight: large values
    as_[4] = 1e-9         # subnormal and zero results
    as_[5] = np.float32(np.inf)
    as_[6] = np.float32(np.nan)
    ws = rng.uniform(1e-3, 5e-3, n).astype(np.float32)
    ws[3] = 65504.0
    ws[4] = 65519.996
    ws[5] = 65520.0
    ws[6] = 0.0
    ws[7] = -0.0
    bias = (rng.standard_normal(n) * 0.02).astype(np.float32)
    bias[8] = np.float32(np.nan)
    bias[9] = np.float32(-np.inf)
    acc[3, 3:6] = 1       # 65504, 65519.996 (rounds to 65504), 65520 (rounds to inf)
    acc[3, 10] = 70000    # as 1 * 70000 * ws: past 65520 before the bias
    ws[10] = 1.0
    return acc, as_, ws, bias


@pytest.mark.parametrize("with_bias", [True, False])
def test_epilogue_f32_and_f16_match_numpy(with_bias):
    """The fp32 output is numpy's float32 (acc * as) * ws + bias, one IEEE
    operation at a time (bit-exact, NaN positions equal); the fp16 output is
    numpy's float16 cast of that value with every NaN as 0x7e00.  Both are
    independent of the C code; a swapped multiplication order or a double
    rounding through bf16 must show."""
    acc, as_, ws, bias = _edge_epilogue_inputs()
    b = bias if with_bias else None
    with np.errstate(all="ignore"):
        v = (acc.astype(np.float32) * as_[:, None]) * ws[None, :]
        if b is not None:
            v = v + b[None, :]
        f32 = oracle.epilogue_f32(acc, as_, ws, b)
        nan = np.isnan(v)
        np.testing.assert_array_equal(np.isnan(f32), nan)
        np.testing.assert_array_equal(f32.view(np.uint32)[~nan], v.view(np.uint32)[~nan])
        f16 = oracle.epilogue_f16(acc, as_, ws, b)
        ref16 = v.astype(np.float16).view(np.uint16).copy()
        ref16[nan] = 0x7E00
        np.testing.assert_array_equal(f16, ref16)
        # every class is reached
        h = f16[~nan].view(np.float16)
        assert np.isinf(h).any() and (h == 65504).any() and (f16 == 0x7E00).any()
        if b is None:  # (a bias of ~0.02 keeps every result normal)
            assert (f16[~nan] & 0x7FFF == 0).any()
            assert (((f16 & 0x7C00) == 0) & ((f16 & 0x3FF) != 0)).any()  # fp16 subnormals
        # plausible mistakes
        swapped = ((acc.astype(np.float32) * ws[None, :]) * as_[:, None])
        if b is not None:
            swapped = swapped + b[None, :]
        assert np.any(swapped.view(np.uint32)[~nan] != f32.view(np.uint32)[~nan])
        via_bf16 = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(v)).reshape(v.shape).astype(np.float16)
        assert np.any(via_bf16.view(np.uint16)[~nan] != f16[~nan])


def test_epilogue_f16_scalar_weight_scale_and_slice():
    rng = np.random.default_rng(19)
    acc = rng.integers(-(2 ** 20), 2 ** 20, (9, 24)).astype(np.int32)
    as_ = rng.uniform(1e-3, 1e-2, 9).astype(np.float32)
    ws = np.array([3e-3], np.float32)
    out = oracle.epilogue_f16(acc, as_, ws, None, cols=17)
    v = (acc[:, :17].astype(np.float32) * as_[:, None]) * np.float32(3e-3)
    np.testing.assert_array_equal(out, v.astype(np.float16).view(np.uint16))
