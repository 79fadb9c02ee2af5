"""Pins the Sage part of the CPU oracle without the GPU.

  * K mean: within one bf16 step of the fp64 mean;
  * block quantizer: scale == amax / 127 recomputed in numpy, max |code| == 127,
    dequantization error <= half a step, round-half-even and saturation;
  * attention: against fp64 softmax on the dequantized inputs (the only
    difference is P rounded to bf16), against fp32 SDPA on the raw inputs with
    the reference's own gate (rtol 0.08 / atol 0.06, validate_compatible.py
    :458-489), causal masking, GQA, and the shift invariance that makes K
    smoothing exact in real arithmetic.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from tests import inputs


def _f(bits):
    return oracle.bf16_bits_to_f32(bits).reshape(bits.shape)


@pytest.mark.parametrize("l", [1, 127, 128, 300, 1000])
@pytest.mark.parametrize("d", [64, 128])
def test_kmean_close_to_fp64_mean(l, d):
    _, k, _ = inputs.attention(2, 3, l, d, l + d)
    kb = inputs.bits(k)
    mean = _f(oracle.sage_kmean(kb))
    ref = _f(kb).astype(np.float64).mean(axis=2)
    step = np.abs(ref) * 2.0 ** -7 + 1e-6 + l * 2.0 ** -23 * np.abs(_f(kb)).max()
    assert np.all(np.abs(mean - ref) <= step)


@pytest.mark.parametrize("blk", [16, 64, 128])
@pytest.mark.parametrize("smooth", [False, True])
def test_block_quant_invariants(blk, smooth):
    _, k, _ = inputs.attention(1, 3, 333, 128, blk)
    kb = inputs.bits(k)
    mean = oracle.sage_kmean(kb) if smooth else None
    q, s = oracle.sage_quant(kb, blk, mean)
    x = _f(kb) - (_f(mean)[:, :, None, :] if smooth else 0)
    nblk = s.shape[-1]
    for b in range(nblk):
        xs = x[:, :, b * blk:(b + 1) * blk]
        qs = q[:, :, b * blk:(b + 1) * blk].astype(np.int32)
        amax = np.maximum(np.abs(xs).max(axis=(2, 3)), np.float32(1e-7)).astype(np.float32)
        np.testing.assert_array_equal(s[:, :, b].view(np.uint32), (amax / np.float32(127)).view(np.uint32))
        assert np.all(np.abs(qs).max(axis=(2, 3)) == 127)
        err = np.abs(qs * (amax / 127)[:, :, None, None] - xs)
        assert np.all(err <= 0.5 * (amax / 127)[:, :, None, None] * (1 + 1e-5))


def test_block_quant_rounding_half_even_and_saturation():
    # one block whose amax is 127 so that the multiplier is exactly 1
    x = np.zeros((1, 1, 16, 128), np.float32)
    x[0, 0, 0, :6] = [127.0, 0.5, 1.5, 2.5, -0.5, -2.5]
    q, s = oracle.sage_quant(oracle.f32_to_bf16_bits(x), 16)
    assert s[0, 0, 0] == np.float32(1.0)
    assert list(q[0, 0, 0, :6]) == [127, 0, 2, 2, 0, -2]


def _sdpa64(qd, kd, v, sm, causal=False):
    s = np.einsum("bhid,bhjd->bhij", qd, kd) * sm
    if causal:
        li, lj = s.shape[-2:]
        s = np.where(np.arange(lj)[None, :] > np.arange(li)[:, None], -np.inf, s)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    return np.einsum("bhij,bhjd->bhid", p / p.sum(-1, keepdims=True), v)


def _quantized(q, k, blkq=128, blkk=128, smooth=True):
    qb, kb = inputs.bits(q), inputs.bits(k)
    mean = oracle.sage_kmean(kb) if smooth else None
    q8, qs = oracle.sage_quant(qb, blkq)
    k8, ks = oracle.sage_quant(kb, blkk, mean)
    return q8, qs, k8, ks


def _all_rows(b, h, l):
    return np.array([[bi, hi, i] for bi in range(b) for hi in range(h) for i in range(l)], np.int64)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_matches_fp64_softmax_on_dequantized_inputs(causal):
    q, k, v = inputs.attention(1, 2, 200, 128, 3)
    q8, qs, k8, ks = _quantized(q, k, 64, 64)
    sm = 128 ** -0.5
    out = oracle.sage_attn_rows(q8, qs, 64, k8, ks, 64, inputs.bits(v), sm, _all_rows(1, 2, 200), causal)
    qd = q8.astype(np.float64) * np.repeat(qs, 64, axis=2)[:, :, :200, None]
    kd = k8.astype(np.float64) * np.repeat(ks, 64, axis=2)[:, :, :200, None]
    ref = _sdpa64(qd, kd, _f(inputs.bits(v)).astype(np.float64), sm, causal).reshape(-1, 128)
    # P is rounded to bf16 in the oracle (relative 2^-9 per weight)
    np.testing.assert_allclose(out, ref, rtol=0, atol=6e-3)
    cos = (out * ref).sum() / np.linalg.norm(out) / np.linalg.norm(ref)
    assert cos > 0.99999


def test_attention_reference_gate_vs_sdpa_with_gqa():
    q, _, _ = inputs.attention(1, 4, 150, 128, 8)
    _, k, v = inputs.attention(1, 2, 170, 128, 9)
    q8, qs, k8, ks = _quantized(q, k)
    out = oracle.sage_attn_rows(q8, qs, 128, k8, ks, 128, inputs.bits(v), 128 ** -0.5, _all_rows(1, 4, 150))
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), enable_gqa=True)
    torch.testing.assert_close(torch.from_numpy(out).reshape(ref.shape), ref, rtol=0.08, atol=0.06)


def test_attention_reference_preflight_inputs():
    """The reference preflight's arange-modulo inputs (turing_sage/__init__.py:612-663)."""
    d = 128
    qv = torch.arange(4 * 65 * d, dtype=torch.float32)
    kv = torch.arange(2 * 73 * d, dtype=torch.float32)
    q = (((qv % 29) - 14) / 32).reshape(1, 4, 65, d).to(torch.bfloat16)
    k = ((((kv * 3) % 31) - 15) / 32).reshape(1, 2, 73, d).to(torch.bfloat16)
    v = ((((kv * 5) % 37) - 18) / 32).reshape(1, 2, 73, d).to(torch.bfloat16)
    q8, qs, k8, ks = _quantized(q, k)
    out = oracle.sage_attn_rows(q8, qs, 128, k8, ks, 128, inputs.bits(v), d ** -0.5, _all_rows(1, 4, 65))
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), enable_gqa=True)
    torch.testing.assert_close(torch.from_numpy(out).reshape(ref.shape), ref, rtol=0.08, atol=0.05)


def test_smoothing_is_shift_invariant():
    """Subtracting the channel mean of K shifts each score row by a constant:
    exact-arithmetic softmax is unchanged, so smoothed and unsmoothed oracle
    outputs agree to quantization precision."""
    q, k, v = inputs.attention(1, 2, 256, 128, 12)
    rows = _all_rows(1, 2, 256)
    a = oracle.sage_attn_rows(*_quantized(q, k, smooth=True)[:2], 128, *_quantized(q, k, smooth=True)[2:], 128,
                              inputs.bits(v), 128 ** -0.5, rows)
    b = oracle.sage_attn_rows(*_quantized(q, k, smooth=False)[:2], 128, *_quantized(q, k, smooth=False)[2:], 128,
                              inputs.bits(v), 128 ** -0.5, rows)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float()).reshape(-1, 128).numpy()
    ea, eb = np.abs(a - ref).max(), np.abs(b - ref).max()
    assert ea < 0.05 and np.abs(a - b).max() < 0.05
    # smoothing removes the per-head channel bias from K's quantization range
    assert ea <= eb * 1.5
