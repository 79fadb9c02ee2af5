"""Pins the fused Q/K preprocessor's W8A8 variant (rotate_qk / stabilize_k)
in the CPU oracle, without the GPU.

The fused variant is RMSNorm + RoPE (the already pinned or_qk_rms_rope_int8
path, whose processed values are exactly representable in the input type)
followed by the W8A8 transform (the already pinned or_w8a8_* functions).  So:
  * row scope: the fused anchor equals or_w8a8_detect_anchor on the processed
    values, the anchor values are the anchor row's processed values, and the
    fused codes and scales equal or_w8a8_quant_tiles on the processed values,
    bit for bit;
  * head scope: the anchor's samples use a sequential fma for rrms
    (qk_preprocess.cu:283-296) while the tiles use the lane butterfly, so the
    same composition holds to one code;
  * with rotate and no anchor, the fused variant equals the composition for
    every scope; with neither, it is or_qk_rms_rope_int8;
  * the rotation leaves dequantized Q.K products at the unrotated values.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _case(h, l, d, dtype, scope, rot, seed, offset=3.0, per_token=True):
    """Inputs with a per-head channel offset.  Frequencies per token rotate
    that offset differently for each token (the anchor then rarely helps);
    one shared frequency row keeps it common (the anchor fires)."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(1, h, l, d, generator=g) + offset * torch.randn(1, h, 1, d, generator=g)).to(dtype)
    w = (1 + 0.1 * torch.randn(d if scope == "head" else h * d, generator=g)).to(dtype)
    theta = torch.rand((1, l if per_token else 1, rot // 2), generator=g) * 6.28
    freqs = torch.stack([torch.stack([theta.cos(), -theta.sin()], -1),
                         torch.stack([theta.sin(), theta.cos()], -1)], -2).to(dtype).float().numpy() if rot else None
    return x, w, freqs


def _to_bits(values: np.ndarray, dtype) -> np.ndarray:
    t = torch.from_numpy(values).to(dtype)
    assert torch.equal(t.float(), torch.from_numpy(values)), "processed values must be representable"
    return _bits(t)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d,rot,split", [(128, 128, False), (128, 64, True), (64, 64, False), (64, 0, False)])
@pytest.mark.parametrize("per_token", [True, False])
def test_row_scope_is_the_composition_bit_for_bit(dtype, d, rot, split, per_token):
    dt = oracle.DTYPE_FP16 if dtype == torch.float16 else oracle.DTYPE_BF16
    x, w, freqs = _case(4, 150, d, dtype, "row", rot, d + rot, per_token=per_token)
    args = (_bits(x), dt, _bits(w), "row", 1e-6, freqs, rot, split)
    anchors, values = oracle.qk_fused_anchor(*args)
    processed = oracle.qk_processed(*args)
    pb = _to_bits(processed, dtype)
    np.testing.assert_array_equal(anchors, oracle.w8a8_detect_anchor(pb, dt))
    if not per_token:
        assert (anchors >= 0).any()
    for h in range(4):
        expect = processed[0, h, anchors[0, h]] if anchors[0, h] >= 0 else np.zeros(d, np.float32)
        np.testing.assert_array_equal(values[0, h], expect)
    for tile, ntiles in ((16, 40), (64, 3)):
        q, s = oracle.qk_rms_rope_int8_ex(*args, tile, ntiles, True, anchors, values)
        rq, rs = oracle.w8a8_quant_tiles(pb, tile, ntiles, True, anchors, dt)
        np.testing.assert_array_equal(q, rq)
        np.testing.assert_array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("d", [64, 128])
def test_head_scope_matches_the_composition_to_one_code(d):
    x, w, freqs = _case(6, 130, d, torch.bfloat16, "head", d, 7 + d, per_token=False)
    args = (_bits(x), oracle.DTYPE_BF16, _bits(w), "head", 1e-6, freqs, d, False)
    anchors, values = oracle.qk_fused_anchor(*args)
    processed = oracle.qk_processed(*args)
    pb = _to_bits(processed, torch.bfloat16)
    np.testing.assert_array_equal(anchors, oracle.w8a8_detect_anchor(pb, oracle.DTYPE_BF16))
    q, s = oracle.qk_rms_rope_int8_ex(*args, 64, 3, True, anchors, values)
    rq, rs = oracle.w8a8_quant_tiles(pb, 64, 3, True, anchors, oracle.DTYPE_BF16)
    assert np.abs(q.astype(np.int32) - rq).max() <= 1
    np.testing.assert_allclose(s, rs, rtol=2e-3)


@pytest.mark.parametrize("scope", ["head", "row"])
def test_rotation_without_anchor_is_the_composition(scope):
    x, w, freqs = _case(3, 100, 128, torch.bfloat16, scope, 128, 11)
    args = (_bits(x), oracle.DTYPE_BF16, _bits(w), scope, 1e-6, freqs, 128, False)
    pb = _to_bits(oracle.qk_processed(*args), torch.bfloat16)
    q, s = oracle.qk_rms_rope_int8_ex(*args, 16, 28, True)
    rq, rs = oracle.w8a8_quant_tiles(pb, 16, 28, True, None)
    np.testing.assert_array_equal(q, rq)
    np.testing.assert_array_equal(s.view(np.uint32), rs.view(np.uint32))
    q0, s0 = oracle.qk_rms_rope_int8_ex(*args, 16, 28)
    r0, rs0 = oracle.qk_rms_rope_int8(*args, 16, 28)
    np.testing.assert_array_equal(q0, r0)
    np.testing.assert_array_equal(s0, rs0)


def test_rotation_preserves_dequantized_dot_products():
    x, w, freqs = _case(1, 64, 128, torch.bfloat16, "head", 128, 3, offset=0.0)
    args = (_bits(x), oracle.DTYPE_BF16, _bits(w), "head", 1e-6, freqs, 128, False)
    processed = oracle.qk_processed(*args)[0, 0].astype(np.float64)
    q, s = oracle.qk_rms_rope_int8_ex(*args, 64, 1, True)
    deq = q[0, 0].astype(np.float64) * s[0, 0, 0]
    ref = processed @ processed.T
    got = deq @ deq.T
    assert np.abs(got - ref).max() < 0.02 * np.abs(ref).max()
