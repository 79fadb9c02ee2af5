"""Pins the W8A8 attention part of the CPU oracle without the GPU.

  * Hadamard: equals (1/sqrt D) H_D diag(s) with H_D the Sylvester matrix of
    scipy.linalg.hadamard (fp64), preserves norms and Q.K dot products, and is
    undone channel by channel by the inverse in the reference's validation
    script, whose sign table is a second statement of s;
  * K anchor: the decision of an fp64 numpy restatement of the detector on
    inputs with a clear margin, the sampled-row formula, and the two regimes
    (a common channel offset is removed, centred keys keep -1);
  * rotated tile quantizer: scale == amax / 127 of the fp64 rotated tile,
    max |code| == 127, dequantization error <= half a step, floor scale past L;
  * V quantizer: per-channel closed form, zero padding;
  * dense W8A8 attention: the reference's own preflight self-test
    (turing_sage/__init__.py:573-609: arange inputs, B1 Hq4 Hkv2 Lq129 Lk151,
    D 64/128, allclose rtol 0.12 / atol 0.09 to fp32 SDPA), fp64 softmax on
    the dequantized inputs, causal masking, and closed forms (one visible key,
    constant V) that fix the u8 probability offset and the final v_scale.
"""
from __future__ import annotations

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import oracle
from tests import inputs


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _signs(d: int) -> np.ndarray:
    return np.array([-1.0 if oracle.w8a8_sign_negative(c) else 1.0 for c in range(d)])


def _rotation(d: int) -> np.ndarray:
    return scipy.linalg.hadamard(d).astype(np.float64) * _signs(d)[None, :] / np.sqrt(d)


@pytest.mark.parametrize("d", [64, 128])
def test_hadamard_is_signed_sylvester_matrix(d):
    rng = np.random.default_rng(d)
    r = _rotation(d)
    for _ in range(20):
        x = rng.standard_normal(d).astype(np.float32) * 3
        y = oracle.w8a8_hadamard(x)
        np.testing.assert_allclose(y, r @ x.astype(np.float64), rtol=0, atol=2e-6 * np.abs(x).sum() / np.sqrt(d))
    # basis vectors give the columns of the signed matrix
    for c in (0, 1, 7, 8, d - 1):
        e = np.zeros(d, np.float32)
        e[c] = 1.0
        np.testing.assert_allclose(oracle.w8a8_hadamard(e), r[:, c], atol=1e-7)


def _inverse_rotation_of_validation_script(y: np.ndarray) -> np.ndarray:
    """The reference validation script's inverse of the kernel rotation
    (kernel/scripts/validate_compatible.py:613-629): in-place Sylvester
    butterflies over spans 1, 2, 4, ..., then 1/sqrt(D), then the channel
    signs of the script's own table (bit c of word c >> 5 clear -> -1).
    That table is a second statement of the rotation's signs, independent of
    the kernel source the oracle's table was taken from."""
    words = (0x1035997B, 0x8087F5EE, 0xEE2E4E1A, 0x71132418)
    d = y.shape[-1]
    r = y.astype(np.float64)
    span = 1
    while span < d:
        pairs = r.reshape(-1, 2, span)
        r = np.concatenate((pairs[:, 0] + pairs[:, 1], pairs[:, 0] - pairs[:, 1]), axis=-1).reshape(d)
        span *= 2
    signs = np.array([1.0 if (words[c >> 5] >> (c & 31)) & 1 else -1.0 for c in range(d)])
    return r / np.sqrt(d) * signs


@pytest.mark.parametrize("d", [64, 128])
def test_hadamard_inverts_with_the_validation_scripts_sign_table(d):
    # every basis vector comes back exactly where it started: a single sign
    # bit that differs between the two tables, a flipped bit-to-sign mapping
    # or the signs applied after the butterflies instead of before would send
    # some e_c to -e_c or smear it over other channels
    for c in range(d):
        e = np.zeros(d, np.float32)
        e[c] = 1.0
        back = _inverse_rotation_of_validation_script(oracle.w8a8_hadamard(e))
        np.testing.assert_allclose(back, e, atol=1e-6, err_msg=f"channel {c}")
    rng = np.random.default_rng(11)
    x = rng.standard_normal(d).astype(np.float32)
    np.testing.assert_allclose(_inverse_rotation_of_validation_script(oracle.w8a8_hadamard(x)), x, atol=1e-5)


@pytest.mark.parametrize("d", [64, 128])
def test_hadamard_preserves_norms_and_dot_products(d):
    rng = np.random.default_rng(7)
    q = rng.standard_normal(d).astype(np.float32)
    k = rng.standard_normal(d).astype(np.float32) + 2
    rq, rk = oracle.w8a8_hadamard(q), oracle.w8a8_hadamard(k)
    assert abs(np.dot(rq.astype(np.float64), rk) - np.dot(q.astype(np.float64), k)) < 1e-4
    assert abs(np.linalg.norm(rq.astype(np.float64)) - np.linalg.norm(q.astype(np.float64))) < 1e-5


def _anchor_fp64(k: np.ndarray) -> int:
    """fp64 statement of the detector's decision (fused.cu:409-575)."""
    length = k.shape[0]
    rows = [s * (length - 1) // 8 for s in range(9)]
    x = k[rows].astype(np.float64)
    energy, vmax = (x * x).sum(), np.abs(x).max()
    dist = ((9 * x - x.sum(axis=0)) ** 2).sum(axis=1)
    best = int(np.argmin(dist))
    r = x - x[best]
    keep = (r * r).sum() < energy and np.abs(r).max() <= vmax * 1.125
    return rows[best] if keep else -1


@pytest.mark.parametrize("length", [1, 2, 9, 151, 1000])
@pytest.mark.parametrize("d", [64, 128])
def test_anchor_matches_fp64_decision(length, d):
    g = torch.Generator().manual_seed(length + d)
    for offset in (0.0, 3.0):
        k = (torch.randn(2, 3, length, d, generator=g) + offset * torch.randn(2, 3, 1, d, generator=g)).to(torch.bfloat16)
        got = oracle.w8a8_detect_anchor(_bits(k))
        kf = k.float().numpy()
        for b in range(2):
            for h in range(3):
                assert got[b, h] == _anchor_fp64(kf[b, h]), (b, h, offset)


def test_anchor_regimes():
    g = torch.Generator().manual_seed(3)
    # a large common offset: the anchor is the sampled key nearest the mean
    k = (torch.randn(1, 1, 512, 128, generator=g) * 0.1 + 5.0).to(torch.bfloat16)
    a = int(oracle.w8a8_detect_anchor(_bits(k))[0, 0])
    assert a in [s * 511 // 8 for s in range(9)]
    # symmetric keys around zero: centring cannot lower the energy
    k = torch.randn(1, 1, 512, 128, generator=g).to(torch.bfloat16)
    k[0, 0, ::2] = -k[0, 0, 1::2]
    assert int(oracle.w8a8_detect_anchor(_bits(k))[0, 0]) == -1
    # fp16 input path reads fp16 bit patterns
    k16 = (torch.randn(1, 1, 100, 64, generator=g) + 4).to(torch.float16)
    a16 = oracle.w8a8_detect_anchor(_bits(k16), oracle.DTYPE_FP16)
    assert a16[0, 0] == _anchor_fp64(k16.float().numpy()[0, 0])


@pytest.mark.parametrize("tile", [16, 64])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("anchored", [False, True])
def test_rotated_tile_quant_invariants(tile, d, anchored):
    _, k, _ = inputs.attention(1, 2, 150, d, tile + d)
    kb = _bits(k)
    anchors = oracle.w8a8_detect_anchor(kb) if anchored else None
    ntiles = (150 + tile - 1) // tile + 1  # one tile past the end
    q, s = oracle.w8a8_quant_tiles(kb, tile, ntiles, True, anchors)
    kf = k.float().numpy().astype(np.float64)
    r = _rotation(d)
    for h in range(2):
        x = kf[0, h]
        if anchored and anchors[0, h] >= 0:
            x = x - x[anchors[0, h]]
        y = x @ r.T
        for t in range(ntiles):
            ys = y[t * tile:(t + 1) * tile]
            qs = q[0, h, t * tile:(t + 1) * tile].astype(np.float64)
            if ys.size == 0:
                assert s[0, h, t] == np.float32(1e-7) / np.float32(127)
                continue
            amax = max(np.abs(ys).max(), 1e-7)
            assert abs(s[0, h, t] * 127 - amax) <= 2e-6 * amax
            assert np.abs(qs).max() == 127
            assert np.all(np.abs(qs * s[0, h, t] - ys) <= 0.5 * s[0, h, t] + 4e-6 * amax)


def test_unrotated_tile_quant_is_plain_per_tile_int8():
    _, k, _ = inputs.attention(1, 1, 64, 128, 5)
    q, s = oracle.w8a8_quant_tiles(_bits(k), 64, 1, rotate=False)
    x = k.float().numpy()[0, 0]
    amax = np.float32(np.abs(x).max())
    assert s[0, 0, 0] == amax / np.float32(127)
    np.testing.assert_array_equal(q[0, 0], np.clip(np.rint(x * (np.float32(127) / amax)), -128, 127).astype(np.int8))


@pytest.mark.parametrize("length", [1, 64, 151, 200])
def test_v_quant_closed_form(length):
    _, _, v = inputs.attention(2, 2, length, 128, length)
    v = v * 3
    q, s = oracle.w8a8_quant_v(_bits(v))
    lpad = (length + 63) // 64 * 64
    assert q.shape == (2, 2, 128, lpad) and s.shape == (2, 2, 128)
    x = v.float().numpy()
    amax = np.abs(x).max(axis=2)
    np.testing.assert_array_equal(s, np.maximum(amax / np.float32(127), np.float32(1e-12)))
    inv = (np.float32(1) / s)[:, :, None, :]
    codes = np.clip(np.rint(x * inv), -128, 127).astype(np.int8)
    np.testing.assert_array_equal(q[..., :length], codes.transpose(0, 1, 3, 2))
    assert not q[..., length:].any()
    assert np.all(np.abs(q).max(axis=3) == 127)


def test_v_quant_zero_channel_floor():
    v = torch.zeros(1, 1, 10, 64, dtype=torch.bfloat16)
    q, s = oracle.w8a8_quant_v(_bits(v))
    assert np.all(s == np.float32(1e-12)) and not q.any()


def _reference_preflight_inputs(head_dim: int):
    qv = torch.arange(4 * 129 * head_dim, dtype=torch.float32)
    kv = torch.arange(2 * 151 * head_dim, dtype=torch.float32)
    q = (((qv % 29) - 14) / 16).reshape(1, 4, 129, head_dim).to(torch.bfloat16)
    k = ((((kv * 3) % 31) - 15) / 16).reshape(1, 2, 151, head_dim).to(torch.bfloat16)
    v = ((((kv * 5) % 37) - 18) / 16).reshape_as(k).to(torch.bfloat16)
    return q, k, v


def _oracle_w8a8(q, k, v, causal=False, sm_scale=None, stabilize_k=True, rotate=True, dtype=oracle.DTYPE_BF16):
    b, hq, lq, d = q.shape
    lk = k.shape[2]
    q8, qs, k8, ks, _ = oracle.w8a8_quant_qk(_bits(q), _bits(k), dtype, rotate, stabilize_k)
    v8, vs = oracle.w8a8_quant_v(_bits(v), dtype)
    rows = np.array([(bi, h, i) for bi in range(b) for h in range(hq) for i in range(lq)])
    scale = d ** -0.5 if sm_scale is None else sm_scale
    return torch.from_numpy(oracle.w8a8_attn_rows(q8, qs, k8, ks, v8, vs, lk, scale, rows, causal)).reshape(q.shape)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_reference_preflight_self_test(head_dim):
    """turing_sage/__init__.py:573-609, the reference's own W8A8 gate."""
    q, k, v = _reference_preflight_inputs(head_dim)
    out = _oracle_w8a8(q, k, v).to(torch.bfloat16)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), enable_gqa=True)
    assert torch.isfinite(out).all()
    assert torch.allclose(out.float(), ref, rtol=0.12, atol=0.09)
    assert (out.float() - ref).abs().max() < 5e-3  # far inside the gate


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("lk", [2, 64, 151, 300])
def test_attention_against_fp64_softmax(causal, lk):
    q, k, v = inputs.attention(1, 4, 130, 128, lk, hkv=2, lk=lk)
    out = _oracle_w8a8(q, k, v, causal=causal).double()
    ref = torch.nn.functional.scaled_dot_product_attention(q.double(), k.double(), v.double(), is_causal=causal,
                                                           enable_gqa=True)
    if causal and lk < 130:
        ref = ref[:, :, :lk]  # rows past Lk see all keys; SDPA's mask is top-left too
        out = out[:, :, :lk]
    cos = torch.nn.functional.cosine_similarity(out.flatten(), ref.flatten(), dim=0)
    assert cos > 0.999 and (out - ref).abs().max() < 0.05


def test_finite_mask_of_the_reference_with_a_zero_key_tile():
    """The reference masks raw scores with -5e6 before scaling
    (attn_utils.cuh:436-462), so when a K tile quantizes to zeros (Lk = 1:
    the anchor is the only key) the scale is 1e-7/127 and the 63 padded keys
    get p = 255 like the real one: out = v / 64.  The oracle keeps that."""
    q, k, v = inputs.attention(1, 1, 8, 128, 1, lk=1)
    out = _oracle_w8a8(q, k, v)
    v8, vs = oracle.w8a8_quant_v(_bits(v))
    deq = torch.from_numpy(v8[0, 0, :, 0].astype(np.float32) * vs[0, 0])
    torch.testing.assert_close(out[0, 0], (deq / 64).expand(8, 128), rtol=1e-5, atol=1e-7)
    # without the anchor the key keeps its codes and the mask holds
    out = _oracle_w8a8(q, k, v, stabilize_k=False)
    torch.testing.assert_close(out[0, 0], deq.expand(8, 128), rtol=1e-5, atol=1e-7)


def test_one_visible_key_returns_its_dequantized_value():
    # causal row 0 sees only key 0: p = 255 exactly once, out = v8[0] * v_scale
    q, k, v = inputs.attention(1, 1, 64, 128, 11)
    q8, qs, k8, ks, _ = oracle.w8a8_quant_qk(_bits(q), _bits(k))
    v8, vs = oracle.w8a8_quant_v(_bits(v))
    out = oracle.w8a8_attn_rows(q8, qs, k8, ks, v8, vs, 64, 128 ** -0.5, np.array([(0, 0, 0)]), causal=True)
    # d = sum p = 2^(log2 255 rounded to fp32) ~ 255, P = 255
    expect = v8[0, 0, :, 0].astype(np.float64) * 255 / 255 * vs[0, 0]
    np.testing.assert_allclose(out[0], expect, rtol=2e-6, atol=1e-7)


def test_constant_value_rows_are_exact():
    # every key carries the same V row: out = v (up to V's own quantization)
    q, k, _ = inputs.attention(1, 2, 100, 128, 21)
    v = torch.linspace(-2, 2, 128).to(torch.bfloat16).expand(1, 2, 100, 128).contiguous()
    out = _oracle_w8a8(q, k, v)
    v8, vs = oracle.w8a8_quant_v(_bits(v))
    deq = torch.from_numpy(v8[0, 0, :, 0].astype(np.float32) * vs[0, 0])
    # sum P_u8 / sum p differs from 1 by the u8 rounding of p only
    assert (out - deq).abs().max() < 2.5e-2 * deq.abs().max()


def test_fp16_inputs_and_gqa():
    q, k, v = inputs.attention(1, 4, 70, 64, 33, hkv=1, lk=90)
    q, k, v = q.to(torch.float16), k.to(torch.float16), v.to(torch.float16)
    out = _oracle_w8a8(q, k, v, dtype=oracle.DTYPE_FP16)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), enable_gqa=True)
    assert torch.allclose(out, ref, rtol=0.12, atol=0.09)
    assert torch.nn.functional.cosine_similarity(out.flatten(), ref.flatten(), dim=0) > 0.999
