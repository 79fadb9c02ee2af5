"""Pins the ConvRot part of the CPU oracle (oracle/tu_oracle.c) without the GPU.

Checks are chosen so that plausible mistakes fail one of them:
  * the staged butterflies equal the dense Kronecker matrix of the reference's
    R4 (convrot_quant.cu:104-116) -> catches a wrong sign pattern, stride or
    stage order that changes the transform;
  * orthogonality / involution / basis columns / the regular-row property;
  * quantizer invariants and an independent re-derivation with torch's bf16
    cast and numpy rint;
  * the reference's own cross-check: staged and row-buffer quantizers give
    bit-equal codes and scales within rtol 1e-6 (validate_compatible.py:43-64);
  * the exhaustive proof that the GPU's reciprocal-multiply quotient gives the
    same INT8 codes as IEEE division.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from tests import inputs

R4 = 0.5 * np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
H2 = np.array([[1, 1], [1, -1]], dtype=np.float64) / np.sqrt(2.0)


def dense(group: int) -> np.ndarray:
    """Dense transform; np.kron's first factor acts on the most significant digit
    (stride 64), the last on the stride-1 digit."""
    if group == 256:
        return np.kron(R4, np.kron(R4, np.kron(R4, R4)))
    return np.kron(H2, np.kron(R4, np.kron(R4, R4)))


@pytest.mark.parametrize("group", [128, 256])
def test_rotation_matches_dense_matrix(group):
    rng = np.random.default_rng(group)
    m = dense(group)
    for _ in range(20):
        x = rng.standard_normal(group).astype(np.float32) * rng.choice([1e-3, 1.0, 50.0])
        y = oracle.rotate_group(x, group)
        ref = m @ x.astype(np.float64)
        np.testing.assert_allclose(y, ref, rtol=0, atol=4e-7 * np.abs(x).max() * 4)


@pytest.mark.parametrize("group", [128, 256])
def test_rotation_is_orthogonal_and_involutive(group):
    m = dense(group)
    np.testing.assert_allclose(m @ m.T, np.eye(group), atol=1e-12)
    np.testing.assert_allclose(m, m.T, atol=1e-15)  # symmetric -> involution
    rng = np.random.default_rng(7)
    x = rng.standard_normal(group).astype(np.float32)
    twice = oracle.rotate_group(oracle.rotate_group(x, group), group)
    np.testing.assert_allclose(twice, x, rtol=0, atol=2e-6 * np.abs(x).max())


@pytest.mark.parametrize("group", [128, 256])
def test_rotation_basis_columns_exact(group):
    """e_i maps to column i; every entry is +-1/16 (G=256) or +-fp32(1/sqrt2)/8 (G=128),
    exactly representable, so the comparison is bit-exact."""
    m = dense(group)
    c = np.float32(0.70710678118654752440)
    for i in range(0, group, 7):
        e = np.zeros(group, np.float32)
        e[i] = 1.0
        col = m[:, i]
        expect = (np.sign(col) * (np.float32(1 / 16) if group == 256 else c / np.float32(8))).astype(np.float32)
        np.testing.assert_array_equal(oracle.rotate_group(e, group), expect)


def test_regular_row_property_distinguishes_groups():
    """Every R4 row sums to 1, so a constant row is a fixed point of the G=256
    transform; the G=128 transform (H2 on the top digit) is not regular."""
    x = np.full(256, 3.0, np.float32)
    np.testing.assert_array_equal(oracle.rotate_group(x, 256), x)
    y = oracle.rotate_group(np.full(128, 3.0, np.float32), 128)
    assert np.all(y[64:] == 0) and np.allclose(y[:64], 3.0 * np.sqrt(2), rtol=1e-6)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([
        (rng.standard_normal(200000) * 10.0 ** rng.integers(-30, 30, 200000)).astype(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, 3.3895313e38, -3.3895313e38, 1e-40, -1e-40, np.inf, -np.inf], np.float32),
        # ties: mantissa low half exactly 0x8000 with even and odd upper halves
        np.array([0x3f808000, 0x3f818000, 0xbf808000, 0x00008000], np.uint32).view(np.float32),
    ]).astype(np.float32)
    got = oracle.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, ref)
    assert oracle.f32_to_bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FFF  # canonical NaN


def _rows_y(x_bits: np.ndarray, group: int) -> np.ndarray:
    xf = oracle.bf16_bits_to_f32(x_bits).reshape(x_bits.shape)
    m, k = xf.shape
    y = np.empty_like(xf)
    for r in range(m):
        for g in range(k // group):
            y[r, g * group:(g + 1) * group] = oracle.rotate_group(xf[r, g * group:(g + 1) * group], group)
    return y


@pytest.mark.parametrize("group", [128, 256])
def test_quantizer_invariants_and_rederivation(group):
    x = inputs.activation(24, 1536, 11)
    xb = inputs.bits(x)
    q, s = oracle.convrot_quant(xb, group)
    y = _rows_y(xb, group)
    absmax = np.abs(y).max(axis=1)
    expect_scale = np.maximum(np.minimum(absmax, np.float32(3.38953139e38)) / np.float32(127), np.float32(1e-30))
    np.testing.assert_array_equal(s.view(np.uint32), expect_scale.astype(np.float32).view(np.uint32))
    # independent re-derivation with torch's bf16 cast and numpy rint
    yb = torch.from_numpy(y).to(torch.bfloat16).float()
    rs = torch.from_numpy(s).to(torch.bfloat16).float()[:, None]
    ref = torch.clamp(torch.round((yb / rs).to(torch.bfloat16).float()), -128, 127).to(torch.int8).numpy()
    np.testing.assert_array_equal(q, ref)
    assert q.min() >= -128 and q.max() <= 127
    assert np.all(np.abs(q.astype(np.int32)).max(axis=1) >= 126)
    # dequantization error bound: half a code plus the bf16 double rounding
    err = np.abs(q.astype(np.float64) - y.astype(np.float64) / rs.numpy())
    assert np.all(err <= 0.5 + np.abs(y / rs.numpy()) * 2.0 ** -7 + 1e-6)


def test_quantizer_zero_and_extreme_rows():
    x = np.zeros((3, 256), np.float32)
    x[1, 5] = 1e4
    x[2, :] = -2.5e38
    q, s = oracle.convrot_quant(oracle.f32_to_bf16_bits(x), 256)
    assert np.all(q[0] == 0) and s[0] == np.float32(1e-30)
    assert np.abs(q[1].astype(int)).max() == 127
    assert np.isfinite(s[2]) and np.abs(q[2].astype(int)).max() >= 126


@pytest.mark.parametrize("group", [128, 256])
def test_staged_equals_row_buffer(group):
    """The reference's own KAT: staged and row-buffer quantizers produce bit-equal
    codes, scales within rtol 1e-6 (kernel/scripts/validate_compatible.py:43-64)."""
    xb = inputs.bits(inputs.activation(64, 5120, 21))
    q1, s1 = oracle.convrot_quant(xb, group, staged=False)
    q2, s2 = oracle.convrot_quant(xb, group, staged=True)
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_allclose(s1, s2, rtol=1e-6, atol=5e-8)


def test_reciprocal_quotient_is_code_exact_on_the_quantizer_domain():
    """The GPU's a * RN(1/b) quotient gives the IEEE-division INT8 code on all
    ~1.05e9 (value, scale) pairs, although ~2e8 of its fp32 quotients differ
    in the last place (so the check is not vacuous)."""
    bad, pairs, fp32_diff = oracle.check_recip_quant()
    assert pairs > 1_000_000_000
    assert fp32_diff > 100_000_000
    assert bad == 0, f"{bad} (value, scale) pairs give a different INT8 code"


# ---------------------------------------------------------------------------
# fused input activations (convrot_quant.cu:137-156): this build's fixed fp32
# exp / tanh, pinned against double precision
# ---------------------------------------------------------------------------
def test_exp_det_accuracy_and_edges():
    v = np.concatenate([np.linspace(-87.0, 88.7, 40001), np.linspace(-1, 1, 2001)]).astype(np.float32)
    got = np.array([oracle.exp_det(float(t)) for t in v], np.float64)
    rel = np.abs(got / np.exp(v.astype(np.float64)) - 1)
    assert rel.max() < 1.5e-7  # ~1.3 ulp
    assert oracle.exp_det(0.0) == 1.0
    assert oracle.exp_det(100.0) == np.inf and oracle.exp_det(-100.0) == 0.0
    assert np.isnan(oracle.exp_det(float("nan")))


def test_tanh_det_accuracy_and_symmetry():
    u = np.concatenate([np.linspace(-12, 12, 48001), np.geomspace(1e-8, 1e-2, 2000)]).astype(np.float32)
    got = np.array([oracle.tanh_det(float(t)) for t in u], np.float64)
    assert np.abs(got - np.tanh(u.astype(np.float64))).max() < 1.3e-7
    neg = np.array([oracle.tanh_det(float(-t)) for t in u], np.float64)
    np.testing.assert_array_equal(neg, -got)
    assert oracle.tanh_det(0.0) == 0.0 and oracle.tanh_det(20.0) == 1.0


def _gelu64(x):
    x = x.astype(np.float64)
    return 0.5 * x * (1 + np.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def test_gelu_tanh_matches_fp64_and_torch():
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.standard_normal(20000) * 3, np.linspace(-6, 6, 4001)]).astype(np.float32)
    x = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits(x))  # bf16 inputs, as the kernel sees them
    got = np.array([oracle.gelu_tanh_bf16(float(t)) for t in x], np.float32)
    # bf16 output: within one bf16 step of the fp64 value (plus the reference
    # formula's own cancellation near x << 0, where values are ~1e-7)
    ref = _gelu64(x)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -8 + 1e-6)
    # and equal to torch's tanh-GELU in fp32 rounded to bf16 except at rare
    # rounding ties (tanh differs in the last fp32 ulp) and around x ~ -5, where
    # 1 + tanh cancels and each library's last tanh ulp shows in the bf16 result
    tg = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").to(torch.bfloat16).float().numpy()
    assert np.mean(tg[x > -4] == got[x > -4]) > 0.999
    assert np.all(np.abs(tg - got) <= np.abs(tg) * 2.0 ** -6 + 1e-6)


def test_swiglu_matches_fp64():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(20000) * 4).astype(np.float32)
    u = rng.standard_normal(20000).astype(np.float32)
    got = np.array([oracle.swiglu(float(a), float(b)) for a, b in zip(g, u)], np.float64)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u.astype(np.float64)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 6e-7 + 1e-30)
    assert oracle.swiglu(-200.0, 1.0) == 0.0 and oracle.swiglu(200.0, 2.0) == 400.0


@pytest.mark.parametrize("group", [128, 256])
def test_gelu_quantizer_is_gelu_then_quantizer(group):
    """act 1 = bf16 tanh-GELU applied elementwise, then the plain quantizer."""
    xb = inputs.bits(inputs.activation(16, 1024, 31))
    xf = oracle.bf16_bits_to_f32(xb).reshape(xb.shape)
    gb = oracle.f32_to_bf16_bits(np.vectorize(oracle.gelu_tanh_bf16, otypes=[np.float32])(xf))
    q1, s1 = oracle.convrot_quant(xb, group, act=oracle.ACT_GELU_TANH)
    q0, s0 = oracle.convrot_quant(gb, group)
    np.testing.assert_array_equal(q1, q0)
    np.testing.assert_array_equal(s1.view(np.uint32), s0.view(np.uint32))


@pytest.mark.parametrize("group", [128, 256])
def test_swiglu_quantizer_bounds(group):
    """act 2 on [gate | up] rows: scales = amax/127 of the rotated fp64 SwiGLU
    within fp32 rounding, codes within half a step of the exact quotient plus
    the three bf16 roundings (y, scale, quotient; 2^-8 relative each)."""
    rng = np.random.default_rng(group)
    x = (rng.standard_normal((8, 2 * 512)) * 2).astype(np.float32)
    xb = oracle.f32_to_bf16_bits(x)
    xf = oracle.bf16_bits_to_f32(xb).reshape(xb.shape).astype(np.float64)
    q, s = oracle.convrot_quant(xb, group, act=oracle.ACT_SWIGLU)
    assert q.shape == (8, 512)
    act = xf[:, :512] / (1 + np.exp(-xf[:, :512])) * xf[:, 512:]
    y = (act.reshape(8, -1, group) @ dense(group).T).reshape(8, 512)
    np.testing.assert_allclose(s, np.abs(y).max(axis=1) / 127, rtol=1e-5)
    err = np.abs(q - y / s[:, None])
    assert np.all(err <= 0.5 + np.abs(y / s[:, None]) * 3 * 2.0 ** -8 + 1e-3)


@pytest.mark.parametrize("act", [1, 2])
def test_staged_equals_row_buffer_with_activation(act):
    """The same cross-check for the fused activations (validate_wan_fusions.py:45-80
    compares the fused GELU codes against a two-pass quantizer)."""
    k = 1024
    xb = inputs.bits(inputs.activation(32, 2 * k if act == 2 else k, 22 + act))
    q1, s1 = oracle.convrot_quant(xb, 256, staged=False, act=act)
    q2, s2 = oracle.convrot_quant(xb, 256, staged=True, act=act)
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_allclose(s1, s2, rtol=1e-6, atol=5e-8)


# ---------------------------------------------------------------------------
# fp16 elements (the two-pass ops' float16 input, convrot_quant.cu:158-248)
# ---------------------------------------------------------------------------
def _f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def _rows_y_f16(xb: np.ndarray, group: int) -> np.ndarray:
    xf = xb.view(np.float16).astype(np.float32)
    m, k = xf.shape
    y = np.empty_like(xf)
    for r in range(m):
        for g in range(k // group):
            y[r, g * group:(g + 1) * group] = oracle.rotate_group(xf[r, g * group:(g + 1) * group], group)
    return y


def _f16_codes(y: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """numpy's float16 casts (independent of the oracle's converter):
    clamp(rint(f16(f16(y) / f16(scale)))) with fmax/fmin NaN semantics."""
    yh = y.astype(np.float16).astype(np.float32)
    rs = scale.astype(np.float16).astype(np.float32)[:, None]
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        d = (yh / rs).astype(np.float16).astype(np.float32)
    return np.fmin(np.float32(127), np.fmax(np.float32(-128), np.rint(d))).astype(np.int8)


@pytest.mark.parametrize("group", [128, 256])
def test_fp16_quantizer_rederivation(group):
    rng = np.random.default_rng(100 + group)
    x = rng.standard_normal((12, 1024)).astype(np.float32) * np.array([1e-2, 1, 30, 3000] * 3, np.float32)[:, None]
    # the sign pattern of a column of the (involutive) rotation concentrates a
    # group onto one output: |y| ~ 60000 * 16 (G=256) or 60000 * 8 sqrt2 (G=128),
    # above 65504 -> the scale clip applies and the fp16 row buffer holds inf
    sign = np.sign(dense(group)[:, 0]).astype(np.float32)
    x[5, :group] = 60000.0 * sign
    x[6, group:2 * group] = -50000.0 * np.sign(dense(group)[:, 3]).astype(np.float32)
    xb = _f16_bits(x)
    q, s = oracle.convrot_quant(xb, group, staged=True, fp16=True)
    y = _rows_y_f16(xb, group)
    absmax = np.abs(y).max(axis=1)
    expect = np.maximum(np.minimum(absmax, np.float32(65504)) * np.float32(1.0 / 127.0), np.float32(1e-30))
    np.testing.assert_array_equal(s.view(np.uint32), expect.astype(np.float32).view(np.uint32))
    assert absmax[5] > 65504 and absmax[6] > 65504
    np.testing.assert_array_equal(q, _f16_codes(y, s))
    assert s[5] == s[6] == np.float32(65504) * np.float32(1.0 / 127.0)
    assert q[5, 0] == 127 and q[6, group + 3] == -128  # +-inf / fp16(scale) saturates


def test_fp16_zero_and_tiny_rows_divide_by_a_zero_scale():
    """fp16(scale) is 0 for scale < 2^-25: the reference divides by zero and
    its clamp maps +-inf to 127 / -128 and 0 / 0 (NaN) to -128."""
    x = np.zeros((3, 256), np.float32)
    x[1, 3] = 1e-6   # absmax 1e-6 / 16 after rotation: scale ~ 5e-10 -> fp16 0
    x[2, 3] = 1.0    # an ordinary row for contrast
    q, s = oracle.convrot_quant(_f16_bits(x), 256, staged=True, fp16=True)
    assert s[0] == np.float32(1e-30) and np.all(q[0] == -128)
    y = _rows_y_f16(_f16_bits(x), 256)
    assert np.float16(s[1]) == 0
    np.testing.assert_array_equal(q[1], np.where(y[1] > 0, 127, -128).astype(np.int8))
    assert np.abs(q[2].astype(int)).max() == 127


def test_gelu_tanh_f16_matches_fp64_and_torch():
    x = np.arange(0, 0x7c00, dtype=np.uint16)
    x = np.concatenate([x, x | 0x8000]).view(np.float16).astype(np.float32)  # every finite fp16
    got = np.array([oracle.gelu_tanh_f16(float(t)) for t in x], np.float32)
    ref = _gelu64(x)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -11 + 2.0 ** -24 + np.abs(x) * 2e-7)
    assert np.array_equal(got.astype(np.float16).astype(np.float32), got)  # fp16 values
    tg = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").half().float().numpy()
    assert np.mean(tg[x > -4] == got[x > -4]) > 0.999


@pytest.mark.parametrize("group", [128, 256])
def test_fp16_gelu_quantizer_is_gelu_then_quantizer(group):
    rng = np.random.default_rng(group + 3)
    xb = _f16_bits(rng.standard_normal((8, 512)) * 2)
    xf = xb.view(np.float16).astype(np.float32)
    gb = _f16_bits(np.vectorize(oracle.gelu_tanh_f16, otypes=[np.float32])(xf))
    q1, s1 = oracle.convrot_quant(xb, group, staged=True, act=oracle.ACT_GELU_TANH, fp16=True)
    q0, s0 = oracle.convrot_quant(gb, group, staged=True, fp16=True)
    np.testing.assert_array_equal(q1, q0)
    np.testing.assert_array_equal(s1.view(np.uint32), s0.view(np.uint32))


@pytest.mark.parametrize("group", [128, 256])
def test_fp16_swiglu_quantizer_bounds(group):
    rng = np.random.default_rng(group + 9)
    xb = _f16_bits(rng.standard_normal((8, 1024)) * 2)
    xf = xb.view(np.float16).astype(np.float64)
    q, s = oracle.convrot_quant(xb, group, staged=True, act=oracle.ACT_SWIGLU, fp16=True)
    act = xf[:, :512] / (1 + np.exp(-xf[:, :512])) * xf[:, 512:]
    y = (act.reshape(8, -1, group) @ dense(group).T).reshape(8, 512)
    np.testing.assert_allclose(s, np.abs(y).max(axis=1) / 127, rtol=1e-5)
    err = np.abs(q - y / s[:, None])
    assert np.all(err <= 0.5 + np.abs(y / s[:, None]) * 3 * 2.0 ** -11 + 1e-3)
