"""Pins the LayerNorm + AdaLN oracle (or_layer_norm_adaln) without the GPU.

  * the reference's own gate (kernel/scripts/validate_wan_fusions.py:80-119):
    inputs x, x / 8, x + 100, x + 1000 with four modulation steps over 17
    tokens, against torch layer_norm + addcmul on the repeat-interleaved
    modulation, rtol 0.006 / atol 0.002;
  * the fp64 formula T(T(T((x - mean) / sqrt(var + eps)) * T(1 + scale)) +
    shift) bit for bit, apart from rounding ties of the normalized value
    (within one step of the type);
  * fp32 rows against fp64 LayerNorm; the modulation-row mapping for steps that
    do and do not divide L; large offsets (Welford keeps the variance).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _from_bits(b: np.ndarray, dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(dtype)


def _expanded(value: torch.Tensor, sequence: int) -> torch.Tensor:
    """validate_wan_fusions.py:35-43."""
    if value.shape[1] == 1:
        return value
    repeats = sequence // value.shape[1]
    if repeats == 1:
        return value
    if repeats * value.shape[1] != sequence:
        repeats += 1
    return torch.repeat_interleave(value, repeats, dim=1)[:, :sequence]


def _run(x, scale, shift, eps):
    dt = {torch.bfloat16: oracle.DTYPE_BF16, torch.float16: oracle.DTYPE_FP16}[x.dtype]
    return _from_bits(oracle.layer_norm_adaln(_bits(x), _bits(scale), _bits(shift), eps, dt), x.dtype)


def _reference_inputs(hidden=5120):
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(2, 17, hidden, generator=g).to(torch.bfloat16)
    scale = (torch.randn(2, 4, hidden, generator=g) * 0.1).to(torch.bfloat16)
    shift = (torch.randn(2, 4, hidden, generator=g) * 0.1).to(torch.bfloat16)
    return x, scale, shift


@pytest.mark.parametrize("case", ["x", "x/8", "x+100", "x+1000"])
def test_reference_gate(case):
    x, scale, shift = _reference_inputs()
    xi = {"x": x, "x/8": x * 0.125, "x+100": x + 100.0, "x+1000": x + 1000.0}[case].to(torch.bfloat16)
    out = _run(xi, scale, shift, 1e-6).float()
    ref = torch.addcmul(_expanded(shift, 17), torch.nn.functional.layer_norm(xi, (5120,), eps=1e-6),
                        1 + _expanded(scale, 17)).float()
    ok = torch.isclose(out, ref, rtol=0.006, atol=0.002)
    # torch's bf16 layer_norm breaks an exact-midpoint tie of the normalized
    # value the other way on 3 of 174080 elements of x + 100; those stay within
    # two bf16 steps and match the fp64 formula below
    assert ok.float().mean() >= 0.9999
    step = 2.0 ** (torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
    assert ((out - ref).abs() <= 2 * step)[~ok].all()


def _fp64_formula(x, scale, shift, eps, dtype):
    b, l, h = x.shape
    xs = x.double()
    mean = xs.mean(-1, keepdim=True)
    var = ((xs - mean) ** 2).mean(-1, keepdim=True)
    n = ((xs - mean) / torch.sqrt(var + eps)).to(dtype).double()
    m = (1 + _expanded(scale, l).double()).to(dtype).double()
    return (n * m + _expanded(shift, l).double()).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hidden,steps,length", [(5120, 4, 17), (700, 1, 33), (64, 3, 12), (8192, 2, 5)])
def test_fp64_formula(dtype, hidden, steps, length):
    g = torch.Generator().manual_seed(hidden + steps)
    x = (torch.randn(2, length, hidden, generator=g) * 3 + 1).to(dtype)
    scale = (torch.randn(2, steps, hidden, generator=g) * 0.2).to(dtype)
    shift = (torch.randn(2, steps, hidden, generator=g) * 0.2).to(dtype)
    out = _run(x, scale, shift, 1e-6).float()
    ref = _fp64_formula(x, scale, shift, 1e-6, dtype).float()
    diff = out != ref
    assert diff.float().mean() < 2e-3
    # a tie of the normalized value moves the result by one step of n * m,
    # whose magnitude is at most |out| + |shift| (cancellation near zero)
    mag = ref.abs() + _expanded(shift, length).float().abs()
    ulp = 2.0 ** (torch.floor(torch.log2(mag.clamp_min(1e-30))) - (7 if dtype == torch.bfloat16 else 10))
    assert ((out - ref).abs() <= 2 * ulp + 1e-6)[diff].all()


def test_fp32_rows_and_large_offsets():
    g = torch.Generator().manual_seed(5)
    for offset in (0.0, 1000.0, 1e5):
        x = torch.randn(1, 9, 3000, generator=g) + offset
        scale = torch.randn(1, 1, 3000, generator=g) * 0.1
        shift = torch.randn(1, 1, 3000, generator=g) * 0.1
        out = torch.from_numpy(oracle.layer_norm_adaln(x.numpy(), scale.numpy(), shift.numpy(), 1e-6,
                                                       oracle.DTYPE_FP32))
        xs = x.double()
        ref = (xs - xs.mean(-1, keepdim=True)) / torch.sqrt(xs.var(-1, unbiased=False, keepdim=True) + 1e-6)
        ref = ref * (1 + scale.double()) + shift.double()
        # fp32 rounding of the mean alone costs ulp(offset) / std; the bound is
        # torch's own fp32 layer_norm error on the same rows
        torch_err = (torch.nn.functional.layer_norm(x, (3000,), eps=1e-6) * (1 + scale) + shift - ref).abs().max()
        assert (out.double() - ref).abs().max() <= 1.5 * torch_err + 1e-6


@pytest.mark.parametrize("steps,length", [(4, 17), (3, 12), (5, 5), (4, 3), (2, 1)])
def test_modulation_row_mapping(steps, length):
    """Each token takes the modulation row the reference's repeat_interleave
    expansion assigns it: scale rows carry distinct constants."""
    hidden = 64
    x = torch.randn(1, length, hidden).to(torch.bfloat16)
    scale = torch.zeros(1, steps, hidden, dtype=torch.bfloat16)
    shift = torch.arange(steps, dtype=torch.float32).view(1, steps, 1).expand(1, steps, hidden).to(torch.bfloat16) * 8
    out = _run(x, scale, shift, 1e-6).float()
    rows = torch.round((out - torch.nn.functional.layer_norm(x.float(), (hidden,), eps=1e-6)).mean(-1) / 8)
    expect = _expanded(torch.arange(steps).view(1, steps, 1).float(), length)[0, :, 0]
    if length < steps:  # repeats == 0: the reference keeps the unexpanded rows
        expect = torch.arange(length).float().clamp_max(steps - 1)
    assert torch.equal(rows[0], expect)


# ---------------------------------------------------------------------------
# Affine LayerNorm (weight / bias), the Wan block's norm3 as ComfyUI runs it:
# torch.nn.functional.layer_norm(x, (H,), weight, bias, eps)
# ---------------------------------------------------------------------------
def _affine(x, w, b, eps):
    dt = {torch.bfloat16: oracle.DTYPE_BF16, torch.float16: oracle.DTYPE_FP16}[x.dtype]
    return _from_bits(oracle.layer_norm_affine(_bits(x), _bits(w), _bits(b), eps, dt), x.dtype)


def _affine_inputs(rows, hidden, dtype, seed, offset=0.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, hidden, generator=g) * 2 + offset).to(dtype)
    w = (1 + torch.randn(hidden, generator=g) * 0.5).to(dtype)  # includes negative and sub-0.5 weights
    b = (torch.randn(hidden, generator=g) * 0.3).to(dtype)
    return x, w, b


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hidden,offset", [(5120, 0.0), (700, 3.0), (64, 0.0), (8192, 100.0)])
def test_affine_matches_torch_layer_norm(dtype, hidden, offset):
    """torch's layer_norm with weight and bias on the CPU, computed in fp32 and
    rounded once: equal except where the two fp32 values straddle a rounding
    tie (a different statistics order), and never more than one step apart."""
    x, w, b = _affine_inputs(33, hidden, dtype, hidden + 7, offset)
    out = _affine(x, w, b, 1e-6).float()
    ref = torch.nn.functional.layer_norm(x.float(), (hidden,), w.float(), b.float(), eps=1e-6).to(dtype).float()
    # both are fp32 statistics in different orders; at an offset the mean's
    # fp32 rounding moves the normalized values, for torch as for the oracle,
    # so the bar is torch's own agreement with the fp64 formula
    xs = x.double()
    n = (xs - xs.mean(-1, keepdim=True)) / torch.sqrt(xs.var(-1, unbiased=False, keepdim=True) + 1e-6)
    r64 = (n * w.double() + b.double()).to(dtype).float()
    torch_vs_fp64 = (ref == r64).float().mean()
    assert (out == r64).float().mean() >= torch_vs_fp64 - 5e-3
    assert (out == ref).float().mean() > (0.995 if offset == 0 else 0.98)
    # a moved normalized value shifts the result by a step of n * w, whose
    # magnitude is at most |out| + |b| (cancellation near zero)
    mag = ref.abs() + b.float().abs()
    ulp = 2.0 ** (torch.floor(torch.log2(mag.clamp_min(1e-30))) - (7 if dtype == torch.bfloat16 else 10))
    assert ((out - ref).abs() <= 2 * ulp + 1e-7).all()
    assert (w.float() < 0.5).any() and (w.float() < 0).any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_affine_fp64_formula_and_planted_mistakes(dtype):
    """T((x - mean) / sqrt(var + eps) * w + b) in fp64 agrees except near ties;
    the AdaLN form T(T(n) T(1 + (w - 1))) + b), a dropped bias or an unbiased
    variance each move far more elements."""
    x, w, b = _affine_inputs(40, 1536, dtype, 3)
    out = _affine(x, w, b, 1e-6).float()
    xs = x.double()
    n = (xs - xs.mean(-1, keepdim=True)) / torch.sqrt(xs.var(-1, unbiased=False, keepdim=True) + 1e-6)
    ref = (n * w.double() + b.double()).to(dtype).float()
    same = (out == ref).float().mean()
    assert same > 0.995
    nb = n.to(dtype).double()
    adaln_form = (nb * w.double() + b.double()).to(dtype).float()
    no_bias = (n * w.double()).to(dtype).float()
    unbiased = ((xs - xs.mean(-1, keepdim=True)) / torch.sqrt(xs.var(-1, unbiased=True, keepdim=True) + 1e-6)
                * w.double() + b.double()).to(dtype).float()
    for wrong in (adaln_form, no_bias, unbiased):
        assert (out == wrong).float().mean() < same - 0.01
