"""GPU parity: LayerNorm + AdaLN (HIP, tu_layer_norm_adaln) vs the CPU oracle
(oracle/tu_oracle.c or_layer_norm_adaln, a restatement of
kernel/csrc/turing/segmented_rms_adaln.cu:236-307), bit for bit in bf16,
fp16 and fp32, and the reference's own gate
(kernel/scripts/validate_wan_fusions.py:80-119) through the op.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.test_oracle_adaln import _expanded

pytestmark = pytest.mark.gpu

_DT = {torch.bfloat16: oracle.DTYPE_BF16, torch.float16: oracle.DTYPE_FP16, torch.float32: oracle.DTYPE_FP32}


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def _oracle(x, scale, shift, eps):
    return _oracle_bits(_np(x), _np(scale), _np(shift), eps, x.dtype)


def _oracle_bits(x, scale, shift, eps, dtype):
    out = oracle.layer_norm_adaln(x, scale, shift, eps, _DT[dtype])
    return out.view(np.uint32) if dtype == torch.float32 else out


def _bits_of(t: torch.Tensor) -> np.ndarray:
    a = _np(t.cpu())
    return a.view(np.uint32) if t.dtype == torch.float32 else a


def _case(b, l, h, steps, dtype, seed, offset=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(b, l, h, generator=g) * 3 + offset).to(dtype)
    scale = (torch.randn(b, steps, h, generator=g) * 0.2).to(dtype)
    shift = (torch.randn(b, steps, h, generator=g) * 0.2).to(dtype)
    return x, scale, shift


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("b,l,h,steps", [(2, 17, 5120, 4), (2, 33, 700, 1), (1, 5, 8192, 2), (2, 7, 9000, 3),
                                         (1, 1, 64, 1), (3, 12, 1536, 5), (1, 40, 257, 40), (1, 3, 4096, 4)])
def test_bit_exact_vs_oracle(gpu_device, dtype, b, l, h, steps):
    from comfyui_turing_utils_kernel import turing_layer_norm_adaln

    print(f"layer_norm_adaln {dtype} b={b} l={l} h={h} steps={steps}", flush=True)
    x, scale, shift = _case(b, l, h, steps, dtype, b * 1000 + l + h + steps)
    out = turing_layer_norm_adaln(x.to(gpu_device), scale.to(gpu_device), shift.to(gpu_device), 1e-6)
    torch.cuda.synchronize(gpu_device)
    np.testing.assert_array_equal(_bits_of(out), _oracle(x, scale, shift, 1e-6))


@pytest.mark.parametrize("offset", [0.0, 100.0, 1000.0, 1e5])
def test_offsets_bit_exact(gpu_device, offset):
    from comfyui_turing_utils_kernel import turing_layer_norm_adaln

    for dtype in (torch.bfloat16, torch.float32):
        x, scale, shift = _case(2, 9, 5120, 1, dtype, 3, offset)
        out = turing_layer_norm_adaln(x.to(gpu_device), scale.to(gpu_device), shift.to(gpu_device), 1e-5)
        torch.cuda.synchronize(gpu_device)
        np.testing.assert_array_equal(_bits_of(out), _oracle(x, scale, shift, 1e-5))


def test_division_edge_rows_bit_exact(gpu_device):
    """Rows whose Welford and combine quotients leave the range where the
    kernel's reciprocal-multiply division is exact, so the wave takes the
    IEEE division for those lanes: all-zero rows, constant rows (every later
    delta is 0), rows with exact zeros between normal values, tiny (1e-30)
    and huge (1e30) values, and a row mixing all of them; widths 5120
    (every count known) and 700 (ragged), bf16 and fp32."""
    from comfyui_turing_utils_kernel import turing_layer_norm_adaln

    for dtype in (torch.bfloat16, torch.float32):
        for h in (5120, 700):
            g = torch.Generator().manual_seed(h)
            rows = [torch.zeros(h), torch.full((h,), 2.5), torch.randn(h, generator=g),
                    torch.randn(h, generator=g) * 1e-30, torch.randn(h, generator=g) * 1e30,
                    torch.randn(h, generator=g)]
            rows[2][::3] = 0.0
            mixed = rows[5]
            mixed[::5] = 0.0
            mixed[1::7] *= 1e-30
            mixed[2::11] *= 1e25
            x = torch.stack(rows).unsqueeze(0).to(dtype)
            scale = (torch.randn(1, 1, h, generator=g) * 0.2).to(dtype)
            shift = (torch.randn(1, 1, h, generator=g) * 0.2).to(dtype)
            print(f"layer_norm_adaln edge rows {dtype} h={h}", flush=True)
            out = turing_layer_norm_adaln(x.to(gpu_device), scale.to(gpu_device), shift.to(gpu_device), 1e-6)
            torch.cuda.synchronize(gpu_device)
            np.testing.assert_array_equal(_bits_of(out), _oracle(x, scale, shift, 1e-6))


@pytest.mark.parametrize("case", ["x", "x/8", "x+100", "x+1000"])
def test_reference_gate(gpu_device, case):
    """validate_wan_fusions.py:80-119: rtol 0.006 / atol 0.002 against torch
    layer_norm + addcmul, on x and its scaled / offset variants (the oracle
    test states the 3-element tie exception of x + 100)."""
    from comfyui_turing_utils_kernel import turing_layer_norm_adaln

    g = torch.Generator().manual_seed(1234)
    x = torch.randn(2, 17, 5120, generator=g).to(torch.bfloat16)
    scale = (torch.randn(2, 4, 5120, generator=g) * 0.1).to(torch.bfloat16)
    shift = (torch.randn(2, 4, 5120, generator=g) * 0.1).to(torch.bfloat16)
    xi = {"x": x, "x/8": x * 0.125, "x+100": x + 100.0, "x+1000": x + 1000.0}[case].to(torch.bfloat16)
    out = turing_layer_norm_adaln(xi.to(gpu_device), scale.to(gpu_device), shift.to(gpu_device), 1e-6).cpu()
    ref = torch.addcmul(_expanded(shift, 17), torch.nn.functional.layer_norm(xi, (5120,), eps=1e-6),
                        1 + _expanded(scale, 17))
    ok = torch.isclose(out.float(), ref.float(), rtol=0.006, atol=0.002)
    assert ok.float().mean() >= 0.9999


def test_wan_shape_rows(gpu_device):
    """Wan 2.1 14B 720p norm1 shape: 32760 tokens x 5120, one modulation row;
    a seeded sample of 600 rows (first, last and random) bit-exact."""
    from comfyui_turing_utils_kernel import turing_layer_norm_adaln

    g = torch.Generator(device=gpu_device).manual_seed(9)
    x = torch.randn(1, 32760, 5120, generator=g, device=gpu_device).to(torch.bfloat16)
    scale = (torch.randn(1, 1, 5120, generator=g, device=gpu_device) * 0.1).to(torch.bfloat16)
    shift = (torch.randn(1, 1, 5120, generator=g, device=gpu_device) * 0.1).to(torch.bfloat16)
    out = turing_layer_norm_adaln(x, scale, shift, 1e-6)
    rows = torch.cat([torch.tensor([0, 32759]), torch.randperm(32760, generator=torch.Generator().manual_seed(1))[:598]])
    got = _bits_of(out[0, rows.to(gpu_device)])
    ref = _oracle_bits(_np(x[0, rows.to(gpu_device)].cpu()[None]), _np(scale.cpu()), _np(shift.cpu()), 1e-6,
                       torch.bfloat16)
    np.testing.assert_array_equal(got, ref[0])


def test_errors(gpu_device):
    from comfyui_turing_utils_kernel import turing_layer_norm_adaln

    x = torch.randn(1, 4, 64, device=gpu_device, dtype=torch.bfloat16)
    s = torch.zeros(1, 1, 64, device=gpu_device, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="epsilon"):
        turing_layer_norm_adaln(x, s, s, 0.0)
    with pytest.raises(RuntimeError, match="epsilon"):
        turing_layer_norm_adaln(x, s, s, float("nan"))
    with pytest.raises(ValueError):
        turing_layer_norm_adaln(x, s[:, :, :32], s[:, :, :32], 1e-6)
    with pytest.raises(TypeError):
        turing_layer_norm_adaln(x[0], s, s, 1e-6)


# ---------------------------------------------------------------------------
# Affine LayerNorm (turing_utils::layer_norm_affine, tu_layer_norm_affine):
# the Wan block's norm3 with weights of any sign and size
# ---------------------------------------------------------------------------
def _affine_case(rows, h, dtype, seed, offset=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, h, generator=g) * 3 + offset).to(dtype)
    w = (1 + torch.randn(h, generator=g) * 0.5).to(dtype)  # N(1, 0.5): negative and sub-0.5 weights
    b = (torch.randn(h, generator=g) * 0.3).to(dtype)
    return x, w, b


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,h", [(34, 5120), (33, 700), (5, 8192), (7, 9000), (1, 64), (12, 1536), (40, 257)])
def test_affine_bit_exact_vs_oracle(gpu_device, dtype, rows, h):
    print(f"layer_norm_affine {dtype} rows={rows} h={h}", flush=True)
    x, w, b = _affine_case(rows, h, dtype, rows * 7 + h)
    out = torch.ops.turing_utils.layer_norm_affine(x.to(gpu_device), w.to(gpu_device), b.to(gpu_device), 1e-6)
    torch.cuda.synchronize(gpu_device)
    ref = oracle.layer_norm_affine(_np(x), _np(w), _np(b), 1e-6, _DT[dtype])
    np.testing.assert_array_equal(_bits_of(out), ref.view(np.uint32) if dtype == torch.float32 else ref)
    assert (w.float() < 0).any()


def test_affine_wan_shape_rows_and_3d(gpu_device):
    """[1, 32760, 5120] bf16 through the op (3-D input, rows flattened); 600
    rows checked against the oracle; the whole output against torch's
    layer_norm within one bf16 step."""
    print("layer_norm_affine Wan shape 32760x5120", flush=True)
    g = torch.Generator(device=gpu_device).manual_seed(3)
    x = (torch.randn(1, 32760, 5120, generator=g, device=gpu_device) * 2).to(torch.bfloat16)
    w = (1 + torch.randn(5120, generator=g, device=gpu_device) * 0.5).to(torch.bfloat16)
    b = (torch.randn(5120, generator=g, device=gpu_device) * 0.3).to(torch.bfloat16)
    out = torch.ops.turing_utils.layer_norm_affine(x, w, b, 1e-6)
    torch.cuda.synchronize(gpu_device)
    rows = torch.randperm(32760, generator=torch.Generator().manual_seed(1))[:600].to(gpu_device)
    ref = oracle.layer_norm_affine(_np(x[0, rows].cpu()), _np(w.cpu()), _np(b.cpu()), 1e-6, oracle.DTYPE_BF16)
    np.testing.assert_array_equal(_bits_of(out[0, rows]), ref)
    t = torch.nn.functional.layer_norm(x.float(), (5120,), w.float(), b.float(), eps=1e-6).to(torch.bfloat16)
    diff = (out.float() - t.float()).abs()
    mag = t.float().abs() + b.float().abs()
    ulp = torch.exp2(torch.floor(torch.log2(mag.clamp_min(1e-30))) - 7)
    assert (diff <= 2 * ulp + 1e-6).all()
    assert (out == t).float().mean() > 0.99
