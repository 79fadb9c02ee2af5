"""GPU parity: LayerNorm fused with the ConvRot INT8 quantizer
(tu_layer_norm_adaln_convrot_quant_i8 / tu_layer_norm_affine_convrot_quant_i8,
the Wan block's norm1 / norm2 / norm3 feeding their projections).

The fused kernel must give the codes and row scales of the two ops it
replaces, bit for bit: the bf16 LayerNorm (oracle or_layer_norm_adaln /
or_layer_norm_affine, restating kernel/csrc/turing/segmented_rms_adaln.cu:236-307)
followed by the row-buffer quantizer (oracle or_convrot_quant_i8_t, restating
kernel/csrc/turing/convrot_quant.cu:350-444) on that bf16 output.  Checked
against the oracle chain on small shapes and against the two GPU ops at the
Wan-14B width (5120) on ragged row counts.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

G = 128


def _u16(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _adaln_case(b, l, h, steps, seed, offset=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(b, l, h, generator=g) * 3 + offset).to(torch.bfloat16)
    scale = (torch.randn(b, steps, h, generator=g) * 0.2).to(torch.bfloat16)
    shift = (torch.randn(b, steps, h, generator=g) * 0.2).to(torch.bfloat16)
    return x, scale, shift


def _fused_adaln(x, scale, shift, eps, dev):
    from comfyui_turing_utils_kernel import turing_layer_norm_adaln_int8_convrot_quantize

    q, s = turing_layer_norm_adaln_int8_convrot_quantize(x.to(dev), scale.to(dev), shift.to(dev), eps, G)
    torch.cuda.synchronize(dev)
    return q.cpu().numpy(), s.cpu().numpy().reshape(-1)


def _two_ops_gpu(normed, dev):
    from comfyui_turing_utils_kernel import turing_bf16_int8_convrot_quantize

    q, s = turing_bf16_int8_convrot_quantize(normed.reshape(-1, normed.shape[-1]).contiguous(), G)
    torch.cuda.synchronize(dev)
    return q.cpu().numpy(), s.cpu().numpy().reshape(-1)


def _assert_same(got, want, what):
    q, s = got
    q_ref, s_ref = want
    np.testing.assert_array_equal(s.view(np.uint32), s_ref.view(np.uint32), err_msg=f"{what}: row scales")
    np.testing.assert_array_equal(q, q_ref, err_msg=f"{what}: codes")


@pytest.mark.parametrize("b,l,h,steps", [(1, 9, 256, 1), (2, 17, 768, 3), (1, 13, 1536, 1), (3, 10, 3072, 4),
                                         (2, 11, 5120, 2), (1, 40, 1280, 40)])
def test_adaln_vs_oracle_chain(gpu_device, b, l, h, steps):
    """Odd per (768 = 3 x 256, 1280 = 5 x 256) ends on a half pass; steps > 1
    puts several modulation rows in one workgroup (the unstaged path)."""
    print(f"ln_adaln_convrot b={b} l={l} h={h} steps={steps}", flush=True)
    x, scale, shift = _adaln_case(b, l, h, steps, 7000 + b * 100 + l + h + steps)
    normed = oracle.layer_norm_adaln(_u16(x), _u16(scale), _u16(shift), 1e-6)
    want = oracle.convrot_quant(normed.reshape(b * l, h), G)
    _assert_same(_fused_adaln(x, scale, shift, 1e-6, gpu_device), want, "adaln fused vs oracle")


@pytest.mark.parametrize("rows,h", [(1, 256), (9, 1536), (23, 5120), (8, 2560)])
def test_affine_vs_oracle_chain(gpu_device, rows, h):
    from comfyui_turing_utils_kernel import turing_layer_norm_affine_int8_convrot_quantize

    print(f"ln_affine_convrot rows={rows} h={h}", flush=True)
    g = torch.Generator().manual_seed(rows * 31 + h)
    x = (torch.randn(rows, h, generator=g) * 2 - 0.5).to(torch.bfloat16)
    # wide weights, negative ones included, as norm3 checkpoints may hold
    w = (1 + 0.5 * torch.randn(h, generator=g)).to(torch.bfloat16)
    bias = (0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    normed = oracle.layer_norm_affine(_u16(x), _u16(w), _u16(bias), 1e-6)
    want = oracle.convrot_quant(normed, G)
    q, s = turing_layer_norm_affine_int8_convrot_quantize(x.to(gpu_device), w.to(gpu_device), bias.to(gpu_device),
                                                          1e-6, G)
    torch.cuda.synchronize(gpu_device)
    _assert_same((q.cpu().numpy(), s.cpu().numpy().reshape(-1)), want, "affine fused vs oracle")


@pytest.mark.parametrize("rows", [1, 7, 8, 1003, 32760])
def test_adaln_vs_two_ops_wan14b_width(gpu_device, rows):
    """The Wan-14B width at ragged row counts up to C5's 32760 tokens (the
    last workgroup's spare half-waves compute and store nothing)."""
    from comfyui_turing_utils_kernel import turing_layer_norm_adaln

    print(f"ln_adaln_convrot vs two ops rows={rows}", flush=True)
    x, scale, shift = _adaln_case(1, rows, 5120, 1, rows, offset=-0.25)
    dev = gpu_device
    normed = turing_layer_norm_adaln(x.to(dev), scale.to(dev), shift.to(dev), 1e-6)
    _assert_same(_fused_adaln(x, scale, shift, 1e-6, dev), _two_ops_gpu(normed, dev), "adaln fused vs two ops")


def test_special_rows(gpu_device):
    """Constant rows (variance 0), all-zero rows, rows near the bf16 range,
    tiny rows, and rows holding inf / NaN, against the oracle chain."""
    h = 1536
    g = torch.Generator().manual_seed(99)
    rows = [torch.full((h,), 3.0), torch.zeros(h), torch.randn(h, generator=g) * 1e37,
            torch.randn(h, generator=g) * 1e-30, torch.randn(h, generator=g)]
    inf_row = torch.randn(h, generator=g)
    inf_row[17] = float("inf")
    nan_row = torch.randn(h, generator=g)
    nan_row[1000] = float("nan")
    rows += [inf_row, nan_row, torch.randn(h, generator=g) * 50 + 1e4]
    x = torch.stack(rows).to(torch.bfloat16).reshape(1, len(rows), h)
    scale = (torch.randn(1, 1, h, generator=g) * 0.3).to(torch.bfloat16)
    shift = (torch.randn(1, 1, h, generator=g) * 0.3).to(torch.bfloat16)
    print("ln_adaln_convrot special rows", flush=True)
    normed = oracle.layer_norm_adaln(_u16(x), _u16(scale), _u16(shift), 1e-6)
    want = oracle.convrot_quant(normed.reshape(len(rows), h), G)
    _assert_same(_fused_adaln(x, scale, shift, 1e-6, gpu_device), want, "special rows")


def test_fallback_shapes_match_two_ops(gpu_device):
    """Shapes outside the one-kernel path (group 256, width 6144, fp16 input
    is refused by the quantizer) run the two ops and give their result."""
    from comfyui_turing_utils_kernel import (turing_bf16_int8_convrot_quantize, turing_layer_norm_adaln,
                                             turing_layer_norm_adaln_int8_convrot_quantize)

    dev = gpu_device
    for h, group in ((5120, 256), (6144, 128), (640, 128)):
        print(f"ln_adaln_convrot fallback h={h} group={group}", flush=True)
        x, scale, shift = _adaln_case(1, 5, h, 1, h + group)
        x, scale, shift = x.to(dev), scale.to(dev), shift.to(dev)
        q, s = turing_layer_norm_adaln_int8_convrot_quantize(x, scale, shift, 1e-6, group)
        q2, s2 = turing_bf16_int8_convrot_quantize(turing_layer_norm_adaln(x, scale, shift, 1e-6).reshape(5, h), group)
        assert torch.equal(q, q2) and torch.equal(s.view(torch.int32), s2.view(torch.int32))
    with pytest.raises(TypeError):
        x, scale, shift = _adaln_case(1, 5, 1536, 1, 3)
        turing_layer_norm_adaln_int8_convrot_quantize(x.half().to(dev), scale.half().to(dev), shift.half().to(dev),
                                                      1e-6, 128)
