"""GPU parity: ConvRot INT8 quantizer (HIP) vs the CPU oracle, bit-exact codes and scales.

Oracle: oracle/tu_oracle.c or_convrot_quant_i8, a restatement of
kernel/csrc/turing/convrot_quant.cu:350-444.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from tests import inputs

pytestmark = pytest.mark.gpu


def _run(x: torch.Tensor, group: int, dev):
    q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(x.to(dev), group)
    torch.cuda.synchronize(dev)
    return q.cpu().numpy(), s.cpu().numpy().reshape(-1)


def _assert_exact(x: torch.Tensor, group: int, dev, label: str):
    print(f"[convrot] {label} shape={tuple(x.shape)} group={group}", flush=True)
    q, s = _run(x, group, dev)
    q_ref, s_ref = oracle.convrot_quant(inputs.bits(x), group)
    bad_s = np.flatnonzero(s.view(np.uint32) != s_ref.view(np.uint32))
    assert bad_s.size == 0, f"{label}: {bad_s.size} scales differ, first row {bad_s[:5]}: {s[bad_s[:5]]} vs {s_ref[bad_s[:5]]}"
    bad_q = np.argwhere(q != q_ref)
    assert bad_q.size == 0, f"{label}: {len(bad_q)} codes differ, first {bad_q[:5].tolist()}"


@pytest.mark.parametrize("group", [128, 256])
@pytest.mark.parametrize("m,k,seed", [(1, 256, 11), (3, 512, 12), (17, 1536, 13), (64, 5120, 14), (8, 13824, 15)])
def test_convrot_random(gpu_device, group, m, k, seed):
    _assert_exact(inputs.activation(m, k, seed), group, gpu_device, f"random m={m} k={k}")


@pytest.mark.parametrize("group", [128, 256])
def test_convrot_config1_full(gpu_device, group):
    """BASELINE config 1 activation (M=4096, K=1536, seed 0), every row."""
    _assert_exact(inputs.activation(4096, 1536, 0), group, gpu_device, "config1")


@pytest.mark.parametrize("group", [128, 256])
def test_convrot_edge_rows(gpu_device, group):
    k = 1024
    rows = [
        torch.zeros(k),                                  # zero row: scale 1e-30, codes 0
        torch.full((k,), 3.0),                           # constant row
        torch.arange(k, dtype=torch.float32) - 512.0,    # ramp
        torch.where(torch.arange(k) == 5, 1e4, 1e-3),    # single spike
        torch.full((k,), -2.5e38),                       # near the bf16 max, negative
        torch.linspace(-1e-38, 1e-38, k),                # subnormal magnitudes
        torch.full((k,), 1e-30),                         # tiny constant (scale floor region)
        torch.tensor([(-1.0) ** i * (i % 7) for i in range(k)]),
    ]
    x = torch.stack(rows).to(torch.bfloat16)
    _assert_exact(x, group, gpu_device, "edge rows")


def test_convrot_c4_rows(gpu_device):
    """Wan-14B FFN-down input width (K=13824) at 512 rows, G=128, seed 3."""
    _assert_exact(inputs.activation(512, 13824, 3), 128, gpu_device, "c4 ffn-down rows")


def test_convrot_rejects_bad_width(gpu_device):
    x = torch.zeros(2, 200, dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(ValueError):
        torch.ops.turing_utils.bf16_int8_convrot_quantize(x, 128)
