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
@pytest.mark.parametrize("m,k,seed", [(1, 256, 11), (3, 512, 12), (17, 1536, 13), (64, 5120, 14), (8, 13824, 15),
                                      (5, 20480, 16), (3, 32768, 17), (2, 65536, 19)])
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
    x = torch.zeros(2, 65536 + 128, dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(ValueError, match="limit"):
        torch.ops.turing_utils.bf16_int8_convrot_quantize(x, 128)


def test_convrot_misaligned_view(gpu_device):
    """A view whose data pointer is not 16-byte aligned is copied, not refused."""
    base = inputs.activation(1, 4 * 256 + 8, 18).reshape(-1)
    view = base.to(gpu_device)[1:1 + 4 * 256].reshape(4, 256)
    assert view.data_ptr() % 16 != 0
    q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(view, 128)
    q_ref, s_ref = oracle.convrot_quant(inputs.bits(base[1:1 + 4 * 256].reshape(4, 256).contiguous()), 128)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))


# ---------------------------------------------------------------------------
# fused input activations: tanh-GELU (turing_utils::bf16_gelu_int8_convrot_quantize)
# and SwiGLU (bf16_int8_convrot_quantize(swiglu=True)), bit-exact vs the oracle
# ---------------------------------------------------------------------------
def _edge_values(m, k, seed):
    x = inputs.activation(m, k, seed).float()
    g = torch.Generator().manual_seed(seed + 1)
    x[0, : k // 2] = torch.linspace(-12, 12, k // 2)                 # the whole tanh range
    x[1, :8] = torch.tensor([0.0, -0.0, 1e-30, -1e-30, 3e38, -3e38, 1e4, -1e4])
    x[2] = torch.randn(k, generator=g) * 1e-3                           # tiny row
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("group", [128, 256])
# 40960 columns take 10 waves: past the table kernel's 8, so every GELU is computed
@pytest.mark.parametrize("m,k,seed", [(5, 512, 41), (64, 5120, 42), (32, 13824, 43), (3, 40960, 44)])
def test_gelu_quant_exact(gpu_device, group, m, k, seed):
    print(f"[convrot gelu] m={m} k={k} group={group}", flush=True)
    x = _edge_values(m, k, seed)
    q, s = torch.ops.turing_utils.bf16_gelu_int8_convrot_quantize(x.to(gpu_device), group)
    q_ref, s_ref = oracle.convrot_quant(inputs.bits(x), group, act=oracle.ACT_GELU_TANH)
    np.testing.assert_array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


def test_gelu_every_bf16_input(gpu_device):
    """Every finite bf16 value x, one per row at columns 0 and 17 of an
    otherwise zero row (the low half of one packed pair and the high half of
    another): the row scale carries the bits of gelu(x), so the whole
    activation domain is checked bit for bit against the oracle in both
    halves."""
    print("[convrot gelu] every finite bf16 input", flush=True)
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    bits = bits[(bits & 0x7F80) != 0x7F80]
    x = np.zeros((bits.size, 128), np.uint16)
    x[:, 0] = bits
    x[:, 17] = bits
    xt = inputs.from_bits(x)
    q, s = torch.ops.turing_utils.bf16_gelu_int8_convrot_quantize(xt.to(gpu_device), 128)
    q_ref, s_ref = oracle.convrot_quant(x, 128, act=oracle.ACT_GELU_TANH)
    got = s.cpu().numpy().reshape(-1).view(np.uint32)
    bad = np.flatnonzero(got != s_ref.view(np.uint32))
    assert bad.size == 0, f"{bad.size} scales differ, first inputs {[hex(int(v)) for v in bits[bad[:5]]]}"
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


def test_gelu_every_bf16_input_beside_large_negatives(gpu_device):
    """The same sweep with the rest of each row at -8.0 instead of 0:
    gelu(-8) is -0, so the row scale still carries the bits of gelu(x), and a
    wave's pass now holds no zero unless x is one. That sends every x with an
    exponent field in [2, 254] through the short select (table, |x| >= 8, and
    the exponent-lowering bf16(0.5 x) for |x| < 2^-12), which the zero rows
    above never reach."""
    print("[convrot gelu] every finite bf16 input beside -8.0", flush=True)
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    bits = bits[(bits & 0x7F80) != 0x7F80]
    x = np.full((bits.size, 128), 0xC100, np.uint16)  # -8.0
    x[:, 0] = bits
    x[:, 17] = bits
    xt = inputs.from_bits(x)
    q, s = torch.ops.turing_utils.bf16_gelu_int8_convrot_quantize(xt.to(gpu_device), 128)
    q_ref, s_ref = oracle.convrot_quant(x, 128, act=oracle.ACT_GELU_TANH)
    got = s.cpu().numpy().reshape(-1).view(np.uint32)
    bad = np.flatnonzero(got != s_ref.view(np.uint32))
    assert bad.size == 0, f"{bad.size} scales differ, first inputs {[hex(int(v)) for v in bits[bad[:5]]]}"
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


def test_swiglu_every_bf16_gate(gpu_device):
    """Every finite bf16 gate g with up = 1, one per row at column 0 of
    [gate | up] rows that are otherwise zero: the row scale carries the bits of
    g / (1 + exp(-g)) over the gate's whole bf16 domain, checked bit for bit."""
    print("[convrot swiglu] every finite bf16 gate", flush=True)
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    bits = bits[(bits & 0x7F80) != 0x7F80]
    x = np.zeros((bits.size, 256), np.uint16)
    x[:, 0] = bits
    x[:, 128] = 0x3F80  # up = 1.0
    q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(inputs.from_bits(x).to(gpu_device), 128, swiglu=True)
    q_ref, s_ref = oracle.convrot_quant(x, 128, act=oracle.ACT_SWIGLU)
    got = s.cpu().numpy().reshape(-1).view(np.uint32)
    bad = np.flatnonzero(got != s_ref.view(np.uint32))
    assert bad.size == 0, f"{bad.size} scales differ, first gates {[hex(int(v)) for v in bits[bad[:5]]]}"
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("group", [128, 256])
@pytest.mark.parametrize("m,k,seed", [(5, 512, 51), (48, 5120, 52)])
def test_swiglu_quant_exact(gpu_device, group, m, k, seed):
    print(f"[convrot swiglu] m={m} k={k} group={group}", flush=True)
    x = _edge_values(m, 2 * k, seed)
    q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(x.to(gpu_device), group, swiglu=True)
    q_ref, s_ref = oracle.convrot_quant(inputs.bits(x), group, act=oracle.ACT_SWIGLU)
    assert q.shape == (m, k)
    np.testing.assert_array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("act,name", [(1, "gelu_int8_convrot_quantize"), (2, "swiglu_int8_convrot_quantize")])
@pytest.mark.parametrize("group", [128, 256])
def test_staged_ops_exact(gpu_device, act, name, group):
    """The two-pass op names: staged scale formula, same codes contract."""
    m, k = 37, 5120
    print(f"[convrot staged] {name} m={m} k={k} group={group}", flush=True)
    x = _edge_values(m, 2 * k if act == 2 else k, 60 + act)
    q, s = getattr(torch.ops.turing_utils, name)(x.to(gpu_device), group)
    q_ref, s_ref = oracle.convrot_quant(inputs.bits(x), group, staged=True, act=act)
    np.testing.assert_array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


# ---------------------------------------------------------------------------
# float16 input to the two-pass ops (ops.py:163-186, :215-233; InputType = half
# of convrot_quant.cu:158-248)
# ---------------------------------------------------------------------------
def _f16(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float16)


def _f16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _assert_f16_exact(x: torch.Tensor, name: str, act: int, group: int, dev, label: str):
    print(f"[convrot fp16] {name} {label} shape={tuple(x.shape)} group={group}", flush=True)
    q, s = getattr(torch.ops.turing_utils, name)(x.to(dev), group)
    q_ref, s_ref = oracle.convrot_quant(_f16_bits(x), group, staged=True, act=act, fp16=True)
    got = s.cpu().numpy().reshape(-1).view(np.uint32)
    bad = np.flatnonzero(got != s_ref.view(np.uint32))
    assert bad.size == 0, f"{label}: {bad.size} scales differ, first rows {bad[:5]}"
    bad_q = np.argwhere(q.cpu().numpy() != q_ref)
    assert bad_q.size == 0, f"{label}: {len(bad_q)} codes differ, first {bad_q[:5].tolist()}"


@pytest.mark.parametrize("act,name", [(1, "gelu_int8_convrot_quantize"), (2, "swiglu_int8_convrot_quantize")])
@pytest.mark.parametrize("group", [128, 256])
def test_staged_ops_fp16_exact(gpu_device, act, name, group):
    """fp16 rows of several magnitudes (tiny rows whose fp16 scale underflows,
    large rows whose rotated absmax passes 65504) plus random rows."""
    rng = np.random.default_rng(70 + act + group)
    k = 5120
    width = 2 * k if act == 2 else k
    x = rng.standard_normal((40, width)).astype(np.float32)
    x *= np.array([1e-7, 1e-4, 1e-2, 1, 30, 3000, 60000, 1] * 5, np.float32)[:, None]
    x[7, :] = 0.0
    x = np.clip(x, -65504, 65504)
    _assert_f16_exact(_f16(x), name, act, group, gpu_device, "magnitudes")


def test_gelu_fp16_every_input(gpu_device):
    """Every finite fp16 x, one per row at column 0 of a zero row: the scale
    carries gelu(x) bit for bit over the fp16 domain."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    bits = bits[(bits & 0x7C00) != 0x7C00]
    x = np.zeros((bits.size, 128), np.uint16)
    x[:, 0] = bits
    xt = torch.from_numpy(x.view(np.int16)).view(torch.float16)
    _assert_f16_exact(xt, "gelu_int8_convrot_quantize", 1, 128, gpu_device, "every finite fp16 input")


def test_swiglu_fp16_every_gate(gpu_device):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    bits = bits[(bits & 0x7C00) != 0x7C00]
    x = np.zeros((bits.size, 256), np.uint16)
    x[:, 0] = bits
    x[:, 128] = 0x3C00  # up = 1.0
    xt = torch.from_numpy(x.view(np.int16)).view(torch.float16)
    _assert_f16_exact(xt, "swiglu_int8_convrot_quantize", 2, 128, gpu_device, "every finite fp16 gate")


def test_row_buffer_ops_refuse_fp16(gpu_device):
    x = torch.zeros((2, 256), dtype=torch.float16, device=gpu_device)
    with pytest.raises(TypeError):
        torch.ops.turing_utils.bf16_int8_convrot_quantize(x, 256)
    with pytest.raises(TypeError):
        torch.ops.turing_utils.bf16_gelu_int8_convrot_quantize(x, 256)


@pytest.mark.parametrize("group", [128, 256])
def test_gelu_quant_inf_nan_rows(gpu_device, group):
    """+-inf and NaN inputs take the GELU's direct path (the table covers
    finite inputs): codes and scales still equal the oracle's, with rows of
    8 sharing one workgroup."""
    print(f"[convrot gelu] inf / NaN rows group={group}", flush=True)
    g = torch.Generator().manual_seed(group)
    x = torch.randn(21, 512, generator=g)
    x[3, 17] = float("inf")
    x[5, 0] = float("-inf")
    x[9, 300] = float("nan")
    x[12, :] = float("-inf")
    x[20, 5] = float("inf")
    x[20, 6] = -9.5
    xb = x.to(torch.bfloat16)
    q, s = torch.ops.turing_utils.bf16_gelu_int8_convrot_quantize(xb.to(gpu_device), group)
    q_ref, s_ref = oracle.convrot_quant(inputs.bits(xb), group, act=oracle.ACT_GELU_TANH)
    np.testing.assert_array_equal(s.cpu().numpy().reshape(-1).view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
