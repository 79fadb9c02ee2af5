"""Fake-tensor contracts, fullgraph-leaf behaviour and host-side error paths of
the registered ops, mirroring the reference's contract tests
(tests/test_kernel_custom_ops.py:194-266, tests/test_turing_sage_quant.py:88-122,
tests/test_attention_correctness.py).  CPU only: meta tensors never reach the
HIP library, and CPU tensors must be refused before any launch."""
from __future__ import annotations

import pytest
import torch

import comfyui_turing_utils_kernel as kernel
from comfyui_turing_utils_kernel import ops, turing_sage  # noqa: F401
from comfyui_turing_utils_kernel.turing_sage import core, quant
from comfyui_turing_utils_kernel.turing_sage.correctness import (
    attention_error_metrics,
    require_attention_correctness,
)

META = "meta"


@pytest.mark.parametrize("group", [128, 256])
def test_convrot_fake_contract(group):
    x = torch.empty((3, 512), dtype=torch.bfloat16, device=META)
    q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(x, group)
    assert q.shape == (3, 512) and q.dtype == torch.int8 and q.device.type == META
    assert s.shape == (3, 1) and s.dtype == torch.float32
    # reference tests/test_kernel_custom_ops.py:194-217
    q, s = torch.ops.turing_utils.bf16_gelu_int8_convrot_quantize(x, group)
    assert q.shape == (3, 512) and s.shape == (3, 1) and q.dtype == torch.int8
    q, s = kernel.turing_bf16_int8_convrot_quantize(x, group, swiglu=True)
    assert q.shape == (3, 256) and s.shape == (3, 1)
    # two-pass op names (reference ops.py:163-186, :215-233)
    q, s = kernel.turing_gelu_int8_convrot_quantize(x, group)
    assert q.shape == (3, 512) and s.shape == (3, 1) and q.dtype == torch.int8
    q, s = kernel.turing_swiglu_int8_convrot_quantize(x, group)
    assert q.shape == (3, 256) and s.shape == (3, 1) and s.dtype == torch.float32


def test_linear_and_epilogue_fake_contracts():
    activation = torch.empty((7, 128), dtype=torch.int8, device=META)
    weight = torch.empty((64, 128), dtype=torch.int8, device=META)
    row_scale = torch.empty((7,), dtype=torch.float32, device=META)
    column_scale = torch.empty((64,), dtype=torch.float32, device=META)
    out = torch.ops.turing_utils.int8_linear(activation, weight, row_scale, column_scale)
    assert out.shape == (7, 64) and out.dtype == torch.bfloat16
    acc = torch.ops.turing_utils.int8_gemm_i32(activation, weight)
    assert acc.shape == (7, 64) and acc.dtype == torch.int32
    accumulator = torch.empty((7, 80), dtype=torch.int32, device=META)
    epi = torch.ops.turing_utils.dequantize_int8_bf16(accumulator, row_scale, column_scale, 64)
    assert epi.shape == (7, 64) and epi.dtype == torch.bfloat16
    epi = torch.ops.turing_utils.dequantize_int8_bf16(accumulator, row_scale, column_scale)
    assert epi.shape == (7, 80)
    residual = torch.empty((7, 64), dtype=torch.bfloat16, device=META)
    gate = torch.empty((2, 64), dtype=torch.bfloat16, device=META)
    out = torch.ops.turing_utils.int8_linear_residual(activation, weight, row_scale, column_scale, None,
                                                      residual, gate, 4)
    assert out.shape == (7, 64) and out.dtype == torch.bfloat16
    with pytest.raises(Exception, match="gate"):
        torch.ops.turing_utils.int8_linear_residual(activation, weight, row_scale, column_scale, None,
                                                    residual, gate, 1)


def test_sage_fake_contract_and_fullgraph_leaf():
    q = torch.empty((1, 4, 129, 128), dtype=torch.bfloat16, device=META)
    k = torch.empty((1, 2, 151, 128), dtype=torch.bfloat16, device=META)
    out = turing_sage.sageattn_compiled(q, k, k)
    assert out.shape == q.shape and out.dtype == q.dtype and out.device.type == META
    compiled = torch.compile(lambda a, b, c: turing_sage.sageattn_compiled(a, b, c), backend="eager", fullgraph=True)
    assert compiled(q, k, k).shape == q.shape


def test_linear_chain_is_a_fullgraph_leaf():
    def chain(x, w, ws):
        q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(x, 128)
        return torch.ops.turing_utils.int8_linear(q, w, s.reshape(-1), ws)

    x = torch.empty((5, 256), dtype=torch.bfloat16, device=META)
    w = torch.empty((48, 256), dtype=torch.int8, device=META)
    ws = torch.empty((48,), dtype=torch.float32, device=META)
    out = torch.compile(chain, backend="eager", fullgraph=True)(x, w, ws)
    assert out.shape == (5, 48) and out.dtype == torch.bfloat16


def test_cpu_tensors_are_refused():
    x = torch.zeros((4, 256), dtype=torch.bfloat16)
    for op in (torch.ops.turing_utils.bf16_int8_convrot_quantize, torch.ops.turing_utils.bf16_gelu_int8_convrot_quantize,
               torch.ops.turing_utils.gelu_int8_convrot_quantize, torch.ops.turing_utils.swiglu_int8_convrot_quantize):
        with pytest.raises(RuntimeError, match="CUDA|HIP"):
            op(x, 256)
    a = torch.zeros((4, 128), dtype=torch.int8)
    with pytest.raises(RuntimeError, match="CUDA|HIP"):
        torch.ops.turing_utils.int8_linear(a, a, torch.ones(4), torch.ones(4))
    q = torch.zeros((1, 2, 64, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA"):  # reference core.py raises ValueError here
        core.sageattn(q, q, q)
    with pytest.raises((RuntimeError, ValueError)):
        quant.per_block_int8(q, q)


def test_public_sage_api():
    assert turing_sage.__all__ == [
        "available", "w8a8_available", "split_prequantization_available", "fused_qk_preprocessing_available",
        "sageattn", "sageattn_compiled", "prequantize_sageattn", "prequantize_rms_rope_qk",
        "prequantize_sageattn_from_qk", "sageattn_from_prequantized", "w8a8attn", "w8a8attn_compiled",
        "prequantize_sol_sageattn", "prequantize_sol_sageattn_from_qk", "sol_sparse_sageattn_from_prequantized",
        "preflight", "preflight_w8a8",
    ]
    assert turing_sage.w8a8_available() is turing_sage.available()
    assert turing_sage.split_prequantization_available() is turing_sage.w8a8_available()
    assert kernel.__version__


def test_w8a8_fake_contract_and_fullgraph_leaf():
    """Reference custom_ops.py:171-210: the op returns empty_like(query)."""
    q = torch.empty((1, 4, 129, 128), dtype=torch.bfloat16, device=META)
    k = torch.empty((1, 2, 151, 128), dtype=torch.bfloat16, device=META)
    out = torch.ops.turing_utils.w8a8_attention(q, k, k, "HND", False, -1.0, 0, True, True)
    assert out.shape == q.shape and out.dtype == q.dtype and out.device.type == META
    out = turing_sage.w8a8attn_compiled(q, k, k, is_causal=True, key_tile_tokens=128)
    assert out.shape == q.shape
    q16 = torch.empty((2, 65, 3, 64), dtype=torch.float16, device=META)
    compiled = torch.compile(lambda a, b, c: turing_sage.w8a8attn_compiled(a, b, c, tensor_layout="NHD"),
                             backend="eager", fullgraph=True)
    out = compiled(q16, q16, q16)
    assert out.shape == q16.shape and out.dtype == torch.float16


def test_w8a8_refusals():
    q = torch.zeros((1, 2, 64, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA"):
        core.w8a8attn(q, q, q)
    with pytest.raises(ValueError, match="CUDA"):
        core.prequantize_sol_sageattn(q, q, q, use_w8a8=True, force_dense=True)
    with pytest.raises(ValueError, match="dense W8A8"):
        core.prequantize_sol_sageattn(q, q, q, use_w8a8=False, force_dense=True)
    with pytest.raises(ValueError, match="tensor_layout"):
        core.w8a8attn(q, q, q, tensor_layout="BHSD")
    with pytest.raises(ValueError, match="head_dim"):
        wide = torch.zeros((1, 1, 4, 130), dtype=torch.bfloat16)
        core.w8a8attn(wide, wide, wide)
    with pytest.raises(ValueError, match="divisible"):
        core.w8a8attn(q, q[:, :1].expand(1, 3, 64, 128), q[:, :1].expand(1, 3, 64, 128))
    with pytest.raises(ValueError, match="key_tile_tokens"):
        core._key_tile_tokens(96, 100)
    assert core._key_tile_tokens(0, 1025) == 128 and core._key_tile_tokens(0, 1024) == 64
    with pytest.raises(ValueError, match="CUDA"):
        quant.per_warp_int8_hadamard(q, q)
    with pytest.raises(ValueError, match="BLKQ"):
        quant.per_warp_int8_hadamard(q, q, BLKQ=128)


def test_key_splits_refused_for_causal_attention():
    """attention_from_vt checks an explicit kv_splits before any kernel call:
    it must be >= 1, and 1 for causal attention (the split kernel is
    non-causal)."""
    q8 = torch.zeros(1, 2, 300, 128, dtype=torch.int8)
    k8 = torch.zeros(1, 2, 2000, 128, dtype=torch.int8)
    qs = torch.ones(1, 2, 3)
    ks = torch.ones(1, 2, 16)
    vt = torch.zeros(1, 2, 128, 2048, dtype=torch.bfloat16)
    for splits, causal in ((2, True), (0, False)):
        with pytest.raises(ValueError, match="kv_splits"):
            core.attention_from_vt(q8, qs, k8, ks, vt, is_causal=causal, kv_splits=splits)


def test_key_split_workspace_checked_and_sized():
    """A caller workspace for a split call is checked before any kernel call,
    and split_workspace_bytes matches what tu_sage_attn_fwd_split requires:
    ranges x B x H x Lq x (D + 2) fp32 values, ranges = ceil(tiles / per)."""
    q8 = torch.zeros(1, 2, 300, 128, dtype=torch.int8)
    k8 = torch.zeros(1, 2, 2000, 128, dtype=torch.int8)
    qs = torch.ones(1, 2, 3)
    ks = torch.ones(1, 2, 16)
    vt = torch.zeros(1, 2, 128, 2048, dtype=torch.bfloat16)
    need = core.split_workspace_bytes(1, 2, 300, 2000, 128, 2) // 4
    assert need == 2 * 1 * 2 * 300 * 130
    # 32 tiles over 5 ranges: 7 per range covers them in 5 ranges
    assert core.split_workspace_bytes(1, 1, 1, 2048, 64, 5) == 5 * 66 * 4
    # 33 tiles over 8 ranges: 5 per range covers them in 7 ranges
    assert core.split_workspace_bytes(2, 3, 10, 2049, 128, 8) == 7 * 2 * 3 * 10 * 130 * 4
    for bad in (torch.zeros(need - 1), torch.zeros(need, dtype=torch.float64), torch.zeros(2 * need)[::2]):
        with pytest.raises(ValueError, match="workspace"):
            core.attention_from_vt(q8, qs, k8, ks, vt, kv_splits=2, workspace=bad)


def test_preflight_refuses_cpu():
    with pytest.raises(RuntimeError, match="GPU"):
        turing_sage.preflight(torch.device("cpu"))


# correctness gate (reference tests/test_attention_correctness.py:19-51)
def test_metrics_accept_identical_tensors():
    ref = torch.tensor(((1.0, -2.0), (0.5, 4.0)))
    res = attention_error_metrics(ref.clone(), ref)
    assert res.finite and res.max_abs == 0.0 and res.relative_l2 == 0.0
    assert abs(res.cosine - 1.0) < 1e-6
    require_attention_correctness(res, max_abs=0.0, relative_l2=0.0, cosine=0.999)


def test_gate_reports_every_failed_bound():
    res = attention_error_metrics(torch.tensor((1.0, float("nan"))), torch.tensor((0.0, 1.0)),
                                  candidate_name="sol", reference_name="sage", selected_blocks=3, possible_blocks=4)
    with pytest.raises(AssertionError, match="non-finite output") as raised:
        require_attention_correctness(res, max_abs=0.1, relative_l2=0.1, cosine=0.99)
    assert "selected 3/4" in str(raised.value)


def test_gate_names_each_bound():
    res = attention_error_metrics(torch.tensor((1.0, 0.0)), torch.tensor((0.0, 1.0)))
    with pytest.raises(AssertionError) as raised:
        require_attention_correctness(res, max_abs=0.1, relative_l2=0.1, cosine=0.99)
    text = str(raised.value)
    assert "max_abs" in text and "relative_l2" in text and "cosine" in text


def test_shape_mismatch_fails_before_reduction():
    with pytest.raises(AssertionError, match="shape"):
        attention_error_metrics(torch.zeros(2), torch.zeros(3))


def test_qk_rms_rope_fake_contract_and_fullgraph_leaf():
    """Reference tests/test_turing_sage_quant.py:22-90."""
    from comfyui_turing_utils_kernel.turing_sage.custom_ops import qk_rms_rope_int8

    query = torch.empty((2, 4, 129, 128), dtype=torch.bfloat16, device=META)
    key = torch.empty((2, 2, 129, 128), dtype=torch.bfloat16, device=META)
    norm = torch.empty((128,), dtype=torch.bfloat16, device=META)
    freqs = torch.empty((1, 129, 1, 64, 2, 2), dtype=torch.bfloat16, device=META)
    qi, qs, ki, ks = qk_rms_rope_int8(query, key, norm, norm, freqs, 1e-6, 128, "HND", "head", True, False, False)
    assert qi.shape == query.shape and qi.dtype == torch.int8 and qs.shape == (2, 4, 12)
    assert ki.shape == key.shape and ks.shape == (2, 2, 3) and ks.dtype == torch.float32
    q64 = torch.empty((1, 129, 4, 64), dtype=torch.float16, device=META)
    k64 = torch.empty((1, 129, 2, 64), dtype=torch.float16, device=META)
    n64 = torch.empty((64,), dtype=torch.float16, device=META)
    compiled = torch.compile(
        lambda q, k, qw, kw, f: qk_rms_rope_int8(q, k, qw, kw, f, 1e-6, 0, "NHD", "head", False, False, False),
        backend="eager", fullgraph=True)
    qi, qs, ki, ks = compiled(q64, k64, n64, n64, torch.empty((0,), dtype=torch.float16, device=META))
    assert qi.shape == q64.shape and qs.shape == (1, 4, 12) and ks.shape == (1, 2, 3)


def test_qk_rms_rope_refuses_what_is_not_built():
    from comfyui_turing_utils_kernel.turing_sage.quant import rms_rope_per_warp_int8

    x = torch.zeros((1, 2, 16, 128), dtype=torch.bfloat16)
    w = torch.ones(128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="head_dim"):
        rms_rope_per_warp_int8(x[..., :96], x[..., :96], w, w, None, epsilon=1e-6, rot_dim=0,
                               tensor_layout="HND", norm_scope="head", split_half=False)
    with pytest.raises(ValueError, match="norm weight"):
        rms_rope_per_warp_int8(x, x, w, w, None, epsilon=1e-6, rot_dim=0, tensor_layout="HND", norm_scope="row",
                               split_half=False)


def test_layer_norm_adaln_fake_contract_and_refusals():
    """reference ops.py:399-418: empty_like fake; CPU tensors and non-3D or
    integer inputs refused before any launch."""
    x = torch.empty((2, 9, 5120), dtype=torch.bfloat16, device=META)
    mod = torch.empty((2, 4, 5120), dtype=torch.bfloat16, device=META)
    out = torch.ops.turing_utils.layer_norm_adaln(x, mod, mod, 1e-6)
    assert out.shape == x.shape and out.dtype == x.dtype and out.device.type == META
    compiled = torch.compile(lambda a, s, t: kernel.turing_layer_norm_adaln(a, s, t, 1e-6), backend="eager",
                             fullgraph=True)
    assert compiled(x, mod, mod).shape == x.shape
    cpu = torch.zeros((1, 4, 64), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA|HIP"):
        kernel.turing_layer_norm_adaln(cpu, cpu[:, :1], cpu[:, :1])
    assert "turing_layer_norm_adaln" in kernel.__all__


def test_layer_norm_convrot_fake_contract_and_refusals():
    """The LayerNorm-fused ConvRot quantizers (no reference op): codes
    [rows, H] int8 and row scales [rows, 1] fp32, as bf16_int8_convrot_quantize
    returns them; CPU tensors refused before any launch."""
    x = torch.empty((2, 9, 5120), dtype=torch.bfloat16, device=META)
    mod = torch.empty((2, 4, 5120), dtype=torch.bfloat16, device=META)
    q, s = torch.ops.turing_utils.layer_norm_adaln_int8_convrot_quantize(x, mod, mod, 1e-6, 128)
    assert q.shape == (18, 5120) and q.dtype == torch.int8 and q.device.type == META
    assert s.shape == (18, 1) and s.dtype == torch.float32
    w = torch.empty((5120,), dtype=torch.bfloat16, device=META)
    q, s = torch.ops.turing_utils.layer_norm_affine_int8_convrot_quantize(x, w, w, 1e-6, 128)
    assert q.shape == (18, 5120) and s.shape == (18, 1)
    compiled = torch.compile(
        lambda a, m: kernel.turing_layer_norm_adaln_int8_convrot_quantize(a, m, m, 1e-6, 128), backend="eager",
        fullgraph=True)
    assert compiled(x, mod)[0].shape == (18, 5120)
    cpu = torch.zeros((1, 4, 256), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="CUDA|HIP"):
        kernel.turing_layer_norm_adaln_int8_convrot_quantize(cpu, cpu[:, :1], cpu[:, :1])
    with pytest.raises(RuntimeError, match="CUDA|HIP"):
        kernel.turing_layer_norm_affine_int8_convrot_quantize(cpu[0], cpu[0, 0], cpu[0, 0])
    for name in ("turing_layer_norm_adaln_int8_convrot_quantize", "turing_layer_norm_affine_int8_convrot_quantize"):
        assert name in kernel.__all__
