"""Known-answer vectors (tests/golden/kat.npz, written by tests/golden/make_golden.py
from dense-matrix / plain-numpy derivations) checked against the C oracle on
the CPU and against the HIP kernels on the GPU."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import oracle
from tests import inputs

KAT = np.load(os.path.join(os.path.dirname(__file__), "golden", "kat.npz"))
SM = np.float32(128 ** -0.5)
ATTN_CASES = [(16, 64, False), (16, 64, True), (128, 128, False)]


def _attn_rows(lq, hq):
    return np.array([[0, h, i] for h in range(hq) for i in range(lq)], np.int64)


# ---------------------------------------------------------------- oracle (CPU)
@pytest.mark.parametrize("group", [128, 256])
def test_oracle_convrot_kat(group):
    q, s = oracle.convrot_quant(KAT["convrot_x"], group)
    np.testing.assert_array_equal(q, KAT[f"convrot_q_g{group}"])
    np.testing.assert_array_equal(s.view(np.uint32), KAT[f"convrot_scale_g{group}"].view(np.uint32))


def test_oracle_gemm_kat():
    acc = oracle.int8_gemm_i32(KAT["gemm_a"], KAT["gemm_w"])
    np.testing.assert_array_equal(acc, KAT["gemm_acc"])
    out = oracle.epilogue_bf16(acc, KAT["gemm_a_scale"], KAT["gemm_w_scale"], KAT["gemm_bias"])
    np.testing.assert_array_equal(out, KAT["gemm_out_bias"])
    np.testing.assert_array_equal(oracle.epilogue_bf16(acc, KAT["gemm_a_scale"], KAT["gemm_w_scale"], None),
                                  KAT["gemm_out"])


def test_oracle_sage_quant_kat():
    mean = oracle.sage_kmean(KAT["sage_k"])
    np.testing.assert_array_equal(mean, KAT["sage_kmean"])
    for blkq, blkk in ((16, 64), (128, 128)):
        q8, qs = oracle.sage_quant(KAT["sage_q"], blkq)
        np.testing.assert_array_equal(q8, KAT[f"sage_q8_b{blkq}"])
        np.testing.assert_array_equal(qs.view(np.uint32), KAT[f"sage_qs_b{blkq}"].view(np.uint32))
        k8, ks = oracle.sage_quant(KAT["sage_k"], blkk, mean)
        np.testing.assert_array_equal(k8, KAT[f"sage_k8_b{blkk}"])
        np.testing.assert_array_equal(ks.view(np.uint32), KAT[f"sage_ks_b{blkk}"].view(np.uint32))


@pytest.mark.parametrize("blkq,blkk,causal", ATTN_CASES)
def test_oracle_attention_kat(blkq, blkk, causal):
    q8, qs = KAT[f"sage_q8_b{blkq}"], KAT[f"sage_qs_b{blkq}"]
    k8, ks = KAT[f"sage_k8_b{blkk}"], KAT[f"sage_ks_b{blkk}"]
    out = oracle.sage_attn_rows(q8, qs, blkq, k8, ks, blkk, KAT["sage_v"], SM, _attn_rows(q8.shape[2], q8.shape[1]),
                                causal)
    ref = KAT[f"sage_out_q{blkq}_k{blkk}_c{int(causal)}"].reshape(out.shape)
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-5)


# ------------------------------------------------------------------- HIP (GPU)
@pytest.mark.gpu
@pytest.mark.parametrize("group", [128, 256])
def test_hip_convrot_kat(gpu_device, group):
    print(f"[kat convrot] group={group}", flush=True)
    x = inputs.from_bits(KAT["convrot_x"]).to(gpu_device)
    q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(x, group)
    np.testing.assert_array_equal(q.cpu().numpy(), KAT[f"convrot_q_g{group}"])
    np.testing.assert_array_equal(s.cpu().numpy().reshape(-1).view(np.uint32),
                                  KAT[f"convrot_scale_g{group}"].view(np.uint32))


@pytest.mark.gpu
def test_hip_gemm_kat(gpu_device):
    print("[kat gemm]", flush=True)
    a = torch.from_numpy(KAT["gemm_a"]).to(gpu_device)
    w = torch.from_numpy(KAT["gemm_w"]).to(gpu_device)
    acc = torch.ops.turing_utils.int8_gemm_i32(a, w)
    np.testing.assert_array_equal(acc.cpu().numpy(), KAT["gemm_acc"])
    as_ = torch.from_numpy(KAT["gemm_a_scale"]).to(gpu_device)
    ws = torch.from_numpy(KAT["gemm_w_scale"]).to(gpu_device)
    bias = torch.from_numpy(KAT["gemm_bias"]).to(gpu_device)
    out = torch.ops.turing_utils.int8_linear(a, w, as_, ws, bias)
    np.testing.assert_array_equal(inputs.bits(out), KAT["gemm_out_bias"])
    out = torch.ops.turing_utils.dequantize_int8_bf16(acc, as_, ws)
    np.testing.assert_array_equal(inputs.bits(out), KAT["gemm_out"])


@pytest.mark.gpu
@pytest.mark.parametrize("blkq,blkk,causal", ATTN_CASES)
def test_hip_sage_kat(gpu_device, blkq, blkk, causal):
    from comfyui_turing_utils_kernel.turing_sage import core, quant

    print(f"[kat sage] blkq={blkq} blkk={blkk} causal={causal}", flush=True)
    q = inputs.from_bits(KAT["sage_q"]).to(gpu_device)
    k = inputs.from_bits(KAT["sage_k"]).to(gpu_device)
    v = inputs.from_bits(KAT["sage_v"]).to(gpu_device)
    mean = quant.key_channel_mean(k, "HND")
    np.testing.assert_array_equal(inputs.bits(mean), KAT["sage_kmean"])
    q8, qs = quant.quantize_per_block(q, blkq, "HND")
    k8, ks = quant.quantize_per_block(k, blkk, "HND", mean)
    np.testing.assert_array_equal(q8.cpu().numpy(), KAT[f"sage_q8_b{blkq}"])
    np.testing.assert_array_equal(k8.cpu().numpy(), KAT[f"sage_k8_b{blkk}"])
    np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint32), KAT[f"sage_qs_b{blkq}"].view(np.uint32))
    np.testing.assert_array_equal(ks.cpu().numpy().view(np.uint32), KAT[f"sage_ks_b{blkk}"].view(np.uint32))
    out = core.sageattn_prequantized(q8, qs, k8, ks, v, is_causal=causal, sm_scale=float(SM), blkq=blkq, blkk=blkk)
    ref = torch.from_numpy(KAT[f"sage_out_q{blkq}_k{blkk}_c{int(causal)}"])
    got = out.float().cpu()
    assert (got - ref).abs().max().item() <= 2e-2
    cos = torch.nn.functional.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item()
    assert cos >= 0.999
