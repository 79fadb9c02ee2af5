"""GPU parity: Sage prologue (K mean, per-block INT8 Q/K) bit-exact vs the oracle,
and Sage attention vs the oracle's quantized math within the north-star gate
(cosine >= 0.999, max-abs <= 2e-2), plus the reference's own SDPA gate.

Oracle: or_sage_kmean, or_sage_quant (fused.cu:66-200), or_sage_attn_rows
(qk_int_sv_f16_cuda_sm75.cu:117-118, :375-381; attn_utils.cuh:464-568).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from comfyui_turing_utils_kernel.turing_sage import core, quant
from comfyui_turing_utils_kernel.turing_sage.correctness import (
    attention_error_metrics,
    require_attention_correctness,
)
from oracle import oracle
from tests import inputs

pytestmark = pytest.mark.gpu

GATE = dict(max_abs=2e-2, cosine=0.999)


@pytest.mark.parametrize("b,h,l,d,seed", [(1, 2, 1, 128, 1), (2, 3, 300, 128, 2), (1, 4, 1000, 64, 3), (1, 12, 8190, 128, 1)])
def test_kmean_exact(gpu_device, b, h, l, d, seed):
    print(f"[kmean] b={b} h={h} l={l} d={d}", flush=True)
    _, k, _ = inputs.attention(b, h, l, d, seed)
    mean = quant.key_channel_mean(k.to(gpu_device), "HND")
    np.testing.assert_array_equal(inputs.bits(mean), oracle.sage_kmean(inputs.bits(k)))


@pytest.mark.parametrize("blk", [16, 32, 64, 128])
@pytest.mark.parametrize("smooth", [False, True])
@pytest.mark.parametrize("b,h,l,d", [(1, 2, 77, 128), (2, 3, 300, 64), (1, 4, 513, 128)])
def test_quant_exact(gpu_device, blk, smooth, b, h, l, d):
    print(f"[sage-quant] blk={blk} smooth={smooth} b={b} h={h} l={l} d={d}", flush=True)
    _, k, _ = inputs.attention(b, h, l, d, blk + l)
    kd = k.to(gpu_device)
    mean = quant.key_channel_mean(kd, "HND") if smooth else None
    q8, sc = quant.quantize_per_block(kd, blk, "HND", mean)
    mean_ref = oracle.sage_kmean(inputs.bits(k)) if smooth else None
    q_ref, s_ref = oracle.sage_quant(inputs.bits(k), blk, mean_ref)
    np.testing.assert_array_equal(sc.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(q8.cpu().numpy(), q_ref)


def test_quant_nhd_matches_hnd(gpu_device):
    _, k, _ = inputs.attention(2, 5, 200, 128, 7)
    kd = k.to(gpu_device)
    q_hnd, s_hnd = quant.quantize_per_block(kd, 64, "HND", quant.key_channel_mean(kd, "HND"))
    kn = kd.transpose(1, 2).contiguous()
    q_nhd, s_nhd = quant.quantize_per_block(kn, 64, "NHD", quant.key_channel_mean(kn, "NHD"))
    assert torch.equal(q_hnd, q_nhd.transpose(1, 2))
    assert torch.equal(s_hnd, s_nhd)


def _oracle_rows(q, k, v, rows, blkq, blkk, causal, sm_scale, smooth=True):
    """Oracle attention for (b, h, i) rows of HND bf16 inputs (head_dim <= 128)."""
    d = q.size(-1)
    pad = 128 - d
    qp, kp, vp = (torch.nn.functional.pad(t, (0, pad)) if pad else t for t in (q, k, v))
    mean = oracle.sage_kmean(inputs.bits(kp)) if smooth else None
    q8, qs = oracle.sage_quant(inputs.bits(qp), blkq)
    k8, ks = oracle.sage_quant(inputs.bits(kp), blkk, mean)
    out = oracle.sage_attn_rows(q8, qs, blkq, k8, ks, blkk, inputs.bits(vp), sm_scale, rows, causal)
    return out[:, :d]


def _sample_rows(b, h, l, n, seed):
    rng = np.random.default_rng(seed)
    rows = np.stack([rng.integers(0, b, n), rng.integers(0, h, n), rng.integers(0, l, n)], 1)
    rows[: min(n, 2), 2] = [0, l - 1][: min(n, 2)]
    return rows


@pytest.mark.parametrize(
    "b,h,hkv,lq,lk,d,causal,blkq,blkk",
    [
        (1, 2, 2, 256, 256, 128, False, 128, 128),
        (1, 2, 2, 300, 333, 128, False, 128, 128),
        (2, 4, 2, 65, 73, 128, False, 16, 64),
        (1, 2, 1, 1, 64, 128, False, 128, 128),
        (1, 3, 3, 700, 700, 128, True, 128, 128),
        (1, 2, 2, 130, 257, 64, False, 32, 64),
        (1, 2, 2, 129, 200, 96, True, 64, 128),
    ],
)
def test_attention_vs_oracle(gpu_device, b, h, hkv, lq, lk, d, causal, blkq, blkk):
    print(f"[attn] b={b} h={h} hkv={hkv} lq={lq} lk={lk} d={d} causal={causal} blk=({blkq},{blkk})", flush=True)
    q, _, _ = inputs.attention(b, h, lq, d, 100 + lq)
    _, k, v = inputs.attention(b, hkv, lk, d, 200 + lk)
    sm = d ** -0.5
    out = core.sageattn(q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), tensor_layout="HND",
                        is_causal=causal, BLKQ=blkq, BLKK=blkk)
    torch.cuda.synchronize(gpu_device)
    rows = _sample_rows(b, h, lq, 96, lq + lk)
    ref = _oracle_rows(q, k, v, rows, blkq, blkk, causal, sm)
    got = out.float().cpu()[rows[:, 0], rows[:, 1], rows[:, 2]]
    res = attention_error_metrics(got, torch.from_numpy(ref), candidate_name="hip", reference_name="oracle")
    print(f"  cos={res.cosine:.6f} max_abs={res.max_abs:.3e}", flush=True)
    require_attention_correctness(res, **GATE)


@pytest.mark.parametrize("b,h,hkv,l,causal,blkq,blkk", [
    (1, 12, 12, 8190, True, 128, 128),   # config 2's shape, causal
    (2, 8, 2, 2049, False, 16, 64),      # batch 2, GQA 4:1, the reference's production blocks
    (2, 8, 2, 2049, True, 16, 64),
])
def test_attention_long_causal_and_gqa(gpu_device, b, h, hkv, l, causal, blkq, blkk):
    """Long sequences with the causal diagonal crossing many key tiles, and
    batch-2 GQA: sampled rows (first and last row included) against the
    oracle within the gate."""
    print(f"[attn long] b={b} h={h} hkv={hkv} l={l} causal={causal} blk=({blkq},{blkk})", flush=True)
    q, _, _ = inputs.attention(b, h, l, 128, 300 + h)
    _, k, v = inputs.attention(b, hkv, l, 128, 400 + h)
    out = core.sageattn(q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), tensor_layout="HND",
                        is_causal=causal, BLKQ=blkq, BLKK=blkk)
    torch.cuda.synchronize(gpu_device)
    rows = _sample_rows(b, h, l, 128, l + h)
    ref = _oracle_rows(q, k, v, rows, blkq, blkk, causal, 128 ** -0.5)
    got = out.float().cpu()[rows[:, 0], rows[:, 1], rows[:, 2]]
    res = attention_error_metrics(got, torch.from_numpy(ref), candidate_name="hip", reference_name="oracle")
    print(f"  cos={res.cosine:.6f} max_abs={res.max_abs:.3e}", flush=True)
    require_attention_correctness(res, **GATE)


def test_attention_config2_rows(gpu_device):
    """BASELINE config 2 (B1 H12 L8190 D128, seed 1), 256 sampled rows vs the oracle."""
    q, k, v = inputs.attention(1, 12, 8190, 128, 1)
    out = core.sageattn(q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), tensor_layout="HND")
    torch.cuda.synchronize(gpu_device)
    rows = _sample_rows(1, 12, 8190, 256, 1)
    ref = _oracle_rows(q, k, v, rows, 128, 128, False, 128 ** -0.5)
    got = out.float().cpu()[rows[:, 0], rows[:, 1], rows[:, 2]]
    res = attention_error_metrics(got, torch.from_numpy(ref), candidate_name="hip", reference_name="oracle")
    print(f"  cos={res.cosine:.6f} max_abs={res.max_abs:.3e}", flush=True)
    require_attention_correctness(res, **GATE)


@pytest.mark.parametrize("b,h,hkv,lq,lk,d,blkq,blkk,splits", [
    (1, 12, 12, 8190, 8190, 128, 128, 128, 2),   # config 2: the split the planner picks
    (1, 4, 4, 700, 1000, 128, 128, 128, 3),      # ragged key tail in the last range
    (2, 8, 2, 300, 2049, 128, 16, 64, 5),        # GQA, blkk 64, 33 tiles in ranges of 7: a 1-key last tile
    (1, 4, 4, 513, 1600, 128, 128, 128, 5),      # 25 tiles over 5 ranges of 5: each starts mid K-scale block
    (1, 6, 3, 257, 777, 64, 32, 64, 4),          # head_dim 64
    (1, 2, 2, 1, 64, 128, 128, 128, 1),          # one tile: no split
])
def test_attention_key_splits(gpu_device, b, h, hkv, lq, lk, d, blkq, blkk, splits):
    """Key-split attention (tu_sage_attn_fwd_split: key ranges merged by a
    second kernel) against the oracle within the gate, and against the
    unsplit kernel on the same quantized inputs (the two differ only by the
    fp32 merge and by P's bf16 rounding against each range's own base)."""
    print(f"[attn split] b={b} h={h} hkv={hkv} lq={lq} lk={lk} d={d} blk=({blkq},{blkk}) splits={splits}", flush=True)
    q, _, _ = inputs.attention(b, h, lq, d, 500 + lq)
    _, k, v = inputs.attention(b, hkv, lk, d, 600 + lk)
    state = core.prequantize_sageattn(q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), "HND",
                                      BLKQ=blkq, BLKK=blkk)
    args = (state.query_int8, state.query_scale, state.key_int8, state.key_scale, state.value_t)
    kw = dict(tensor_layout="HND", sm_scale=d ** -0.5, blkq=blkq, blkk=blkk)
    split = core.attention_from_vt(*args, **kw, kv_splits=splits)
    whole = core.attention_from_vt(*args, **kw, kv_splits=1)
    torch.cuda.synchronize(gpu_device)
    rows = _sample_rows(b, h, lq, 96, lq + lk + splits)
    ref = _oracle_rows(q, k, v, rows, blkq, blkk, False, d ** -0.5)
    got = split.float().cpu()[rows[:, 0], rows[:, 1], rows[:, 2]]
    res = attention_error_metrics(got, torch.from_numpy(ref), candidate_name="split", reference_name="oracle")
    print(f"  vs oracle cos={res.cosine:.6f} max_abs={res.max_abs:.3e}", flush=True)
    require_attention_correctness(res, **GATE)
    both = attention_error_metrics(split.float().cpu().flatten(1), whole.float().cpu().flatten(1),
                                   candidate_name="split", reference_name="whole")
    print(f"  vs unsplit cos={both.cosine:.7f} max_abs={both.max_abs:.3e}", flush=True)
    assert both.cosine >= 0.99999 and both.max_abs <= 1e-2
    if splits == 1:
        assert torch.equal(split, whole)
    else:
        # a caller workspace (stale NaN contents) gives the same bits
        need = core.split_workspace_bytes(b, h, lq, lk, d, splits) // 4
        ws = torch.full((need + 5,), float("nan"), dtype=torch.float32, device=gpu_device)
        again = core.attention_from_vt(*args, **kw, kv_splits=splits, workspace=ws)
        torch.cuda.synchronize(gpu_device)
        assert torch.equal(again, split)


def test_attention_key_splits_nhd_layout(gpu_device):
    """The merge kernel writes through the output strides: a split NHD call
    (the planner splits B1 H8 L4096 in two) equals the HND call bit for bit."""
    q, k, v = inputs.attention(1, 8, 4096, 128, 21)
    qd, kd, vd = q.to(gpu_device), k.to(gpu_device), v.to(gpu_device)
    hnd = core.sageattn(qd, kd, vd, tensor_layout="HND")
    nhd = core.sageattn(qd.transpose(1, 2).contiguous(), kd.transpose(1, 2).contiguous(),
                        vd.transpose(1, 2).contiguous(), tensor_layout="NHD")
    torch.cuda.synchronize(gpu_device)
    assert torch.equal(nhd.transpose(1, 2), hnd)


def test_attention_nhd_and_op(gpu_device):
    """NHD layout through torch.ops.turing_utils.sage_attention equals the HND facade."""
    q, k, v = inputs.attention(2, 4, 200, 128, 5)
    dev = gpu_device
    hnd = core.sageattn(q.to(dev), k.to(dev), v.to(dev), tensor_layout="HND")
    nhd = torch.ops.turing_utils.sage_attention(
        q.transpose(1, 2).contiguous().to(dev), k.transpose(1, 2).contiguous().to(dev),
        v.transpose(1, 2).contiguous().to(dev), "NHD", False, -1.0,
    )
    assert torch.equal(hnd, nhd.transpose(1, 2))


def test_attention_reference_sdpa_gate(gpu_device):
    """The reference preflight's gate (turing_sage/__init__.py:612-663): arange-modulo
    inputs vs fp32 SDPA, rtol 0.08 / atol 0.05, head_dim 64/96/128, GQA 4:2."""
    from comfyui_turing_utils_kernel import turing_sage

    turing_sage.preflight(gpu_device)


def test_smoothing_invariance(gpu_device):
    """Subtracting the K mean shifts every score of a row by a constant, so the
    smoothed and unsmoothed kernels agree within the quantization tolerance."""
    q, k, v = inputs.attention(1, 4, 512, 128, 9)
    dev = gpu_device
    a = core.sageattn(q.to(dev), k.to(dev), v.to(dev), smooth_k=True)
    b = core.sageattn(q.to(dev), k.to(dev), v.to(dev), smooth_k=False)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
    ea = attention_error_metrics(a.float().cpu(), ref)
    eb = attention_error_metrics(b.float().cpu(), ref)
    print(f"  smoothed cos={ea.cosine:.6f} raw cos={eb.cosine:.6f}", flush=True)
    assert ea.cosine >= 0.999 and ea.cosine >= eb.cosine - 1e-4


@pytest.mark.parametrize("b,h,hkv,lq,lk,d,causal,layout", [
    (1, 4, 4, 300, 333, 64, False, "HND"),
    (2, 4, 2, 257, 129, 64, True, "HND"),
    (1, 3, 3, 200, 700, 48, False, "NHD"),
    (1, 24, 24, 8190, 8190, 64, False, "HND"),
])
def test_head_dim_64_kernel(gpu_device, b, h, hkv, lq, lk, d, causal, layout):
    """head_dim <= 64 runs the 64-wide kernel (V^T of 64 channels, as the
    reference pads to 64, turing_sage/core.py:436-448) and meets the gate
    against the oracle's quantized math."""
    print(f"[attn d64] b={b} h={h} hkv={hkv} lq={lq} lk={lk} d={d} causal={causal} {layout}", flush=True)
    q, _, _ = inputs.attention(b, h, lq, d, 300 + lq)
    _, k, v = inputs.attention(b, hkv, lk, d, 400 + lk)
    to = (lambda t: t.transpose(1, 2).contiguous()) if layout == "NHD" else (lambda t: t)
    state = core.prequantize_sageattn(to(q).to(gpu_device), to(k).to(gpu_device), to(v).to(gpu_device),
                                      tensor_layout=layout, is_causal=causal)
    assert state.value_t.shape[2] == 64 and state.query_int8.shape[-1] == 64
    out = core.sageattn_from_prequantized(state)
    torch.cuda.synchronize(gpu_device)
    out = out.transpose(1, 2) if layout == "NHD" else out
    assert out.shape == q.shape
    rows = _sample_rows(b, h, lq, 128, lq + lk + d)
    ref = _oracle_rows(q, k, v, rows, 128, 128, causal, d ** -0.5)
    got = out.float().cpu()[rows[:, 0], rows[:, 1], rows[:, 2]]
    res = attention_error_metrics(got, torch.from_numpy(ref), candidate_name="hip", reference_name="oracle")
    print(f"  cos={res.cosine:.6f} max_abs={res.max_abs:.3e}", flush=True)
    require_attention_correctness(res, **GATE)


def test_head_dim_64_matches_the_128_wide_kernel(gpu_device):
    """Zero channels change neither the codes nor the result: the 64-wide
    kernel equals the 128-wide kernel on the same inputs padded to 128, to
    the last rounding of the PV sums."""
    q, k, v = inputs.attention(1, 4, 513, 64, 77)
    dev = gpu_device
    o64 = core.sageattn(q.to(dev), k.to(dev), v.to(dev))
    pad = lambda t: torch.nn.functional.pad(t, (0, 64)).to(dev)  # noqa: E731
    o128 = core.sageattn(pad(q), pad(k), pad(v), sm_scale=64 ** -0.5)[..., :64]
    torch.cuda.synchronize(dev)
    assert o64.shape == o128.shape
    diff = (o64.float() - o128.float()).abs().max().item()
    assert diff <= 2 ** -7 * o128.float().abs().max().item(), diff
