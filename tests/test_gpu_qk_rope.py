"""GPU parity: fused Q/K RMSNorm + RoPE + INT8 (HIP, tu_qk_rms_rope_int8) vs the
CPU oracle, bit-exact codes and scales, and the reference's own known-answer
check against its preprocessing formula (kernel/scripts/validate_compatible.py
:241-421: codes within 2 LSB, scales rtol 0.015 / atol 0.0011).

Oracle: oracle/tu_oracle.c or_qk_rms_rope_int8, a restatement of
kernel/csrc/turing/sage/qk_preprocess.cu:99-197, :417-629.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from tests.test_oracle_qk_rope import _per_block_int8, _reference_formula

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _hnd(t: torch.Tensor, layout: str) -> torch.Tensor:
    return t if layout == "HND" else t.transpose(1, 2)


def _case(b, hq, hk, l, d, dtype, scope, rot, fb, fl, seed, layout="HND"):
    g = torch.Generator().manual_seed(seed)
    shape_q = (b, hq, l, d) if layout == "HND" else (b, l, hq, d)
    shape_k = (b, hk, l, d) if layout == "HND" else (b, l, hk, d)
    q = (torch.randn(shape_q, generator=g) * 2).to(dtype)
    k = (torch.randn(shape_k, generator=g) * 2).to(dtype)
    qw = torch.randn(d if scope == "head" else hq * d, generator=g).to(dtype)
    kw = torch.randn(d if scope == "head" else hk * d, generator=g).to(dtype)
    freqs = torch.randn((fb, fl, 1, rot // 2, 2, 2), generator=g).to(dtype) if rot else None
    return q, k, qw, kw, freqs


def _check_exact(q, k, qw, kw, freqs, rot, scope, split, layout, dev):
    from comfyui_turing_utils_kernel.turing_sage.custom_ops import qk_rms_rope_int8

    empty = torch.empty(0, dtype=q.dtype)
    out = qk_rms_rope_int8(q.to(dev), k.to(dev), qw.to(dev), kw.to(dev),
                           (freqs if freqs is not None else empty).to(dev), 1e-6, rot, layout, scope, split,
                           False, False)
    torch.cuda.synchronize(dev)
    qi, qs, ki, ks = (t.cpu() for t in out)
    dt = oracle.DTYPE_FP16 if q.dtype == torch.float16 else oracle.DTYPE_BF16
    f32 = freqs.float()[:, :, 0].numpy() if freqs is not None else None
    for x, w, got_q, got_s, blk in ((q, qw, qi, qs, 16), (k, kw, ki, ks, 64)):
        xh = _hnd(x, layout)
        nt = got_s.shape[-1]
        ref_q, ref_s = oracle.qk_rms_rope_int8(_bits(xh), dt, _bits(w), scope, 1e-6, f32, rot, split, blk, nt)
        np.testing.assert_array_equal(got_s.numpy().view(np.uint32), ref_s.view(np.uint32))
        np.testing.assert_array_equal(_hnd(got_q, layout).contiguous().numpy(), ref_q)
    return qi, qs, ki, ks


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d,scope,split,rot", [(128, "row", False, 128), (128, "head", True, 96),
                                               (64, "head", False, 64), (64, "row", True, 32), (128, "head", False, 0)])
def test_exact_vs_oracle(gpu_device, dtype, d, scope, split, rot):
    print(f"[qk-rope] {dtype} d={d} {scope} split={split} rot={rot}", flush=True)
    q, k, qw, kw, freqs = _case(2, 4, 2, 129, d, dtype, scope, rot, 2, 129, 100 + d + rot)
    _check_exact(q, k, qw, kw, freqs, rot, scope, split, "HND", gpu_device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("hq,hk,rot_full", [(24, 8, True), (17, 1, False), (40, 40, False), (3, 5, True)])
def test_row_scope_head_counts(gpu_device, dtype, d, hq, hk, rot_full):
    """Row-scope RMSNorm with interleaved full-width RoPE (or none): Q in one
    pass over all heads of a 16-token tile (heads split unevenly over the
    workgroup's waves), K through its pre-pass; ragged token count."""
    rot = d if rot_full else 0
    print(f"[qk-rope] row heads {dtype} d={d} hq={hq} hk={hk} rot={rot}", flush=True)
    q, k, qw, kw, freqs = _case(1, hq, hk, 150, d, dtype, "row", rot, 1, 150, 300 + hq + d)
    _check_exact(q, k, qw, kw, freqs, rot, "row", False, "HND", gpu_device)


@pytest.mark.parametrize("dtype,d,rot_full,layout", [(torch.bfloat16, 128, True, "HND"),
                                                     (torch.float16, 128, False, "NHD"),
                                                     (torch.bfloat16, 64, True, "NHD"),
                                                     (torch.float16, 64, True, "HND")])
def test_row_scope_streamed_tiles(gpu_device, dtype, d, rot_full, layout):
    """Row-scope Q with 17-48 heads runs one workgroup per CU that walks
    several 16-token tiles, loading the next tile while it quantizes the
    current one.  Three batches of 7000 tokens give 1320 tiles: every
    workgroup runs five or six of them (an uneven count), across batch
    boundaries and into the ragged and padded tiles; all of it bit-exact."""
    rot = d if rot_full else 0
    print(f"[qk-rope] streamed row {dtype} d={d} rot={rot} {layout}", flush=True)
    q, k, qw, kw, freqs = _case(3, 20, 4, 7000, d, dtype, "row", rot, 3, 7000, 500 + d + rot, layout=layout)
    _check_exact(q, k, qw, kw, freqs, rot, "row", False, layout, gpu_device)


@pytest.mark.parametrize("d", [64, 128])
def test_row_scope_streamed_broadcast_freqs(gpu_device, d):
    """The streamed row-scope Q kernel with one frequency row for every token
    and batch (f_batches = f_len = 1), 33 heads."""
    print(f"[qk-rope] streamed row broadcast freqs d={d}", flush=True)
    q, k, qw, kw, freqs = _case(2, 33, 3, 301, d, torch.bfloat16, "row", d, 1, 1, 900 + d)
    _check_exact(q, k, qw, kw, freqs, d, "row", False, "HND", gpu_device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("scope,hq", [("row", 20), ("row", 4), ("head", 20)])
def test_non_finite_inputs(gpu_device, dtype, scope, hq):
    """NaN, +-inf and the type's largest values in Q and K: a NaN row
    normalizes to NaN and quantizes to -127 while its tile's amax passes it
    over, as fmaxf does; every path (streamed row-scope Q, the one-pass and
    head-group kernels) bit-exact against the oracle."""
    print(f"[qk-rope] non-finite {dtype} {scope} hq={hq}", flush=True)
    q, k, qw, kw, freqs = _case(1, hq, 2, 300, 128, dtype, scope, 128, 1, 300, 77 + hq)
    big = torch.finfo(dtype).max
    for x in (q, k):
        x[0, 0, 5, 3] = float("nan")
        x[0, 1, 40, :] = float("nan")
        x[0, 1, 70, 9] = float("inf")
        x[0, 0, 130, 0] = -float("inf")
        x[0, 1, 200, 17] = big
        x[0, 0, 201, 18] = -big
    _check_exact(q, k, qw, kw, freqs, 128, scope, False, "HND", gpu_device)


@pytest.mark.parametrize("scope", ["head", "row"])
def test_nhd_strided_and_broadcast_freqs(gpu_device, scope):
    """Wan's call: HND views of an NHD projection ([B, L, H, D].transpose(1, 2)),
    interleaved full-width RoPE, frequencies shared by the batch."""
    print(f"[qk-rope] nhd-view {scope}", flush=True)
    q, k, qw, kw, freqs = _case(2, 5, 5, 70, 128, torch.bfloat16, scope, 128, 1, 70, 7, layout="NHD")
    qv, kv = q.transpose(1, 2), k.transpose(1, 2)  # strided HND views
    _check_exact(qv, kv, qw, kw, freqs, 128, scope, False, "HND", gpu_device)
    _check_exact(q, k, qw, kw, freqs, 128, scope, False, "NHD", gpu_device)
    # one frequency row for every token
    q, k, qw, kw, freqs = _case(1, 2, 2, 33, 128, torch.bfloat16, scope, 64, 1, 1, 8)
    _check_exact(q, k, qw, kw, freqs, 64, scope, True, "HND", gpu_device)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d,scope,split", [(64, "head", True), (128, "head", True), (64, "row", False),
                                           (128, "row", False)])
def test_reference_known_answer(gpu_device, dtype, d, scope, split):
    """validate_compatible.py:289-383 on the GPU result."""
    from comfyui_turing_utils_kernel.turing_sage import prequantize_rms_rope_qk

    print(f"[qk-rope] kat {dtype} d={d} {scope}", flush=True)
    g = torch.Generator().manual_seed(4700 + d + (100 if scope == "row" else 0))
    b, h, l = 1, 3, 129
    q = torch.randn((b, h, l, d), generator=g).to(dtype)
    k = torch.randn((b, h, l, d), generator=g).to(dtype)
    nsz = d if scope == "head" else h * d
    qw = torch.randn(nsz, generator=g).to(dtype)
    kw = torch.randn(nsz, generator=g).to(dtype)
    rot = d if scope == "row" else d - 32
    freqs = torch.randn((b, l, 1, rot // 2, 2, 2), generator=g).to(dtype)
    fused = prequantize_rms_rope_qk(q.to(gpu_device), k.to(gpu_device), qw, kw, freqs, epsilon=1e-6, rot_dim=rot,
                                    norm_scope=scope, split_half=split)
    for x, w, gq, gs, blk in ((q, qw, fused.query_int8, fused.query_scale, 16),
                              (k, kw, fused.key_int8, fused.key_scale, 64)):
        ref_q, ref_s = _per_block_int8(_reference_formula(x, w, freqs, 1e-6, rot, scope, split), blk, gs.shape[-1])
        assert int((gq.cpu().to(torch.int16) - ref_q.to(torch.int16)).abs().max()) <= 2
        np.testing.assert_allclose(gs.cpu().numpy(), ref_s.numpy(), rtol=0.015, atol=0.0011)


@pytest.mark.parametrize("d", [64, 128])
def test_prequantized_qk_attention(gpu_device, d):
    """prequantize_rms_rope_qk -> prequantize_sageattn_from_qk -> attention, against
    the oracle's attention on the same codes (16-token Q / 64-token K scales)."""
    from comfyui_turing_utils_kernel.turing_sage import (prequantize_rms_rope_qk, prequantize_sageattn_from_qk,
                                                           sageattn_from_prequantized)
    from comfyui_turing_utils_kernel.turing_sage.correctness import (attention_error_metrics,
                                                                      require_attention_correctness)

    print(f"[qk-rope] attention d={d}", flush=True)
    q, k, qw, kw, freqs = _case(1, 4, 2, 200, d, torch.bfloat16, "row", d, 1, 200, 11)
    v = torch.randn((1, 2, 200, d), generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    qk = prequantize_rms_rope_qk(q.to(gpu_device), k.to(gpu_device), qw, kw, freqs, epsilon=1e-6, rot_dim=d,
                                 norm_scope="row")
    out = sageattn_from_prequantized(prequantize_sageattn_from_qk(qk, v.to(gpu_device))).float().cpu()
    assert out.shape == (1, 4, 200, d)
    q8 = qk.query_int8.cpu().numpy()
    k8 = qk.key_int8.cpu().numpy()
    pad = 128 - d
    q8p = np.pad(q8, ((0, 0), (0, 0), (0, 0), (0, pad)))
    k8p = np.pad(k8, ((0, 0), (0, 0), (0, 0), (0, pad)))
    vp = np.pad(_bits(v), ((0, 0), (0, 0), (0, 0), (0, pad)))
    qs = qk.query_scale.cpu().numpy()[..., : (200 + 15) // 16].copy()
    ks = qk.key_scale.cpu().numpy()
    rows = np.array([[0, h, i] for h in range(4) for i in (0, 1, 15, 16, 63, 64, 127, 199)])
    ref = oracle.sage_attn_rows(q8p, qs, 16, k8p, ks, 64, vp, d ** -0.5, rows)[:, :d]
    got = out[rows[:, 0], rows[:, 1], rows[:, 2]]
    require_attention_correctness(attention_error_metrics(got, torch.from_numpy(ref)), max_abs=2e-2, cosine=0.999)


def test_wan_shape_slices(gpu_device):
    """Wan-14B self-attention producer at full size (B1 H40 L32760 D128, row
    scope, interleaved full-width RoPE): two token slices checked bit-exactly
    (row-scope rrms and tile scales depend only on the slice's tokens)."""
    from comfyui_turing_utils_kernel.turing_sage.custom_ops import qk_rms_rope_int8

    print("[qk-rope] wan B1 H40 L32760", flush=True)
    h, l, d = 40, 32760, 128
    g = torch.Generator().manual_seed(21)
    x = torch.randn((1, l, h, d), generator=g).to(torch.bfloat16)  # one projection serves as Q and K
    w = (1 + 0.1 * torch.randn(h * d, generator=g)).to(torch.bfloat16)
    theta = torch.rand((1, l, 1, d // 2), generator=g) * 6.28
    freqs = torch.stack([torch.stack([theta.cos(), -theta.sin()], -1),
                         torch.stack([theta.sin(), theta.cos()], -1)], -2).to(torch.bfloat16)
    xd = x.to(gpu_device).transpose(1, 2)
    qi, qs, ki, ks = (t.cpu() for t in qk_rms_rope_int8(xd, xd, w.to(gpu_device), w.to(gpu_device),
                                                          freqs.to(gpu_device), 1e-6, d, "HND", "row", False,
                                                          False, False))
    assert qs.shape == (1, h, (l + 63) // 64 * 4) and ks.shape == (1, h, (l + 63) // 64)
    f32 = freqs.float()[:, :, 0].numpy()
    for t0, t1 in ((0, 1024), (31744, l)):  # the last slice ends on the ragged tiles
        xs = x[:, t0:t1].transpose(1, 2).contiguous()
        fs = f32[:, t0:t1]
        rq, rs = oracle.qk_rms_rope_int8(_bits(xs), 0, _bits(w), "row", 1e-6, fs, d, False, 16, (t1 - t0 + 15) // 16)
        np.testing.assert_array_equal(qi[:, :, t0:t1].numpy(), rq)
        np.testing.assert_array_equal(qs[:, :, t0 // 16:(t1 + 15) // 16].numpy().view(np.uint32), rs.view(np.uint32))
        rk, rks = oracle.qk_rms_rope_int8(_bits(xs), 0, _bits(w), "row", 1e-6, fs, d, False, 64, (t1 - t0 + 63) // 64)
        np.testing.assert_array_equal(ki[:, :, t0:t1].numpy(), rk)
        np.testing.assert_array_equal(ks[:, :, t0 // 64:(t1 + 63) // 64].numpy().view(np.uint32), rks.view(np.uint32))


# --- W8A8 variant: rotate_qk / stabilize_k (qk_preprocess.cu:250-416, :417-563) ---

def _check_w8a8_exact(q, k, qw, kw, freqs, rot, scope, split, stabilize, dev):
    from comfyui_turing_utils_kernel.turing_sage.custom_ops import qk_rms_rope_int8

    empty = torch.empty(0, dtype=q.dtype)
    out = qk_rms_rope_int8(q.to(dev), k.to(dev), qw.to(dev), kw.to(dev),
                           (freqs if freqs is not None else empty).to(dev), 1e-6, rot, "HND", scope, split,
                           True, stabilize)
    torch.cuda.synchronize(dev)
    qi, qs, ki, ks = (t.cpu() for t in out)
    dt = oracle.DTYPE_FP16 if q.dtype == torch.float16 else oracle.DTYPE_BF16
    f32 = freqs.float()[:, :, 0].numpy() if freqs is not None else None
    anchors = values = None
    if stabilize:
        anchors, values = oracle.qk_fused_anchor(_bits(k), dt, _bits(kw), scope, 1e-6, f32, rot, split)
    for x, w, got_q, got_s, blk, anc, val in ((q, qw, qi, qs, 16, None, None), (k, kw, ki, ks, 64, anchors, values)):
        ref_q, ref_s = oracle.qk_rms_rope_int8_ex(_bits(x), dt, _bits(w), scope, 1e-6, f32, rot, split, blk,
                                                  got_s.shape[-1], True, anc, val)
        np.testing.assert_array_equal(got_s.numpy().view(np.uint32), ref_s.view(np.uint32))
        np.testing.assert_array_equal(got_q.numpy(), ref_q)
    return anchors


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("d,scope,split,rot", [(128, "row", False, 128), (128, "head", True, 96),
                                               (64, "head", False, 64), (64, "row", True, 32), (128, "head", False, 0)])
@pytest.mark.parametrize("stabilize", [False, True])
def test_w8a8_variant_exact(gpu_device, dtype, d, scope, split, rot, stabilize):
    """Rotated (and anchored) codes and scales bit-exact vs the oracle; one
    frequency row for all tokens keeps the per-head channel offset common, so
    the anchor fires."""
    print(f"[qk-rope-w8a8] {dtype} d={d} {scope} split={split} rot={rot} anchor={stabilize}", flush=True)
    q, k, qw, kw, freqs = _case(2, 4, 2, 131, d, dtype, scope, rot, 2, 1, 300 + d + rot)
    g = torch.Generator().manual_seed(301 + d)
    k = (k.float() + 4 * torch.randn(2, 2, 1, d, generator=g)).to(dtype)
    anchors = _check_w8a8_exact(q, k, qw, kw, freqs, rot, scope, split, stabilize, gpu_device)
    if stabilize:
        assert (anchors >= 0).any()


def test_w8a8_variant_feeds_both_attentions(gpu_device):
    """prequantize_rms_rope_qk(rotate_qk, stabilize_k) -> the W8A8 attention
    (against the oracle's attention on the same codes) and the Sage attention
    (rotation and anchor leave its softmax unchanged: against the unrotated
    producer's result)."""
    from comfyui_turing_utils_kernel.turing_sage import (prequantize_rms_rope_qk, prequantize_sageattn_from_qk,
                                                           sageattn_from_prequantized)
    from comfyui_turing_utils_kernel.turing_sage.core import prequantize_w8a8attn_from_qk, w8a8attn_from_prequantized
    from comfyui_turing_utils_kernel.turing_sage.correctness import (attention_error_metrics,
                                                                      require_attention_correctness)

    print("[qk-rope-w8a8] attention", flush=True)
    q, k, qw, kw, freqs = _case(1, 4, 2, 300, 128, torch.bfloat16, "row", 128, 1, 1, 41)
    k = (k.float() + 3 * torch.randn(1, 2, 1, 128, generator=torch.Generator().manual_seed(42))).to(torch.bfloat16)
    v = torch.randn((1, 2, 300, 128), generator=torch.Generator().manual_seed(43)).to(torch.bfloat16)
    qd, kd, vd = q.to(gpu_device), k.to(gpu_device), v.to(gpu_device)
    qk = prequantize_rms_rope_qk(qd, kd, qw, kw, freqs, epsilon=1e-6, rot_dim=128, norm_scope="row",
                                 rotate_qk=True, stabilize_k=True)
    assert qk.route_original_basis
    out = w8a8attn_from_prequantized(prequantize_w8a8attn_from_qk(qk, vd)).float().cpu()
    f32 = freqs.float()[:, :, 0].numpy()
    anchors, values = oracle.qk_fused_anchor(_bits(k), 0, _bits(kw), "row", 1e-6, f32, 128, False)
    assert (anchors >= 0).any()
    q8, qs = oracle.qk_rms_rope_int8_ex(_bits(q), 0, _bits(qw), "row", 1e-6, f32, 128, False, 16, 20, True)
    k8, ks = oracle.qk_rms_rope_int8_ex(_bits(k), 0, _bits(kw), "row", 1e-6, f32, 128, False, 64, 5, True,
                                        anchors, values)
    v8, vs = oracle.w8a8_quant_v(_bits(v))
    rows = np.array([[0, h, i] for h in range(4) for i in range(300)])
    ref = oracle.w8a8_attn_rows(q8, qs, k8, ks, v8, vs, 300, 128 ** -0.5, rows).reshape(1, 4, 300, 128)
    require_attention_correctness(attention_error_metrics(out, torch.from_numpy(ref)), max_abs=2e-2, cosine=0.999)
    # Sage on rotated + anchored codes against exact attention on the
    # processed Q/K (the rotation is orthogonal, the anchor a per-row shift):
    # as close as Sage on the plain codes
    sage_rot = sageattn_from_prequantized(prequantize_sageattn_from_qk(qk, vd)).float().cpu()
    plain = prequantize_rms_rope_qk(qd, kd, qw, kw, freqs, epsilon=1e-6, rot_dim=128, norm_scope="row")
    sage_plain = sageattn_from_prequantized(prequantize_sageattn_from_qk(plain, vd)).float().cpu()
    pq = torch.from_numpy(oracle.qk_processed(_bits(q), 0, _bits(qw), "row", 1e-6, f32, 128, False)).double()
    pk = torch.from_numpy(oracle.qk_processed(_bits(k), 0, _bits(kw), "row", 1e-6, f32, 128, False)).double()
    exact = torch.nn.functional.scaled_dot_product_attention(pq, pk, v.double(), enable_gqa=True).float()
    m_rot = attention_error_metrics(sage_rot, exact)
    m_plain = attention_error_metrics(sage_plain, exact)
    assert m_rot.cosine > 0.995 and m_rot.relative_l2 <= 1.5 * m_plain.relative_l2 + 0.005, (m_rot, m_plain)
