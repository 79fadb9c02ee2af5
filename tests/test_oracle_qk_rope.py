"""CPU pinning of the oracle's fused Q/K RMSNorm + RoPE + INT8 restatement
(oracle/tu_oracle.c or_qk_rms_rope_int8, following
kernel/csrc/turing/sage/qk_preprocess.cu:99-197, :417-552).

* binary16 conversions against numpy's float16 casts;
* the reference's own known-answer check (kernel/scripts/validate_compatible.py
  :241-421): a torch restatement of the preprocessing formula followed by the
  per-warp INT8 quantizer must agree with the fused result within 2 INT8 LSB,
  scales within rtol 0.015 / atol 0.0011 -- the formula here is written from
  that description, in float32 torch on the CPU;
* closed forms: RMSNorm against float64, identity and swap RoPE matrices
  (bit-exact relations), rotation by an angle preserving pair norms.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _dt(dtype):
    return oracle.DTYPE_FP16 if dtype == torch.float16 else oracle.DTYPE_BF16


def test_f16_conversion_matches_numpy():
    rs = np.random.RandomState(0)
    v = np.concatenate([
        rs.randn(20000).astype(np.float32) * 10.0 ** rs.uniform(-9, 5, 20000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, -70000.0, 5.96e-8, 2.98e-8, 2.99e-8,
                  6.1e-5, 6.097e-5, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf], np.float32),
        (np.arange(-2048, 2048, dtype=np.float32) * 2.0 ** -25),  # subnormal ties
    ])
    got = np.array([oracle.f32_to_f16_bits(float(t)) for t in v], np.uint16)
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(got, v.astype(np.float16).view(np.uint16))
    assert oracle.f32_to_f16_bits(float("nan")) & 0x7e00 == 0x7e00
    h = np.arange(0, 65536, 7, dtype=np.uint16)
    h = h[(h & 0x7c00) != 0x7c00]
    back = np.array([oracle.f16_bits_to_f32(int(t)) for t in h], np.float32)
    np.testing.assert_array_equal(back, h.view(np.float16).astype(np.float32))


def _reference_formula(x, w, freqs, eps, rot_dim, norm_scope, split_half):
    """Torch restatement (float32 arithmetic, rounding to x.dtype where the
    reference rounds) of the preprocessing formula in validate_compatible.py."""
    b, h, l, d = x.shape
    xf = x.float()
    if norm_scope == "head":
        rr = torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)
        a = (xf * rr * w.float()).to(x.dtype)
    else:
        rows = xf.transpose(1, 2).reshape(b, l, h * d)
        rr = torch.rsqrt(rows.square().mean(-1, keepdim=True) + eps)
        a = (rows * rr * w.float()).to(x.dtype).view(b, l, h, d).transpose(1, 2)
    if rot_dim == 0:
        return a
    p = rot_dim // 2
    pre = a[..., :rot_dim].float()
    if split_half:
        first, second = pre[..., :p], pre[..., p:]
    else:
        first, second = pre[..., 0::2], pre[..., 1::2]
    m = freqs[:, :l, 0].float()  # [fb, l, p, 2, 2]
    o0 = (m[..., 0, 0].unsqueeze(1) * first + m[..., 0, 1].unsqueeze(1) * second).to(x.dtype)
    o1 = (m[..., 1, 0].unsqueeze(1) * first + m[..., 1, 1].unsqueeze(1) * second).to(x.dtype)
    rot = torch.cat((o0, o1), -1) if split_half else torch.stack((o0, o1), -1).reshape(b, h, l, rot_dim)
    return rot if rot_dim == d else torch.cat((rot, a[..., rot_dim:]), -1)


def _per_block_int8(y: torch.Tensor, blk: int, ntiles: int):
    b, h, l, d = y.shape
    yf = y.float()
    q = torch.empty(y.shape, dtype=torch.int8)
    s = torch.empty((b, h, ntiles), dtype=torch.float32)
    for t in range(ntiles):
        seg = yf[:, :, t * blk:(t + 1) * blk]
        amax = seg.abs().amax(dim=(-1, -2)).clamp_min(1e-7) if seg.shape[2] else torch.full((b, h), 1e-7)
        s[:, :, t] = amax / 127
        if seg.shape[2]:
            q[:, :, t * blk:(t + 1) * blk] = torch.round(seg * (127 / amax)[..., None, None]).clamp(-128, 127).to(torch.int8)
    return q, s


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d,scope,split", [(64, "head", True), (128, "head", True), (64, "row", False),
                                           (128, "row", False)])
def test_reference_known_answer(dtype, d, scope, split):
    """validate_compatible.py:289-383: B1 H3 L129, rot_dim = D (row) or D - 32 (head)."""
    g = torch.Generator().manual_seed(4700 + d + (100 if scope == "row" else 0))
    b, h, l = 1, 3, 129
    q = torch.randn((b, h, l, d), generator=g).to(dtype)
    k = torch.randn((b, h, l, d), generator=g).to(dtype)
    nsz = d if scope == "head" else h * d
    qw = torch.randn(nsz, generator=g).to(dtype)
    kw = torch.randn(nsz, generator=g).to(dtype)
    rot = d if scope == "row" else d - 32
    freqs = torch.randn((b, l, 1, rot // 2, 2, 2), generator=g).to(dtype)
    f32 = freqs.float()[:, :, 0].numpy()
    for x, w, blk, nt in ((q, qw, 16, (l + 63) // 64 * 4), (k, kw, 64, (l + 63) // 64)):
        ref_q, ref_s = _per_block_int8(_reference_formula(x, w, freqs, 1e-6, rot, scope, split), blk, nt)
        got_q, got_s = oracle.qk_rms_rope_int8(_bits(x), _dt(dtype), _bits(w), scope, 1e-6, f32, rot, split, blk, nt)
        assert int(np.abs(got_q.astype(np.int16) - ref_q.numpy().astype(np.int16)).max()) <= 2
        np.testing.assert_allclose(got_s, ref_s.numpy(), rtol=0.015, atol=0.0011)


def test_rmsnorm_matches_float64():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn((2, 4, 37, 128), generator=g) * 3).to(torch.bfloat16)
    w = torch.ones(128, dtype=torch.bfloat16)
    # 64-token tiles and scale = amax / 127 give back the normalized values
    q, s = oracle.qk_rms_rope_int8(_bits(x), 0, _bits(w), "head", 1e-6, None, 0, False, 64, 1)
    xd = x.double().numpy()
    a = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-6)
    deq = q.astype(np.float64) * s[..., None].astype(np.float64)
    step = s[..., None] * 0.5 + np.abs(a) * 2.0 ** -8  # half a code + bf16 rounding of a
    assert np.all(np.abs(deq - a) <= step + 1e-9)
    # row scope over 4 heads equals head scope of the [B, L, H*D] row
    qr, sr = oracle.qk_rms_rope_int8(_bits(x), 0, _bits(torch.ones(512, dtype=torch.bfloat16)), "row", 1e-6,
                                     None, 0, False, 64, 1)
    rows = xd.transpose(0, 2, 1, 3).reshape(2, 37, 512)
    ar = (rows / np.sqrt((rows ** 2).mean(-1, keepdims=True) + 1e-6)).reshape(2, 37, 4, 128).transpose(0, 2, 1, 3)
    deqr = qr.astype(np.float64) * sr[..., None]
    assert np.all(np.abs(deqr - ar) <= sr[..., None] * 0.5 + np.abs(ar) * 2.0 ** -8 + 1e-9)


@pytest.mark.parametrize("split", [False, True])
def test_identity_and_swap_rope_are_exact(split):
    g = torch.Generator().manual_seed(6)
    x = torch.randn((1, 2, 70, 64), generator=g).to(torch.float16)
    w = torch.randn(64, generator=g).to(torch.float16)
    rot, p = 48, 24
    base_q, base_s = oracle.qk_rms_rope_int8(_bits(x), 1, _bits(w), "head", 1e-6, None, 0, split, 16, 8)
    ident = np.zeros((1, 1, p, 2, 2), np.float32)
    ident[..., 0, 0] = ident[..., 1, 1] = 1.0
    q, s = oracle.qk_rms_rope_int8(_bits(x), 1, _bits(w), "head", 1e-6, ident, rot, split, 16, 8)
    np.testing.assert_array_equal(q, base_q)
    np.testing.assert_array_equal(s, base_s)
    swap = np.zeros((1, 1, p, 2, 2), np.float32)
    swap[..., 0, 1] = swap[..., 1, 0] = 1.0
    q, s = oracle.qk_rms_rope_int8(_bits(x), 1, _bits(w), "head", 1e-6, swap, rot, split, 16, 8)
    perm = np.arange(64)
    if split:
        perm[:p], perm[p:rot] = np.arange(p, rot), np.arange(p)
    else:
        perm[:rot] = np.arange(rot).reshape(-1, 2)[:, ::-1].reshape(-1)
    np.testing.assert_array_equal(q, base_q[..., perm])
    np.testing.assert_array_equal(s, base_s)


def test_rotation_preserves_pair_norms():
    g = torch.Generator().manual_seed(7)
    l, d = 40, 128
    x = torch.randn((1, 1, l, d), generator=g).to(torch.bfloat16)
    w = torch.ones(d, dtype=torch.bfloat16)
    theta = torch.rand((1, l, d // 2), generator=g).numpy() * 6.28
    f = np.zeros((1, l, d // 2, 2, 2), np.float32)
    f[..., 0, 0], f[..., 0, 1] = np.cos(theta), -np.sin(theta)
    f[..., 1, 0], f[..., 1, 1] = np.sin(theta), np.cos(theta)
    q0, s0 = oracle.qk_rms_rope_int8(_bits(x), 0, _bits(w), "head", 1e-6, None, 0, False, 64, 1)
    q1, s1 = oracle.qk_rms_rope_int8(_bits(x), 0, _bits(w), "head", 1e-6, f, d, False, 64, 1)
    n0 = np.hypot(*(q0.astype(np.float64) * s0[..., None]).reshape(1, 1, l, d // 2, 2).transpose(4, 0, 1, 2, 3))
    n1 = np.hypot(*(q1.astype(np.float64) * s1[..., None]).reshape(1, 1, l, d // 2, 2).transpose(4, 0, 1, 2, 3))
    assert np.abs(n1 - n0).max() <= 2 * max(float(s0.max()), float(s1.max())) + 0.02 * n0.max()


def test_tiles_past_the_sequence_get_the_floor_scale():
    x = torch.randn((1, 1, 20, 64)).to(torch.bfloat16)
    q, s = oracle.qk_rms_rope_int8(_bits(x), 0, _bits(torch.ones(64, dtype=torch.bfloat16)), "head", 1e-6, None,
                                   0, False, 16, 4)
    assert s[0, 0, 2] == s[0, 0, 3] == np.float32(1e-7) / np.float32(127)
    assert s[0, 0, 0] > 1e-3 and s[0, 0, 1] > 1e-3
