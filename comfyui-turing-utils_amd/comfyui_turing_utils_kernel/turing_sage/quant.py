"""Per-block INT8 quantization of Sage Q/K on gfx950, with optional K smoothing.

Mirrors the reference's ``turing_sage/quant.py`` (``per_warp_int8``,
``quantize_query_per_warp``, ``quantize_key_per_block``; :95-179), with the
block sizes of this build as parameters: BLKQ and BLKK in {16, 32, 64, 128}
(default 128, the Wan configuration).  Smoothing subtracts the per-(batch,
head) channel mean of K before quantization, the ``sub_mean`` path of the
reference's QuantInt8Kernel (``kernel/csrc/turing/sage/fused.cu:97-128``).
"""
from __future__ import annotations

import torch

from .. import _lib

SUPPORTED_BLOCKS = (16, 32, 64, 128)


def _layout_dims(x: torch.Tensor, tensor_layout: str) -> tuple[int, int, int, int, int]:
    """(heads, tokens, stride_b, stride_h, stride_l) for HND / NHD tensors."""
    if tensor_layout == "HND":
        return x.size(1), x.size(2), x.stride(0), x.stride(1), x.stride(2)
    if tensor_layout == "NHD":
        return x.size(2), x.size(1), x.stride(0), x.stride(2), x.stride(1)
    raise ValueError(f"Unknown tensor layout: {tensor_layout}")


def key_channel_mean(k: torch.Tensor, tensor_layout: str = "HND") -> torch.Tensor:
    """bf16 [B, H, D] mean of K over tokens, fixed fp32 summation order."""
    heads, tokens, sb, sh, sl = _layout_dims(k, tensor_layout)
    batch, dim = k.size(0), k.size(-1)
    chunks = (tokens + 127) // 128
    scratch = torch.empty((batch, heads, chunks, dim), dtype=torch.float32, device=k.device)
    mean = torch.empty((batch, heads, dim), dtype=torch.bfloat16, device=k.device)
    with torch.cuda.device(k.device):
        _lib.call("tu_sage_kmean", k.data_ptr(), batch, heads, tokens, dim, sb, sh, sl,
                  scratch.data_ptr(), mean.data_ptr(), _lib.stream_of(k.device))
    return mean


def quantize_per_block(
    x: torch.Tensor,
    block: int,
    tensor_layout: str = "HND",
    mean: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """int8 tensor of x's shape and fp32 scales [B, H, ceil(L / block)]."""
    if block not in SUPPORTED_BLOCKS:
        raise ValueError(f"Sage quantization block must be one of {SUPPORTED_BLOCKS}, got {block}")
    heads, tokens, sb, sh, sl = _layout_dims(x, tensor_layout)
    batch, dim = x.size(0), x.size(-1)
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    _, _, qb, qh, ql = _layout_dims(q, tensor_layout)
    scale = torch.empty((batch, heads, (tokens + block - 1) // block), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("tu_sage_quant", x.data_ptr(), _lib.ptr(mean), batch, heads, tokens, dim, sb, sh, sl,
                  block, q.data_ptr(), qb, qh, ql, scale.data_ptr(), _lib.stream_of(x.device))
    return q, scale


def per_block_int8(
    q: torch.Tensor,
    k: torch.Tensor,
    BLKQ: int = 128,
    BLKK: int = 128,
    tensor_layout: str = "HND",
    smooth_k: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Quantize Q per BLKQ tokens and (smoothed) K per BLKK tokens.

    Returns (q_int8, q_scale, k_int8, k_scale, k_mean); k_mean is None when
    smoothing is off.
    """
    mean = key_channel_mean(k, tensor_layout) if smooth_k else None
    q_int8, q_scale = quantize_per_block(q, BLKQ, tensor_layout)
    k_int8, k_scale = quantize_per_block(k, BLKK, tensor_layout, mean)
    return q_int8, q_scale, k_int8, k_scale, mean


def value_transpose(v: torch.Tensor, tensor_layout: str = "HND") -> tuple[torch.Tensor, int]:
    """V^T [B, H, D, Lpad] (keys padded with zeros to a multiple of 64), the
    PV operand layout of the attention kernel.  Returns (vt, lpad)."""
    heads, tokens, sb, sh, sl = _layout_dims(v, tensor_layout)
    batch, dim = v.size(0), v.size(-1)
    lpad = (tokens + 63) // 64 * 64
    vt = torch.empty((batch, heads, dim, lpad), dtype=torch.bfloat16, device=v.device)
    with torch.cuda.device(v.device):
        _lib.call("tu_sage_v_prep", v.data_ptr(), batch, heads, tokens, dim, sb, sh, sl, vt.data_ptr(), lpad,
                  _lib.stream_of(v.device))
    return vt, lpad


def rms_rope_per_warp_int8(
    q: torch.Tensor,
    k: torch.Tensor,
    q_norm: torch.Tensor,
    k_norm: torch.Tensor,
    freqs: torch.Tensor | None,
    *,
    epsilon: float,
    rot_dim: int,
    tensor_layout: str,
    norm_scope: str,
    split_half: bool,
    rotate_qk: bool = False,
    stabilize_k: bool = False,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused Q/K RMSNorm + RoPE + INT8 (Q per 16 tokens, K per 64 tokens), the
    reference's ``rms_rope_per_warp_int8`` (turing_sage/quant.py:6-87).

    Q scales are [B, Hq, ceil(Lq / 64) * 4], K scales [B, Hk, ceil(Lk / 64)].
    ``rotate_qk`` applies the W8A8 path's shared Hadamard rotation after RoPE;
    with ``stabilize_k`` as well, K is first centred on its anchor row (the
    reference's quant.py:57-64: stabilisation only with rotation).
    """
    if tensor_layout not in ("HND", "NHD"):
        raise ValueError(f"Unknown tensor layout: {tensor_layout}")
    if norm_scope not in ("head", "row"):
        raise ValueError("norm_scope must be head or row")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype:
        raise TypeError("fused Q/K preprocessing requires matching FP16 or BF16 inputs")
    if q.ndim != 4 or k.ndim != 4 or q.size(0) != k.size(0) or q.size(-1) != k.size(-1):
        raise ValueError("fused Q/K preprocessing requires compatible four-dimensional tensors")
    head_dim = q.size(-1)
    if head_dim not in (64, 128):
        raise ValueError("fused RMSNorm+RoPE Q/K quantization requires head_dim 64 or 128")
    if q.stride(-1) != 1 or k.stride(-1) != 1:
        raise ValueError("the last Q/K dimension must be contiguous")
    hq, lq, qsb, qsh, qsl = _layout_dims(q, tensor_layout)
    hk, lk, ksb, ksh, ksl = _layout_dims(k, tensor_layout)
    batch = q.size(0)
    if rot_dim < 0 or rot_dim > head_dim or rot_dim % 2:
        raise ValueError("rot_dim must be even and within head_dim")
    expect_q = head_dim if norm_scope == "head" else hq * head_dim
    expect_k = head_dim if norm_scope == "head" else hk * head_dim
    if q_norm.numel() != expect_q or k_norm.numel() != expect_k:
        raise ValueError("Q/K norm weight shapes are incompatible")
    q_norm = q_norm.to(device=q.device, dtype=q.dtype).contiguous()
    k_norm = k_norm.to(device=q.device, dtype=q.dtype).contiguous()
    fb = fl = 1
    fstrides = (0, 0, 0, 0, 0)
    if rot_dim > 0:
        if freqs is None or freqs.ndim != 6:
            raise ValueError("RoPE frequencies must be [B|1, L|1, 1, rot_dim / 2, 2, 2]")
        freqs = freqs.to(device=q.device, dtype=q.dtype)
        if freqs.size(2) != 1 or freqs.size(3) != rot_dim // 2 or freqs.size(4) != 2 or freqs.size(5) != 2:
            raise ValueError("RoPE frequency shape is incompatible")
        fb, fl = freqs.size(0), freqs.size(1)
        if not ((fb == 1 or fb == batch) and (fl == 1 or (fl == lq and lq == lk))):
            raise ValueError("RoPE batch/sequence broadcasting is incompatible")
        fstrides = (freqs.stride(0), freqs.stride(1), freqs.stride(3), freqs.stride(4), freqs.stride(5))
    if any(t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:-1]) for t in (q, k)):
        q, k = q.contiguous(), k.contiguous()
        hq, lq, qsb, qsh, qsl = _layout_dims(q, tensor_layout)
        hk, lk, ksb, ksh, ksl = _layout_dims(k, tensor_layout)
    q_int8 = torch.empty(q.shape, dtype=torch.int8, device=q.device)
    k_int8 = torch.empty(k.shape, dtype=torch.int8, device=k.device)
    _, _, qob, qoh, qol = _layout_dims(q_int8, tensor_layout)
    _, _, kob, koh, kol = _layout_dims(k_int8, tensor_layout)
    q_scale = torch.empty((batch, hq, (lq + 63) // 64 * 4), dtype=torch.float32, device=q.device)
    k_scale = torch.empty((batch, hk, (lk + 63) // 64), dtype=torch.float32, device=k.device)
    anchors = anchor_values = None
    if rotate_qk and stabilize_k:
        anchors = torch.empty((batch, hk), dtype=torch.int32, device=k.device)
        anchor_values = torch.empty((batch, hk, head_dim), dtype=torch.float32, device=k.device)
    q_rrms = k_rrms = None
    if norm_scope == "row":
        q_rrms = torch.empty((batch, lq), dtype=torch.float32, device=q.device)
        k_rrms = torch.empty((batch, lk), dtype=torch.float32, device=k.device)
    with torch.cuda.device(q.device):
        _lib.call(
            "tu_qk_rms_rope_int8",
            q.data_ptr(), k.data_ptr(), 1 if q.dtype == torch.float16 else 0, batch, hq, hk, lq, lk, head_dim,
            qsb, qsh, qsl, ksb, ksh, ksl, q_norm.data_ptr(), k_norm.data_ptr(), 1 if norm_scope == "row" else 0,
            float(epsilon), _lib.ptr(freqs) if rot_dim > 0 else None, int(rot_dim), int(bool(split_half)), fb, fl,
            *fstrides, _lib.ptr(q_rrms), _lib.ptr(k_rrms), q_int8.data_ptr(), qob, qoh, qol,
            k_int8.data_ptr(), kob, koh, kol, q_scale.data_ptr(), k_scale.data_ptr(), int(bool(rotate_qk)),
            _lib.ptr(anchors), _lib.ptr(anchor_values), _lib.stream_of(q.device),
        )
    return q_int8, q_scale, k_int8, k_scale


def per_warp_int8_hadamard(
    q: torch.Tensor,
    k: torch.Tensor,
    BLKQ: int = 64,
    WARPQ: int = 16,
    BLKK: int = 64,
    tensor_layout: str = "HND",
    stabilize_k: bool = True,
    rotate: bool = True,
):
    """Shared randomized Hadamard rotation fused into Q/K INT8 quantization,
    the reference's ``per_warp_int8_hadamard`` (turing_sage/quant.py:182-242):
    Q per 16-token tile with ceil(Lq / 64) * 4 scales, K per 64-token tile,
    K first centred on its stabilisation anchor when ``stabilize_k``.
    Returns (q_int8, q_scale, k_int8, k_scale); codes keep the input layout.
    ``rotate=False`` gives the plain per-warp codes (the reference's
    ``rotate_qk=False`` route, quant.py:95-118)."""
    if (BLKQ, WARPQ, BLKK) != (64, 16, 64):
        raise ValueError("the W8A8 quantizer uses BLKQ=64, WARPQ=16, BLKK=64")
    qh, ql, qsb, qsh, qsl = _layout_dims(q, tensor_layout)
    kh, kl, ksb, ksh, ksl = _layout_dims(k, tensor_layout)
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype:
        raise TypeError("W8A8 Q/K must be matching float16 or bfloat16 tensors")
    if q.ndim != 4 or k.ndim != 4 or q.size(0) != k.size(0) or q.size(-1) != k.size(-1):
        raise ValueError("W8A8 Q/K must be compatible four-dimensional tensors")
    dim = q.size(-1)
    if dim not in (64, 128):
        raise ValueError("the W8A8 Q/K quantizer requires head_dim 64 or 128")
    if q.stride(-1) != 1 or k.stride(-1) != 1:
        raise ValueError("the last Q/K dimension must be contiguous")
    if not q.is_cuda or k.device != q.device:
        raise ValueError("W8A8 Q/K must be CUDA tensors on one device")
    batch = q.size(0)
    q_int8 = torch.empty(q.shape, dtype=torch.int8, device=q.device)
    k_int8 = torch.empty(k.shape, dtype=torch.int8, device=k.device)
    _, _, q8b, q8h, q8l = _layout_dims(q_int8, tensor_layout)
    _, _, k8b, k8h, k8l = _layout_dims(k_int8, tensor_layout)
    q_scale = torch.empty((batch, qh, (ql + BLKQ - 1) // BLKQ * (BLKQ // WARPQ)), dtype=torch.float32,
                          device=q.device)
    k_scale = torch.empty((batch, kh, (kl + BLKK - 1) // BLKK), dtype=torch.float32, device=q.device)
    anchors = torch.empty((batch, kh), dtype=torch.int32, device=q.device) if stabilize_k else None
    with torch.cuda.device(q.device):
        _lib.call("tu_w8a8_quant_qk", q.data_ptr(), k.data_ptr(), 1 if q.dtype == torch.float16 else 0,
                  batch, qh, kh, ql, kl, dim, qsb, qsh, qsl, ksb, ksh, ksl,
                  q_int8.data_ptr(), q8b, q8h, q8l, k_int8.data_ptr(), k8b, k8h, k8l,
                  q_scale.data_ptr(), k_scale.data_ptr(), _lib.ptr(anchors), int(bool(rotate)),
                  _lib.stream_of(q.device))
    return q_int8, q_scale, k_int8, k_scale


def quantize_v_int8(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Channel-wise signed INT8 of HND V, the reference's quantize_v_int8_sm75
    (turing_sage/core.py:772-784): (codes [B, H, D, ceil(L/64)*64] with keys
    in natural order and zero padding, fp32 scales [B, H, D])."""
    if value.ndim != 4 or value.stride(-1) != 1:
        raise ValueError("W8A8 V must be four-dimensional with contiguous channels")
    if value.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("W8A8 V must be float16 or bfloat16")
    batch, heads, length, dim = value.shape
    if dim not in (64, 128):
        raise ValueError("the W8A8 V quantizer requires head_dim 64 or 128")
    if value.data_ptr() % 16 or any(s % 8 for s in value.stride()[:-1]):
        value = value.contiguous()
    lpad = (length + 63) // 64 * 64
    codes = torch.empty((batch, heads, dim, lpad), dtype=torch.int8, device=value.device)
    scale = torch.empty((batch, heads, dim), dtype=torch.float32, device=value.device)
    lib = _lib.load()
    ws_bytes = int(lib.tu_w8a8_quant_v_workspace(batch, heads, length, dim))
    workspace = torch.empty((ws_bytes,), dtype=torch.uint8, device=value.device)
    with torch.cuda.device(value.device):
        _lib.call("tu_w8a8_quant_v", value.data_ptr(), 1 if value.dtype == torch.float16 else 0, batch, heads,
                  length, dim, value.stride(0), value.stride(1), value.stride(2), codes.data_ptr(), lpad,
                  scale.data_ptr(), workspace.data_ptr(), ws_bytes, _lib.stream_of(value.device))
    return codes, scale
