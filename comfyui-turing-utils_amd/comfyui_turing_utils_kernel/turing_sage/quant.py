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
