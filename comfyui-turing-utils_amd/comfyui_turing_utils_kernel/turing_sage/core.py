"""Sage INT8 attention facade on gfx950.

Follows the reference's ``turing_sage/core.py``: validation and head-dim
padding (``prequantize_sageattn``, :409-474), the split prequantize / execute
API (``PrequantizedSageAttention``, ``sageattn_from_prequantized``,
``sageattn_prequantized``, :477-653) and the one-call ``sageattn`` (:543-570).

MI355X build choices (each a parameter with the Wan default):
  * Q and K are quantized per 128-token block (``BLKQ``, ``BLKK``); the
    reference used Q per 16 tokens and K per 64 tokens for its 64-row Turing
    CTA.
  * K is mean-smoothed by default (``smooth_k=True``); the reference's
    production Turing path raises on smoothing (core.py:421-422).
  * PV runs in bf16 on MFMA; the reference converted V to fp16 for Turing.
  * The kernel is used for every sequence length (no SDPA short-sequence
    detour): tails are masked inside the kernel.
  * head_dim <= 64 is zero-padded to 64 and 64 < head_dim <= 128 to 128, as
    the reference pads (core.py:436-448); the kernel is built for both widths,
    and zero channels leave Q.K and P.V exact.
"""
from __future__ import annotations

import dataclasses
import math
from typing import Optional

import torch

from .. import _lib
from .quant import (
    SUPPORTED_BLOCKS,
    _layout_dims,
    per_block_int8,
    per_warp_int8_hadamard,
    quantize_v_int8,
    rms_rope_per_warp_int8,
    value_transpose,
)

KERNEL_HEAD_DIM = 128  # widest head; the W8A8 kernel's only width


def _sage_head_dim(head_dim: int) -> int:
    """Kernel width for a head_dim <= 128: 64 or 128 (reference core.py:436-448)."""
    return 64 if head_dim <= 64 else 128


@dataclasses.dataclass(frozen=True)
class PrequantizedSageAttention:
    """Quantized Q/K plus V^T, ready for ``sageattn_from_prequantized``.

    ``value_t`` is [B, Hkv, 128, Lpad] bf16 (keys padded with zeros to a
    multiple of 64), the layout ``tu_sage_attn_fwd`` reads; the caller may
    release the original Q/K/V once this object exists.
    """

    query_int8: torch.Tensor
    query_scale: torch.Tensor
    key_int8: torch.Tensor
    key_scale: torch.Tensor
    value_t: torch.Tensor
    tensor_layout: str
    original_head_dim: int
    is_causal: bool
    sm_scale: float
    blkq: int
    blkk: int
    output_dtype: torch.dtype


@dataclasses.dataclass(frozen=True)
class PrequantizedQK:
    """Fused-preprocessing result (``prequantize_rms_rope_qk``): INT8 Q with
    16-token scales [B, Hq, ceil(Lq / 64) * 4] and INT8 K with 64-token scales
    [B, Hk, ceil(Lk / 64)], the reference's dataclass (core.py:39-47)."""

    query_int8: torch.Tensor
    query_scale: torch.Tensor
    key_int8: torch.Tensor
    key_scale: torch.Tensor
    tensor_layout: str
    input_dtype: torch.dtype
    original_head_dim: int
    route_original_basis: bool = False


def _validate(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str) -> None:
    if tensor_layout not in ("HND", "NHD"):
        raise ValueError(f"Unsupported tensor_layout: {tensor_layout}")
    if not q.is_cuda:
        raise ValueError("Input tensors must be on CUDA")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("Sage Q/K/V must be float16 or bfloat16")
    if q.device != k.device or q.device != v.device:
        raise ValueError("Q/K/V must be on the same device")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError("Q/K/V must have matching dtypes")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("Sage Q/K/V must be four-dimensional")
    if k.shape != v.shape:
        raise ValueError("K and V must have the same shape")
    qh, ql, *_ = _layout_dims(q, tensor_layout)
    kh, kl, *_ = _layout_dims(k, tensor_layout)
    if q.size(0) != k.size(0) or q.size(-1) != k.size(-1):
        raise ValueError("Q and K must agree in batch and head_dim")
    if kh <= 0 or qh % kh != 0:
        raise ValueError("Q heads must be divisible by KV heads")
    if ql <= 0 or kl <= 0:
        raise ValueError("Sage attention requires non-empty Q/K sequences")
    if q.size(-1) > KERNEL_HEAD_DIM:
        raise ValueError(f"Unsupported head_dim: {q.size(-1)}")


def _prepare(x: torch.Tensor, width: int) -> torch.Tensor:
    """bf16, channels padded to the kernel width, last dim contiguous."""
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    pad = width - x.size(-1)
    if pad:
        x = torch.nn.functional.pad(x, (0, pad))
    if x.stride(-1) != 1 or x.data_ptr() % 16 != 0 or any(s % 8 for s in x.stride()[:-1]):
        x = x.contiguous()
    return x


def prequantize_sageattn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    smooth_k: bool = True,
    BLKQ: int = 128,
    BLKK: int = 128,
) -> PrequantizedSageAttention:
    """Quantize Q/K (K smoothed) and keep V, before the output is allocated."""
    _validate(q, k, v, tensor_layout)
    if BLKQ not in SUPPORTED_BLOCKS or BLKK not in SUPPORTED_BLOCKS or BLKK % 64:
        raise ValueError(f"BLKQ must be in {SUPPORTED_BLOCKS} and BLKK in (64, 128)")
    head_dim = q.size(-1)
    scale = float(sm_scale) if sm_scale is not None else head_dim ** -0.5
    if not (scale > 0.0 and math.isfinite(scale)):
        raise ValueError("sm_scale must be a positive finite number")
    output_dtype = q.dtype
    width = _sage_head_dim(head_dim)
    qp, kp, vp = _prepare(q, width), _prepare(k, width), _prepare(v, width)
    with torch.cuda.device(q.device):
        q_int8, q_scale, k_int8, k_scale, _ = per_block_int8(
            qp, kp, BLKQ=BLKQ, BLKK=BLKK, tensor_layout=tensor_layout, smooth_k=smooth_k
        )
        value_t, _ = value_transpose(vp, tensor_layout)
    return PrequantizedSageAttention(
        query_int8=q_int8, query_scale=q_scale, key_int8=k_int8, key_scale=k_scale, value_t=value_t,
        tensor_layout=tensor_layout, original_head_dim=head_dim, is_causal=bool(is_causal),
        sm_scale=scale, blkq=BLKQ, blkk=BLKK, output_dtype=output_dtype,
    )


def _check_qk(q_int8, q_scale, k_int8, k_scale, tensor_layout, blkq, blkk):
    if tensor_layout not in ("HND", "NHD"):
        raise ValueError(f"Unsupported tensor_layout: {tensor_layout}")
    if q_int8.dtype != torch.int8 or k_int8.dtype != torch.int8:
        raise TypeError("prequantized Sage Q/K must be int8")
    if q_scale.dtype != torch.float32 or k_scale.dtype != torch.float32:
        raise TypeError("prequantized Sage scales must be float32")
    if q_int8.ndim != 4 or k_int8.ndim != 4:
        raise ValueError("prequantized Sage Q/K must be four-dimensional")
    if len({q_int8.device, k_int8.device, q_scale.device, k_scale.device}) != 1:
        raise ValueError("prequantized Sage tensors must share one device")
    if q_int8.size(-1) not in (64, 128) or k_int8.size(-1) != q_int8.size(-1):
        raise ValueError("prequantized Sage requires Q/K head_dim 64 or 128")
    if q_int8.stride(-1) != 1 or k_int8.stride(-1) != 1:
        raise ValueError("the last Q/K dimension must be contiguous")
    hq, lq, *_ = _layout_dims(q_int8, tensor_layout)
    hkv, lk, *_ = _layout_dims(k_int8, tensor_layout)
    batch = q_int8.size(0)
    if k_int8.size(0) != batch:
        raise ValueError("prequantized Sage Q/K batch sizes differ")
    if hkv <= 0 or hq % hkv != 0:
        raise ValueError("prequantized Sage Q heads must be divisible by KV heads")
    if blkk % 64 or blkq <= 0:
        raise ValueError("prequantized Sage needs blkq > 0 and blkk % 64 == 0")
    if q_scale.shape != (batch, hq, (lq + blkq - 1) // blkq):
        raise ValueError("prequantized Sage Q scale shape is incompatible")
    if k_scale.shape != (batch, hkv, (lk + blkk - 1) // blkk):
        raise ValueError("prequantized Sage K scale shape is incompatible")
    return batch, hq, hkv, lq, lk


def attention_from_vt(
    q_int8: torch.Tensor,
    q_scale: torch.Tensor,
    k_int8: torch.Tensor,
    k_scale: torch.Tensor,
    value_t: torch.Tensor,
    *,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    blkq: int = 128,
    blkk: int = 128,
    output: Optional[torch.Tensor] = None,
    kv_splits: Optional[int] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention kernel only: quantized Q/K and V^T from ``value_transpose``.

    ``kv_splits`` (this package only): key ranges computed by separate
    workgroups and merged, for grids that fill the GPU badly; None lets
    ``tu_sage_attn_kv_splits`` choose from the device's compute units, 1
    never splits.  Non-causal only.  A split call needs an fp32 workspace of
    ``split_workspace_bytes(...)`` bytes (ranges x B x H x Lq x (D + 2) x 4:
    about 100 MB at B1 H12 L8190 D128 with two ranges); it comes from
    ``workspace`` (a contiguous float32 tensor on the Q/K device, at least
    that large, reusable across calls on one stream) or else from torch's
    caching allocator.  How many ranges None picks depends on the device's
    compute-unit count, so results are bit-identical across devices only
    with an explicit ``kv_splits``."""
    batch, hq, hkv, lq, lk = _check_qk(q_int8, q_scale, k_int8, k_scale, tensor_layout, blkq, blkk)
    width = q_int8.size(-1)
    lpad = (lk + 63) // 64 * 64
    if value_t.dtype != torch.bfloat16 or value_t.shape != (batch, hkv, width, lpad):
        raise ValueError(f"V^T must be bf16 [{batch}, {hkv}, {width}, {lpad}]")
    if value_t.device != q_int8.device or not value_t.is_contiguous():
        raise ValueError("V^T must be contiguous on the Q/K device")
    scale = float(sm_scale) if sm_scale is not None else width ** -0.5
    if output is None:
        output = torch.empty(q_int8.shape, dtype=torch.bfloat16, device=q_int8.device)
    elif (output.shape != q_int8.shape or output.dtype != torch.bfloat16 or output.device != q_int8.device
          or output.stride(-1) != 1):
        raise ValueError("prequantized Sage output is incompatible")
    _, _, qsb, qsh, qsl = _layout_dims(q_int8, tensor_layout)
    _, _, ksb, ksh, ksl = _layout_dims(k_int8, tensor_layout)
    _, _, osb, osh, osl = _layout_dims(output, tensor_layout)
    q_scale = q_scale.contiguous()
    k_scale = k_scale.contiguous()
    if kv_splits is None:
        splits = int(_lib.load().tu_sage_attn_kv_splits(batch, hq, lq, lk, int(bool(is_causal)),
                                                        _compute_units(q_int8.device)))
    else:
        splits = int(kv_splits)
        if splits < 1 or (is_causal and splits > 1):
            raise ValueError("kv_splits must be >= 1, and 1 for causal attention")
    if splits > 1:
        # key ranges merged by a second kernel: fp32 partial O plus
        # (exponent base, row sum) per row and range
        need = split_workspace_bytes(batch, hq, lq, lk, width, splits) // 4
        if workspace is not None and (workspace.dtype != torch.float32 or workspace.device != q_int8.device
                                      or not workspace.is_contiguous() or workspace.numel() < need):
            raise ValueError(f"Sage split workspace must be a contiguous float32 tensor on the Q/K device "
                             f"with at least {need} elements")
    with torch.cuda.device(q_int8.device):
        if splits > 1:
            partial = workspace if workspace is not None else torch.empty(need, dtype=torch.float32,
                                                                          device=q_int8.device)
            _lib.call(
                "tu_sage_attn_fwd_split",
                q_int8.data_ptr(), q_scale.data_ptr(), blkq, k_int8.data_ptr(), k_scale.data_ptr(), blkk,
                value_t.data_ptr(), lpad, output.data_ptr(), batch, hq, hkv, lq, lk, width,
                qsb, qsh, qsl, ksb, ksh, ksl, osb, osh, osl,
                scale, splits, partial.data_ptr(), partial.numel() * 4, _lib.stream_of(q_int8.device),
            )
        else:
            _lib.call(
                "tu_sage_attn_fwd",
                q_int8.data_ptr(), q_scale.data_ptr(), blkq, k_int8.data_ptr(), k_scale.data_ptr(), blkk,
                value_t.data_ptr(), lpad, output.data_ptr(), batch, hq, hkv, lq, lk, width,
                qsb, qsh, qsl, ksb, ksh, ksl, osb, osh, osl,
                scale, int(bool(is_causal)), _lib.stream_of(q_int8.device),
            )
    return output


def split_workspace_bytes(batch: int, hq: int, lq: int, lk: int, head_dim: int, kv_splits: int) -> int:
    """Bytes of fp32 workspace a key-split call needs: per range and query
    row, the unnormalized O (head_dim floats) plus exponent base and row sum."""
    tiles = (lk + 63) // 64
    per = (tiles + kv_splits - 1) // kv_splits
    used = (tiles + per - 1) // per
    return used * batch * hq * lq * (head_dim + 2) * 4


_CU_COUNT: dict = {}


def _compute_units(device: torch.device) -> int:
    """Compute units of ``device`` (cached): the round size of the attention grid."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _CU_COUNT:
        _CU_COUNT[index] = int(torch.cuda.get_device_properties(index).multi_processor_count)
    return _CU_COUNT[index]


def sageattn_prequantized(
    q_int8: torch.Tensor,
    q_scale: torch.Tensor,
    k_int8: torch.Tensor,
    k_scale: torch.Tensor,
    v: torch.Tensor,
    *,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    blkq: int = 128,
    blkk: int = 128,
    output: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention on already-quantized Q/K and bf16 V (head_dim 64 or 128), the
    counterpart of the reference's ``sageattn_prequantized`` (core.py:573-653)."""
    batch, hq, hkv, lq, lk = _check_qk(q_int8, q_scale, k_int8, k_scale, tensor_layout, blkq, blkk)
    if v.dtype != torch.bfloat16:
        raise TypeError("prequantized Sage V must be bfloat16")
    if v.ndim != 4 or v.device != q_int8.device or v.stride(-1) != 1:
        raise ValueError("prequantized Sage V must be 4D, contiguous in channels, on the Q/K device")
    vh, vl, *_ = _layout_dims(v, tensor_layout)
    if v.size(0) != batch or vh != hkv or vl != lk or v.size(-1) != q_int8.size(-1):
        raise ValueError("prequantized Sage Q/K/V shapes are incompatible")
    value_t, _ = value_transpose(v, tensor_layout)
    return attention_from_vt(q_int8, q_scale, k_int8, k_scale, value_t, tensor_layout=tensor_layout,
                             is_causal=is_causal, sm_scale=sm_scale, blkq=blkq, blkk=blkk, output=output)


def sageattn_from_prequantized(quantized: PrequantizedSageAttention) -> torch.Tensor:
    out = attention_from_vt(
        quantized.query_int8, quantized.query_scale, quantized.key_int8, quantized.key_scale, quantized.value_t,
        tensor_layout=quantized.tensor_layout, is_causal=quantized.is_causal, sm_scale=quantized.sm_scale,
        blkq=quantized.blkq, blkk=quantized.blkk,
    )
    out = out[..., : quantized.original_head_dim]
    if quantized.output_dtype != torch.bfloat16:
        out = out.to(quantized.output_dtype)
    return out


def sageattn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    smooth_k: bool = True,
    BLKQ: int = 128,
    BLKK: int = 128,
) -> torch.Tensor:
    """One-call Sage attention: K mean-smoothing, per-block INT8 Q/K, INT8 QK^T,
    online softmax, bf16 PV.  Output has q's shape and dtype."""
    quantized = prequantize_sageattn(
        q, k, v, tensor_layout=tensor_layout, is_causal=is_causal, sm_scale=sm_scale,
        smooth_k=smooth_k, BLKQ=BLKQ, BLKK=BLKK,
    )
    return sageattn_from_prequantized(quantized)


def prequantize_rms_rope_qk(
    q: torch.Tensor,
    k: torch.Tensor,
    q_norm: torch.Tensor,
    k_norm: torch.Tensor,
    freqs: Optional[torch.Tensor],
    *,
    epsilon: float,
    rot_dim: int,
    tensor_layout: str = "HND",
    norm_scope: str = "head",
    split_half: bool = False,
    rotate_qk: bool = False,
    stabilize_k: bool = False,
) -> PrequantizedQK:
    """Normalized, rotated and quantized Q/K without materializing bf16
    intermediates (reference core.py:222-289), through
    ``torch.ops.turing_utils.qk_rms_rope_int8``."""
    if not q.is_cuda or not k.is_cuda:
        raise ValueError("Q/K inputs must be on CUDA")
    if q.device != k.device:
        raise ValueError("Q/K inputs must share one CUDA device")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype:
        raise TypeError("fused Q/K preprocessing requires matching FP16 or BF16 inputs")
    if q.ndim != 4 or k.ndim != 4 or q.shape[0] != k.shape[0] or q.shape[-1] != k.shape[-1]:
        raise ValueError("fused Q/K preprocessing requires compatible four-dimensional tensors")
    if q.stride(-1) != 1 or k.stride(-1) != 1:
        raise ValueError("the last Q/K dimension must be contiguous")
    head_dim = int(q.shape[-1])
    if head_dim not in (64, 128):
        raise ValueError("fused Q/K preprocessing requires head_dim 64 or 128")
    q_norm = q_norm.to(device=q.device, dtype=q.dtype).contiguous()
    k_norm = k_norm.to(device=q.device, dtype=q.dtype).contiguous()
    freqs = (torch.empty(0, device=q.device, dtype=q.dtype) if freqs is None
             else freqs.to(device=q.device, dtype=q.dtype))
    from .custom_ops import qk_rms_rope_int8

    q_int8, q_scale, k_int8, k_scale = qk_rms_rope_int8(
        q, k, q_norm, k_norm, freqs, float(epsilon), int(rot_dim), tensor_layout, norm_scope,
        bool(split_half), bool(rotate_qk), bool(stabilize_k),
    )
    return PrequantizedQK(
        query_int8=q_int8, query_scale=q_scale, key_int8=k_int8, key_scale=k_scale,
        tensor_layout=tensor_layout, input_dtype=q.dtype, original_head_dim=head_dim,
        route_original_basis=bool(rotate_qk),
    )


def prequantize_sageattn_from_qk(
    qk: PrequantizedQK,
    value: torch.Tensor,
    *,
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
) -> PrequantizedSageAttention:
    """Attach V to a fused Q/K preprocessing result without rereading Q/K
    (reference core.py:477-513).  The fused producer's head_dim (64 or 128)
    is a kernel width, so nothing is padded.  Rotated (and
    anchored) codes are accepted as the reference accepts them: the rotation
    leaves Q.K unchanged and the anchor shifts each query row's scores by a
    constant, which the softmax cancels."""
    if qk.tensor_layout not in ("HND", "NHD"):
        raise ValueError(f"Unsupported tensor_layout: {qk.tensor_layout}")
    if value.dtype != qk.input_dtype:
        raise TypeError("preprocessed Q/K and V must have matching logical dtypes")
    if value.device != qk.query_int8.device:
        raise ValueError("preprocessed Q/K and V must share one CUDA device")
    if value.ndim != 4 or value.stride(-1) != 1:
        raise ValueError("preprocessed Sage V must be four-dimensional with contiguous channels")
    head_axis = 1 if qk.tensor_layout == "HND" else 2
    seq_axis = 2 if qk.tensor_layout == "HND" else 1
    if (value.size(0) != qk.key_int8.size(0) or value.size(head_axis) != qk.key_int8.size(head_axis)
            or value.size(seq_axis) != qk.key_int8.size(seq_axis) or value.size(-1) != qk.key_int8.size(-1)):
        raise ValueError("preprocessed Q/K and V shapes are incompatible")
    scale = float(sm_scale) if sm_scale is not None else qk.original_head_dim ** -0.5
    q_int8, k_int8 = qk.query_int8, qk.key_int8
    width = _sage_head_dim(q_int8.size(-1))
    pad = width - q_int8.size(-1)
    if pad:
        q_int8 = torch.nn.functional.pad(q_int8, (0, pad))
        k_int8 = torch.nn.functional.pad(k_int8, (0, pad))
    lq = q_int8.size(seq_axis)
    # the fused producer pads Q scales to 4 per 64 tokens; the kernel indexes
    # them as ceil(Lq / 16) per head
    q_scale = qk.query_scale[..., : (lq + 15) // 16].contiguous()
    with torch.cuda.device(value.device):
        value_t, _ = value_transpose(_prepare(value, width), qk.tensor_layout)
    return PrequantizedSageAttention(
        query_int8=q_int8, query_scale=q_scale, key_int8=k_int8, key_scale=qk.key_scale, value_t=value_t,
        tensor_layout=qk.tensor_layout, original_head_dim=qk.original_head_dim, is_causal=bool(is_causal),
        sm_scale=scale, blkq=16, blkk=64, output_dtype=value.dtype,
    )


# ---------------------------------------------------------------------------
# Dense W8A8 attention (the reference's loader-default ``w8a8`` backend)
# ---------------------------------------------------------------------------

@dataclasses.dataclass(frozen=True)
class PrequantizedW8A8Attention:
    """INT8 Q/K (Hadamard-rotated, 16-/64-token scales) and channel-wise INT8
    V^T, ready for ``w8a8attn_from_prequantized``: the dense (force_dense,
    use_w8a8) subset of the reference's PrequantizedSolAttention
    (core.py:50-72).  All tensors are HND with the kernel's 128 channels;
    ``value_int8`` is [B, Hkv, 128, Lpad] with keys in natural order."""

    query_int8: torch.Tensor
    query_scale: torch.Tensor
    key_int8: torch.Tensor
    key_scale: torch.Tensor
    value_int8: torch.Tensor
    value_scale: torch.Tensor
    output_dtype: torch.dtype
    sm_scale: float
    original_head_dim: int
    key_tile_tokens: int
    is_causal: bool
    route_original_basis: bool


def _validate_fixed_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tensor_layout: str) -> None:
    """The reference's fixed-length Q/K/V contract (core.py:292-309)."""
    if tensor_layout not in ("HND", "NHD"):
        raise ValueError(f"Unsupported tensor_layout: {tensor_layout}")
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("fixed-length Q/K/V must be four-dimensional")
    head_dim = q.size(-1)
    if k.size(-1) != head_dim or v.size(-1) != head_dim:
        raise ValueError("Q/K/V head dimensions must match")
    head_axis = 1 if tensor_layout == "HND" else 2
    seq_axis = 2 if tensor_layout == "HND" else 1
    if q.size(0) != k.size(0) or q.size(0) != v.size(0):
        raise ValueError("Q/K/V batch sizes must match")
    if k.size(head_axis) != v.size(head_axis) or k.size(seq_axis) != v.size(seq_axis):
        raise ValueError("K/V head counts and sequence lengths must match")
    if k.size(head_axis) == 0 or q.size(head_axis) % k.size(head_axis) != 0:
        raise ValueError("the Q head count must be divisible by the KV head count")
    if q.size(seq_axis) == 0 or k.size(seq_axis) == 0:
        raise ValueError("empty Q/K sequences are not supported")


def _key_tile_tokens(key_tile_tokens: int, key_length: int) -> int:
    """The reference's key-tile validation (core.py:740-745).  The dense path
    runs 64-key tiles whatever the value; the resolved value is kept."""
    key_tile_tokens = int(key_tile_tokens)
    if key_tile_tokens not in (0, 64, 128):
        raise ValueError("key_tile_tokens must be 0 (auto), 64, or 128")
    if key_tile_tokens == 0:
        key_tile_tokens = 128 if key_length > 1024 else 64
    return key_tile_tokens


def _pad_channels(x: torch.Tensor, width: int) -> torch.Tensor:
    pad = width - x.size(-1)
    return torch.nn.functional.pad(x, (0, pad)) if pad else x


def prequantize_w8a8attn_from_qk(
    qk: PrequantizedQK,
    value: torch.Tensor,
    *,
    sm_scale: Optional[float] = None,
    key_tile_tokens: int = 0,
    is_causal: bool = False,
) -> PrequantizedW8A8Attention:
    """Attach channel-wise INT8 V to already quantized Q/K, the dense W8A8
    branch of the reference's prequantize_sol_sageattn_from_qk (core.py
    :711-839 with use_w8a8=True, force_dense=True)."""
    if qk.tensor_layout != "HND":
        raise ValueError("prequantized Sol/W8A8 attention requires HND layout")
    if value.dtype != qk.input_dtype:
        raise TypeError("preprocessed Q/K and V must have matching logical dtypes")
    if value.device != qk.query_int8.device:
        raise ValueError("preprocessed Q/K and V must share one CUDA device")
    if value.ndim != 4 or value.stride(-1) != 1:
        raise ValueError("preprocessed Sol V must be four-dimensional with contiguous channels")
    if value.shape != qk.key_int8.shape:
        raise ValueError("preprocessed Q/K and V shapes are incompatible")
    tile = _key_tile_tokens(key_tile_tokens, qk.key_int8.size(2))
    with torch.cuda.device(value.device):
        value_int8, value_scale = quantize_v_int8(value)
        if value_int8.size(2) != KERNEL_HEAD_DIM:
            pad = KERNEL_HEAD_DIM - value_int8.size(2)
            value_int8 = torch.nn.functional.pad(value_int8, (0, 0, 0, pad))
            value_scale = torch.nn.functional.pad(value_scale, (0, pad), value=1.0e-12)
        q_int8 = _pad_channels(qk.query_int8, KERNEL_HEAD_DIM)
        k_int8 = _pad_channels(qk.key_int8, KERNEL_HEAD_DIM)
    scale = float(sm_scale) if sm_scale is not None else qk.original_head_dim ** -0.5
    return PrequantizedW8A8Attention(
        query_int8=q_int8, query_scale=qk.query_scale, key_int8=k_int8, key_scale=qk.key_scale,
        value_int8=value_int8, value_scale=value_scale, output_dtype=value.dtype,
        sm_scale=scale, original_head_dim=qk.original_head_dim, key_tile_tokens=tile,
        is_causal=bool(is_causal), route_original_basis=bool(qk.route_original_basis),
    )


def prequantize_w8a8attn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    tensor_layout: str = "HND",
    sm_scale: Optional[float] = None,
    key_tile_tokens: int = 0,
    rotate_qk: bool = True,
    stabilize_k: bool = True,
    is_causal: bool = False,
) -> PrequantizedW8A8Attention:
    """Q/K/V quantization of the dense W8A8 path before the output exists,
    the reference's prequantize_sol_sageattn (core.py:841-913) with
    use_w8a8=True, force_dense=True: head_dim padded to 64 or 128, Q/K
    through the rotated (and, with ``stabilize_k``, anchored) quantizer,
    V per channel."""
    if not q.is_cuda:
        raise ValueError("Input tensors must be on CUDA")
    if tensor_layout != "HND":
        raise ValueError("Sol sparse attention currently requires HND layout")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("Sol sparse Q/K/V must be float16 or bfloat16")
    if q.device != k.device or q.device != v.device:
        raise ValueError("Q/K/V must be on the same device")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError("Q/K/V must have matching dtypes")
    _validate_fixed_qkv(q, k, v, tensor_layout)
    head_dim = q.size(-1)
    if not 0 < head_dim <= 128:
        raise ValueError("Sol sparse attention requires head_dim in [1, 128]")
    if q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("the last Q/K/V dimension must be contiguous")
    kernel_head_dim = 64 if head_dim <= 64 else 128
    with torch.cuda.device(q.device):
        q, k, v = (_pad_channels(t, kernel_head_dim) for t in (q, k, v))
        q_int8, q_scale, k_int8, k_scale = per_warp_int8_hadamard(
            q, k, tensor_layout="HND", stabilize_k=bool(stabilize_k) and bool(rotate_qk), rotate=bool(rotate_qk))
    qk = PrequantizedQK(
        query_int8=q_int8, query_scale=q_scale, key_int8=k_int8, key_scale=k_scale, tensor_layout="HND",
        input_dtype=v.dtype, original_head_dim=head_dim, route_original_basis=bool(rotate_qk),
    )
    return prequantize_w8a8attn_from_qk(qk, v, sm_scale=sm_scale, key_tile_tokens=key_tile_tokens,
                                        is_causal=is_causal)


def w8a8attn_from_prequantized(quantized: PrequantizedW8A8Attention) -> torch.Tensor:
    """Runs the dense W8A8 kernel (reference sol_sparse_sageattn_from_prequantized,
    core.py:916-982, W8A8 force-dense branch) with the reference's exact
    running row maximum.  Output [B, Hq, Lq, head_dim] in the input dtype."""
    q8, k8 = quantized.query_int8, quantized.key_int8
    batch, hq, lq, dim = q8.shape
    hkv, lk = k8.size(1), k8.size(2)
    device = q8.device
    if quantized.output_dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("W8A8 output must be float16 or bfloat16")
    with torch.cuda.device(device):
        out = torch.empty((batch, hq, lq, dim), dtype=quantized.output_dtype, device=device)
        _lib.call(
            "tu_w8a8_attn_fwd", q8.data_ptr(), quantized.query_scale.data_ptr(), quantized.query_scale.size(-1),
            k8.data_ptr(), quantized.key_scale.data_ptr(), quantized.key_scale.size(-1),
            quantized.value_int8.data_ptr(), quantized.value_scale.data_ptr(), quantized.value_int8.size(-1), out.data_ptr(), int(quantized.output_dtype == torch.float16),
            batch, hq, hkv, lq, lk, dim, q8.stride(0), q8.stride(1), q8.stride(2),
            k8.stride(0), k8.stride(1), k8.stride(2), out.stride(0), out.stride(1), out.stride(2),
            float(quantized.sm_scale), int(quantized.is_causal), _lib.stream_of(device),
        )
    return out[..., : quantized.original_head_dim]


def w8a8attn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    key_tile_tokens: int = 0,
    rotate_qk: bool = True,
    stabilize_k: bool = True,
) -> torch.Tensor:
    """Dense INT8 QK / INT8 PV attention, the reference's ``w8a8attn``
    (core.py:657-708): NHD inputs are made HND-contiguous, Q/K rotated by
    the shared Hadamard transform (K centred on its anchor), V quantized per
    channel, P packed to unsigned 8 bits with the exp2 offset log2(255)."""
    if tensor_layout not in {"HND", "NHD"}:
        raise ValueError(f"Unsupported tensor_layout: {tensor_layout}")
    if tensor_layout == "NHD":
        q_hnd, k_hnd, v_hnd = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    else:
        q_hnd, k_hnd, v_hnd = q, k, v
    _validate_fixed_qkv(q_hnd, k_hnd, v_hnd, "HND")
    if q_hnd.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("Turing W8A8 Q/K/V must be float16 or bfloat16")
    if q_hnd.dtype != k_hnd.dtype or q_hnd.dtype != v_hnd.dtype:
        raise TypeError("Turing W8A8 Q/K/V must have matching dtypes")
    if not 0 < q_hnd.size(-1) <= 128:
        raise ValueError("Turing W8A8 requires head_dim in [1, 128]")
    quantized = prequantize_w8a8attn(
        q_hnd, k_hnd, v_hnd, tensor_layout="HND", sm_scale=sm_scale, key_tile_tokens=key_tile_tokens,
        rotate_qk=rotate_qk, stabilize_k=stabilize_k, is_causal=bool(is_causal),
    )
    output = w8a8attn_from_prequantized(quantized)
    return output.transpose(1, 2) if tensor_layout == "NHD" else output


# The reference's split API names for the dense W8A8 path (the calls
# comfyui_turing_utils/attention/stable.py:430-518 makes).  Only the
# configuration that path uses is built: use_w8a8=True with force_dense=True
# (the Sol sparse router is out of scope); everything else is refused.

def _require_dense_w8a8(use_w8a8: bool, force_dense: bool, dense_query_ranges, exact_kv_ranges,
                        residual_subblocks: int) -> None:
    if not (use_w8a8 and force_dense):
        raise ValueError("only dense W8A8 (use_w8a8=True, force_dense=True) of the Sol path is built for gfx950")
    if int(residual_subblocks) not in (1, 2):
        raise ValueError("residual_subblocks must be 1 or 2")
    # Sol routing ranges only steer the sparse router; dense attention reads
    # every key, so they are validated for shape and otherwise unused.
    for ranges in (dense_query_ranges, exact_kv_ranges):
        for item in ranges or ():
            if not isinstance(item, (tuple, list)) or len(item) != 2:
                raise ValueError("Sol policy ranges must contain (start, stop) pairs")


def prequantize_sol_sageattn_from_qk(
    qk: PrequantizedQK,
    value: torch.Tensor,
    *,
    sm_scale: Optional[float] = None,
    dense_query_ranges=(),
    exact_kv_ranges=(),
    threshold_sigma: float = 1.0,
    residual_subblocks: int = 1,
    use_w8a8: bool = False,
    force_dense: bool = False,
    key_tile_tokens: int = 0,
    is_causal: bool = False,
) -> PrequantizedW8A8Attention:
    """Reference core.py:711-839, dense W8A8 configuration only."""
    _require_dense_w8a8(use_w8a8, force_dense, dense_query_ranges, exact_kv_ranges, residual_subblocks)
    return prequantize_w8a8attn_from_qk(qk, value, sm_scale=sm_scale, key_tile_tokens=key_tile_tokens,
                                        is_causal=is_causal)


def prequantize_sol_sageattn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    tensor_layout: str = "HND",
    sm_scale: Optional[float] = None,
    dense_query_ranges=(),
    exact_kv_ranges=(),
    threshold_sigma: float = 1.0,
    residual_subblocks: int = 1,
    use_w8a8: bool = False,
    force_dense: bool = False,
    key_tile_tokens: int = 0,
    rotate_qk: bool = True,
    stabilize_k: bool = True,
    is_causal: bool = False,
) -> PrequantizedW8A8Attention:
    """Reference core.py:841-913, dense W8A8 configuration only."""
    _require_dense_w8a8(use_w8a8, force_dense, dense_query_ranges, exact_kv_ranges, residual_subblocks)
    return prequantize_w8a8attn(q, k, v, tensor_layout=tensor_layout, sm_scale=sm_scale,
                                key_tile_tokens=key_tile_tokens, rotate_qk=rotate_qk, stabilize_k=stabilize_k,
                                is_causal=is_causal)


def sol_sparse_sageattn_from_prequantized(quantized: PrequantizedW8A8Attention, *, return_stats: bool = False):
    """Reference core.py:916-982 for a dense W8A8 state.  With
    ``return_stats`` the dense path reports no routed blocks: (output, 0, 0)."""
    output = w8a8attn_from_prequantized(quantized)
    return (output, 0, 0) if return_stats else output
