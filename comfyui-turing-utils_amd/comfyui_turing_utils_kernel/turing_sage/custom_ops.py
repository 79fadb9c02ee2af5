"""``torch.ops.turing_utils.sage_attention``, ``w8a8_attention`` and
``qk_rms_rope_int8`` on gfx950.

Same names, signatures and fake implementations as the reference
(``turing_sage/custom_ops.py:63-168``).  ``sage_attention``: ``sm_scale <= 0``
selects the default ``head_dim ** -0.5`` and the output is
``empty_like(query)``; the implementation is this build's Sage path (K
smoothing on, 128-token Q/K blocks, bf16 PV), see ``core.sageattn``.
``w8a8_attention``: dense INT8 QK / INT8 PV attention (``core.w8a8attn``);
``sm_scale <= 0`` selects the default.
``qk_rms_rope_int8``: fused RMSNorm + RoPE + INT8 of Q (16-token scales,
padded to multiples of 4 per 64 tokens) and K (64-token scales).
"""
from __future__ import annotations

import torch


@torch.library.custom_op("turing_utils::sage_attention", mutates_args=())
def sage_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    tensor_layout: str,
    is_causal: bool,
    sm_scale: float,
) -> torch.Tensor:
    from .core import sageattn

    return sageattn(
        query,
        key,
        value,
        tensor_layout=tensor_layout,
        is_causal=is_causal,
        sm_scale=sm_scale if sm_scale > 0.0 else None,
    )


@sage_attention.register_fake
def _sage_attention_fake(query, key, value, tensor_layout, is_causal, sm_scale):
    return torch.empty_like(query)


@torch.library.custom_op("turing_utils::w8a8_attention", mutates_args=())
def w8a8_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    tensor_layout: str,
    is_causal: bool,
    sm_scale: float,
    key_tile_tokens: int,
    rotate_qk: bool,
    stabilize_k: bool,
) -> torch.Tensor:
    """Reference turing_sage/custom_ops.py:171-195."""
    from .core import w8a8attn

    return w8a8attn(
        query,
        key,
        value,
        tensor_layout=tensor_layout,
        is_causal=is_causal,
        sm_scale=sm_scale if sm_scale > 0.0 else None,
        key_tile_tokens=key_tile_tokens,
        rotate_qk=rotate_qk,
        stabilize_k=stabilize_k,
    )


@w8a8_attention.register_fake
def _w8a8_attention_fake(query, key, value, tensor_layout, is_causal, sm_scale, key_tile_tokens, rotate_qk,
                         stabilize_k):
    return torch.empty_like(query)


@torch.library.custom_op("turing_utils::qk_rms_rope_int8", mutates_args=())
def qk_rms_rope_int8(
    query: torch.Tensor,
    key: torch.Tensor,
    query_norm: torch.Tensor,
    key_norm: torch.Tensor,
    freqs: torch.Tensor,
    epsilon: float,
    rot_dim: int,
    tensor_layout: str,
    norm_scope: str,
    split_half: bool,
    rotate_qk: bool,
    stabilize_k: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused Q/K RMSNorm + RoPE + INT8, the reference's op of the same name
    (turing_sage/custom_ops.py:63-134); an empty ``freqs`` means no RoPE."""
    from .quant import rms_rope_per_warp_int8

    return rms_rope_per_warp_int8(
        query,
        key,
        query_norm,
        key_norm,
        freqs if freqs.numel() else None,
        epsilon=epsilon,
        rot_dim=rot_dim,
        tensor_layout=tensor_layout,
        norm_scope=norm_scope,
        split_half=split_half,
        rotate_qk=rotate_qk,
        stabilize_k=stabilize_k,
    )


@qk_rms_rope_int8.register_fake
def _qk_rms_rope_int8_fake(query, key, query_norm, key_norm, freqs, epsilon, rot_dim, tensor_layout, norm_scope,
                           split_half, rotate_qk, stabilize_k):
    if tensor_layout == "HND":
        batch, query_heads, query_tokens, _ = query.shape
        _, key_heads, key_tokens, _ = key.shape
    elif tensor_layout == "NHD":
        batch, query_tokens, query_heads, _ = query.shape
        _, key_tokens, key_heads, _ = key.shape
    else:
        raise ValueError(f"Unknown tensor layout: {tensor_layout}")
    return (
        torch.empty_like(query, dtype=torch.int8),
        torch.empty((batch, query_heads, (query_tokens + 63) // 64 * 4), dtype=torch.float32, device=query.device),
        torch.empty_like(key, dtype=torch.int8),
        torch.empty((batch, key_heads, (key_tokens + 63) // 64), dtype=torch.float32, device=key.device),
    )
