"""``torch.ops.turing_utils.sage_attention`` on gfx950.

Same name, signature and fake implementation as the reference
(``turing_sage/custom_ops.py:137-168``): ``sm_scale <= 0`` selects the default
``head_dim ** -0.5`` and the output is ``empty_like(query)``.  The
implementation is this build's Sage path (K smoothing on, 128-token Q/K
blocks, bf16 PV); see ``core.sageattn``.
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
