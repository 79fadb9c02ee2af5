"""Sage INT8 attention for gfx950 (MI355X).

Facade functions with the reference's names (``turing_sage/__init__.py``):
``available``, ``w8a8_available``, ``split_prequantization_available``,
``fused_qk_preprocessing_available``, ``sageattn``, ``sageattn_compiled``,
``prequantize_sageattn``, ``sageattn_from_prequantized``, ``preflight``, and the
dense W8A8 path: ``w8a8attn``, ``w8a8attn_compiled``, ``prequantize_sol_sageattn``,
``prequantize_sol_sageattn_from_qk``, ``sol_sparse_sageattn_from_prequantized``,
``preflight_w8a8``.
"""
from __future__ import annotations

import os

import torch

from .. import _lib


def available() -> bool:
    """True when the gfx950 kernel library is present and loads."""
    if not os.path.exists(_lib.LIB_PATH):
        return False
    try:
        _lib.load()
    except RuntimeError:
        return False
    return True


def w8a8_available() -> bool:
    """True when the library (with the dense W8A8 entry points) loads
    (reference turing_sage/__init__.py:52-62)."""
    return available()


def split_prequantization_available() -> bool:
    """The prequantize / execute split of the W8A8 path
    (``prequantize_sol_sageattn[_from_qk]``, ``sol_sparse_sageattn_from_prequantized``)
    in its dense configuration (reference turing_sage/__init__.py:82-95)."""
    return w8a8_available()


def fused_qk_preprocessing_available() -> bool:
    """True when the library (with ``tu_qk_rms_rope_int8``) loads: the fused
    RMSNorm + RoPE + INT8 Q/K preprocessing of the reference's
    ``quant_qk_rms_rope_int8_cuda`` (turing_sage/__init__.py:98-107)."""
    return available()


def sageattn(*args, **kwargs):
    from .core import sageattn as implementation

    return implementation(*args, **kwargs)


def prequantize_sageattn(*args, **kwargs):
    from .core import prequantize_sageattn as implementation

    return implementation(*args, **kwargs)


def prequantize_rms_rope_qk(*args, **kwargs):
    from .core import prequantize_rms_rope_qk as implementation

    return implementation(*args, **kwargs)


def prequantize_sageattn_from_qk(*args, **kwargs):
    from .core import prequantize_sageattn_from_qk as implementation

    return implementation(*args, **kwargs)


def sageattn_from_prequantized(*args, **kwargs):
    from .core import sageattn_from_prequantized as implementation

    return implementation(*args, **kwargs)


def w8a8attn(*args, **kwargs):
    from .core import w8a8attn as implementation

    return implementation(*args, **kwargs)


def prequantize_sol_sageattn(*args, **kwargs):
    from .core import prequantize_sol_sageattn as implementation

    return implementation(*args, **kwargs)


def prequantize_sol_sageattn_from_qk(*args, **kwargs):
    from .core import prequantize_sol_sageattn_from_qk as implementation

    return implementation(*args, **kwargs)


def sol_sparse_sageattn_from_prequantized(*args, **kwargs):
    from .core import sol_sparse_sageattn_from_prequantized as implementation

    return implementation(*args, **kwargs)


def w8a8attn_compiled(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: float | None = None,
    key_tile_tokens: int = 0,
    rotate_qk: bool = True,
    stabilize_k: bool = True,
):
    """Calls the registered ``torch.ops.turing_utils.w8a8_attention`` op
    (reference turing_sage/__init__.py:310-334)."""
    from .custom_ops import w8a8_attention

    return w8a8_attention(q, k, v, tensor_layout, bool(is_causal),
                          float(sm_scale) if sm_scale is not None else -1.0, int(key_tile_tokens),
                          bool(rotate_qk), bool(stabilize_k))


def sageattn_compiled(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    tensor_layout: str = "HND",
    is_causal: bool = False,
    sm_scale: float | None = None,
):
    """Calls the registered ``torch.ops.turing_utils.sage_attention`` op."""
    from .custom_ops import sage_attention

    return sage_attention(q, k, v, tensor_layout, bool(is_causal), float(sm_scale) if sm_scale is not None else -1.0)


def preflight(device: torch.device) -> None:
    """Deterministic self-test against fp32 SDPA (reference gate rtol 0.08 / atol 0.05,
    turing_sage/__init__.py:612-663).  Raises RuntimeError on failure."""
    if device.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError(f"Sage attention requires a GPU device, got {device}")
    if not _lib.device_supported(device):
        raise RuntimeError(f"Sage attention requires a gfx950 GPU, got {device}")
    with torch.inference_mode(), torch.cuda.device(device):
        for head_dim in (64, 96, 128):
            q_values = torch.arange(4 * 65 * head_dim, device=device, dtype=torch.float32)
            kv_values = torch.arange(2 * 73 * head_dim, device=device, dtype=torch.float32)
            q = (((q_values % 29) - 14) / 32).reshape(1, 4, 65, head_dim).to(torch.bfloat16)
            k = ((((kv_values * 3) % 31) - 15) / 32).reshape(1, 2, 73, head_dim).to(torch.bfloat16)
            v = ((((kv_values * 5) % 37) - 18) / 32).reshape(1, 2, 73, head_dim).to(torch.bfloat16)
            output = sageattn(q, k, v, tensor_layout="HND")
            reference = torch.nn.functional.scaled_dot_product_attention(
                q.float(), k.float(), v.float(), enable_gqa=True
            )
            if (
                output.dtype != torch.bfloat16
                or output.shape != q.shape
                or not torch.isfinite(output).all()
                or not torch.allclose(output.float(), reference, rtol=0.08, atol=0.05)
            ):
                raise RuntimeError(f"Sage attention BF16 D={head_dim} self-test failed")
        torch.cuda.synchronize(device)


def preflight_w8a8(device: torch.device) -> None:
    """The reference's W8A8 self-test (turing_sage/__init__.py:573-609):
    arange-derived Q/K/V, B1 Hq4 Hkv2 Lq129 Lk151, D 64 and 128, against
    fp32 SDPA with rtol 0.12 / atol 0.09.  Raises RuntimeError on failure."""
    if device.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError(f"W8A8 attention requires a GPU device, got {device}")
    if not _lib.device_supported(device):
        raise RuntimeError(f"W8A8 attention requires a gfx950 GPU, got {device}")
    if not w8a8_available():
        raise RuntimeError("the W8A8 attention extension is not built")
    with torch.inference_mode(), torch.cuda.device(device):
        for head_dim in (64, 128):
            q_values = torch.arange(4 * 129 * head_dim, device=device, dtype=torch.float32)
            kv_values = torch.arange(2 * 151 * head_dim, device=device, dtype=torch.float32)
            q = (((q_values % 29) - 14) / 16).reshape(1, 4, 129, head_dim).to(torch.bfloat16)
            k = ((((kv_values * 3) % 31) - 15) / 16).reshape(1, 2, 151, head_dim).to(torch.bfloat16)
            v = ((((kv_values * 5) % 37) - 18) / 16).reshape_as(k).to(torch.bfloat16)
            output = w8a8attn(q, k, v)
            reference = torch.nn.functional.scaled_dot_product_attention(
                q.float(), k.float(), v.float(), enable_gqa=True
            )
            if (
                output.dtype != torch.bfloat16
                or output.shape != q.shape
                or not torch.isfinite(output).all()
                or not torch.allclose(output.float(), reference, rtol=0.12, atol=0.09)
            ):
                raise RuntimeError(f"W8A8 attention BF16 D={head_dim} self-test failed")
        torch.cuda.synchronize(device)


# Registers the torch.ops.turing_utils attention ops on import.
from . import custom_ops  # noqa: E402,F401

__all__ = [
    "available",
    "w8a8_available",
    "split_prequantization_available",
    "fused_qk_preprocessing_available",
    "sageattn",
    "sageattn_compiled",
    "prequantize_sageattn",
    "prequantize_rms_rope_qk",
    "prequantize_sageattn_from_qk",
    "sageattn_from_prequantized",
    "w8a8attn",
    "w8a8attn_compiled",
    "prequantize_sol_sageattn",
    "prequantize_sol_sageattn_from_qk",
    "sol_sparse_sageattn_from_prequantized",
    "preflight",
    "preflight_w8a8",
]
