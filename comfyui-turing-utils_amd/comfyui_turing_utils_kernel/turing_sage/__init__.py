"""Sage INT8 attention for gfx950 (MI355X).

Facade functions with the reference's names (``turing_sage/__init__.py``):
``available``, ``w8a8_available``, ``split_prequantization_available``,
``fused_qk_preprocessing_available``, ``sageattn``, ``sageattn_compiled``,
``prequantize_sageattn``, ``sageattn_from_prequantized``, ``preflight``.
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
    """The INT8-PV ``w8a8`` attention variant is not built for gfx950."""
    return False


def split_prequantization_available() -> bool:
    """The reference's split API refers to its Sol W8A8 path, not built here."""
    return False


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


# Registers torch.ops.turing_utils.sage_attention on import.
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
    "preflight",
]
