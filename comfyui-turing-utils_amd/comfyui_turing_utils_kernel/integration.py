"""Plugin-side counterpart of the hot path's two callers, for MI355X.

The reference plugin reaches the kernel package from two places:

* ``comfyui_turing_utils/quantization/dispatch.py:618-670`` -- ``int8_linear``:
  reshape to 2D, ConvRot-quantize the activation (optionally folding a
  tanh-GELU or SwiGLU input activation), run the W8A8 GEMM, reshape back.
  Calls it cannot serve are handed to comfy-kitchen.
* ``comfyui_turing_utils/attention/stable.py:83-200, :593-711`` -- the
  attention override: inspect the call, fall back to the caller's attention
  for anything unsupported (mask, head_dim > 128, dtype/device mismatch,
  non-contiguous channels), normalise NHD/HND and fp32 -> bf16, run Sage,
  restore the caller's layout and dtype.

This module restates both contracts against the gfx950 ops.  The device
predicate is ``_lib.device_supported`` (gfx950) in place of the sm75 check of
``comfyui_turing_utils/hardware.py:24-32``.  comfy-kitchen does not exist on
ROCm, so where the reference delegates to it, ``int8_linear`` raises
``NotImplementedError`` naming the reason; the caller keeps its own path.
"""
from __future__ import annotations

import dataclasses
from typing import Callable

import torch

from . import _lib, ops  # noqa: F401  (ops registers torch.ops.turing_utils.*)

SUPPORTED_INPUT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def is_supported_device(device: torch.device) -> bool:
    """gfx950 predicate (replaces ``is_supported_turing_device``)."""
    try:
        return _lib.device_supported(device)
    except RuntimeError:
        return False


# ---------------------------------------------------------------------------
# W8A8 linear (dispatch.py:618-670)
# ---------------------------------------------------------------------------
def int8_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
    out_dtype: torch.dtype | None = None,
    convrot: bool = False,
    convrot_groupsize: int = 256,
    input_act: str | None = None,
) -> torch.Tensor:
    """ConvRot W8A8 linear: y = dequant(int8(R act(x)) @ W^T) * s_x * s_w + bias.

    x: bf16 [..., K] ([..., 2K] for ``input_act="swiglu"``); weight: int8 [N, K];
    weight_scale: fp32 scalar or [N]; bias: [N] or None; input_act: None /
    "none", "gelu_tanh" or "swiglu" (dispatch.py:326-393), folded into the
    quantizer.  Returns [..., N] in ``out_dtype`` (default x.dtype).

    The defaults are the reference's (dispatch.py:618-627): ``convrot=False``
    (unrotated activations, which only comfy-kitchen serves: refused here) and
    ``convrot_groupsize=256``.  A caller whose weights were rotated with
    groups of 128 (this build's extension) passes ``convrot_groupsize=128``.
    """
    if input_act not in (None, "none", "swiglu", "gelu_tanh"):
        raise ValueError(f"unsupported fused INT8 activation: {input_act!r}")
    if x.dtype != torch.bfloat16:
        raise NotImplementedError("gfx950 W8A8 linear takes bfloat16 activations")
    if not convrot:
        raise NotImplementedError("gfx950 W8A8 linear requires ConvRot activations")
    if not is_supported_device(x.device):
        raise NotImplementedError(f"{x.device} is not a gfx950 device")
    original_shape = x.shape
    x2d = x.reshape(-1, original_shape[-1]).contiguous()
    if input_act == "gelu_tanh":
        q, s_x = torch.ops.turing_utils.bf16_gelu_int8_convrot_quantize(x2d, convrot_groupsize)
    else:
        q, s_x = torch.ops.turing_utils.bf16_int8_convrot_quantize(x2d, convrot_groupsize,
                                                                    swiglu=input_act == "swiglu")
    n = weight.shape[0]
    w_scale = weight_scale.to(device=x.device, dtype=torch.float32).reshape(-1)
    if w_scale.numel() == 1:
        w_scale = w_scale.expand(n)
    if w_scale.numel() != n:
        raise ValueError(f"W8A8 weight scale must be scalar or have {n} values, got {w_scale.numel()}")
    out_dtype = out_dtype or x.dtype
    if out_dtype == torch.bfloat16:
        out = torch.ops.turing_utils.int8_linear(q, weight.contiguous(), s_x.reshape(-1), w_scale.contiguous(), bias)
    else:
        # fp16 / fp32: the epilogue rounds its fp32 value once, to out_dtype
        out = torch.ops.turing_utils.int8_linear_out(q, weight.contiguous(), s_x.reshape(-1), w_scale.contiguous(),
                                                     bias, out_dtype)
    return out.reshape(*original_shape[:-1], n)


# ---------------------------------------------------------------------------
# Attention override (stable.py:83-200, :593-711)
# ---------------------------------------------------------------------------
@dataclasses.dataclass(frozen=True)
class AttentionCall:
    batch: int
    heads: int
    kv_heads: int
    head_dim: int
    query_tokens: int
    key_tokens: int
    tensor_layout: str
    input_dtype: torch.dtype
    skip_output_reshape: bool


def inspect_attention_call(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    heads: int,
    *,
    mask=None,
    skip_reshape: bool = False,
    skip_output_reshape: bool = False,
    enable_gqa: bool = False,
    low_precision_attention: bool = True,
    device_predicate: Callable[[torch.device], bool] = is_supported_device,
) -> tuple[AttentionCall | None, str | None]:
    """Returns (call, None) when Sage can serve the call, else (None, reason).
    The checks and their order are the reference's (stable.py:83-165) so that
    the same calls fall back to the caller's attention."""
    if not all(isinstance(t, torch.Tensor) for t in (q, k, v)):
        return None, "Q/K/V are not tensors"
    if not device_predicate(q.device):
        return None, "Q/K/V are not on a supported gfx950 GPU"
    if mask is not None:
        return None, "an attention mask was supplied"
    if not low_precision_attention:
        return None, "low_precision_attention=False"
    if q.dtype != k.dtype or q.dtype != v.dtype:
        return None, "Q/K/V dtypes do not match"
    if q.dtype not in SUPPORTED_INPUT_DTYPES:
        return None, f"Q/K/V dtype {q.dtype} is unsupported"
    if q.device != k.device or q.device != v.device:
        return None, "Q/K/V devices do not match"
    heads = int(heads)
    if skip_reshape:
        if q.ndim != 4 or k.ndim != 4 or v.ndim != 4 or heads <= 0 or q.shape[1] != heads:
            return None, "skip_reshape Q/K/V layout is incompatible"
        batch, _, query_tokens, head_dim = q.shape
        kv_heads, key_tokens = k.shape[1], k.shape[2]
        layout = "HND"
        if (k.shape[0] != batch or v.shape[0] != batch or k.shape != v.shape or k.shape[-1] != head_dim
                or kv_heads <= 0 or heads % kv_heads):
            return None, "Q/K/V shapes or head counts are incompatible"
    else:
        if q.ndim != 3 or k.ndim != 3 or v.ndim != 3 or heads <= 0 or q.shape[-1] % heads:
            return None, "unreshaped Q/K/V layout is incompatible"
        batch = q.shape[0]
        head_dim = q.shape[-1] // heads
        if head_dim <= 0 or k.shape[0] != batch or v.shape[0] != batch or k.shape != v.shape:
            return None, "unreshaped Q/K/V shapes are incompatible"
        kv_heads = k.shape[-1] // head_dim if enable_gqa else heads
        if kv_heads <= 0 or k.shape[-1] != kv_heads * head_dim or heads % kv_heads:
            return None, "unreshaped K/V head counts are incompatible"
        query_tokens, key_tokens = q.shape[1], k.shape[1]
        layout = "NHD"
    if query_tokens <= 0 or key_tokens <= 0:
        return None, "empty Q/K sequences are unsupported"
    if not 0 < head_dim <= 128:
        return None, f"head_dim={head_dim} is unsupported by Sage"
    if q.stride(-1) != 1 or k.stride(-1) != 1 or v.stride(-1) != 1:
        return None, "the last Q/K/V dimension is not contiguous"
    return AttentionCall(batch, heads, kv_heads, head_dim, query_tokens, key_tokens, layout, q.dtype,
                         bool(skip_output_reshape)), None


def normalize_attention_tensors(q, k, v, call: AttentionCall):
    if call.tensor_layout == "NHD":
        q = q.reshape(call.batch, call.query_tokens, call.heads, call.head_dim)
        k = k.reshape(call.batch, call.key_tokens, call.kv_heads, call.head_dim)
        v = v.reshape(call.batch, call.key_tokens, call.kv_heads, call.head_dim)
    if call.input_dtype == torch.float32:
        q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    return q, k, v


def finish_attention_output(output: torch.Tensor, call: AttentionCall) -> torch.Tensor:
    if call.tensor_layout == "HND":
        result = output if call.skip_output_reshape else output.transpose(1, 2).reshape(
            call.batch, -1, call.heads * call.head_dim)
    elif call.skip_output_reshape:
        result = output.transpose(1, 2)
    else:
        result = output.reshape(call.batch, -1, call.heads * call.head_dim)
    return result.to(call.input_dtype) if call.input_dtype == torch.float32 else result


ATTENTION_TUNING_KEY = "turing_utils_attention_tuning"


@dataclasses.dataclass(frozen=True)
class AttentionKernelTuning:
    """W8A8 attention controls a model patch stores in ``transformer_options``
    (comfyui_turing_utils/attention/tuning.py:8-32)."""
    key_tile_tokens: int = 0
    rotate_qk: bool = True
    stabilize_k: bool = True


def attention_kernel_tuning(transformer_options) -> AttentionKernelTuning:
    """tuning.py:18-32: invalid or missing settings give the defaults; K
    stabilisation needs the rotation."""
    if not isinstance(transformer_options, dict):
        return AttentionKernelTuning()
    raw = transformer_options.get(ATTENTION_TUNING_KEY)
    if not isinstance(raw, dict):
        return AttentionKernelTuning()
    key_tile_tokens = int(raw.get("key_tile_tokens", 0))
    if key_tile_tokens not in (0, 64, 128):
        key_tile_tokens = 0
    rotate_qk = bool(raw.get("rotate_qk", True))
    return AttentionKernelTuning(key_tile_tokens=key_tile_tokens, rotate_qk=rotate_qk,
                                 stabilize_k=rotate_qk and bool(raw.get("stabilize_k", True)))


def sage_attention_override(
    original: Callable,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    heads: int,
    mask=None,
    attn_precision=None,
    skip_reshape: bool = False,
    skip_output_reshape: bool = False,
    *,
    device_predicate: Callable[[torch.device], bool] = is_supported_device,
    **kwargs,
):
    """``attention_override`` body (``turing_sage_attention``,
    stable.py:593-706): serve the call with ``torch.ops.turing_utils.
    sage_attention`` -- or ``w8a8_attention`` when ``_turing_kernel="w8a8"``
    (``turing_w8a8_attention``, the loader default) -- or hand it to
    ``original`` with every argument as received.  ``enable_gqa``,
    ``low_precision_attention``, ``is_causal``, ``scale`` and
    ``transformer_options`` are read from ``kwargs`` as the reference does;
    ``device_predicate`` is this build's test hook and is not forwarded."""
    kernel = kwargs.pop("_turing_kernel", "sage")
    if kernel not in ("sage", "w8a8"):
        raise ValueError(f"unsupported bundled attention kernel: {kernel}")
    call, reason = inspect_attention_call(
        q, k, v, heads, mask=mask, skip_reshape=skip_reshape, skip_output_reshape=skip_output_reshape,
        enable_gqa=bool(kwargs.get("enable_gqa", False)),
        low_precision_attention=kwargs.get("low_precision_attention", True), device_predicate=device_predicate,
    )
    if call is None:
        return original(q, k, v, heads, mask=mask, attn_precision=attn_precision, skip_reshape=skip_reshape,
                        skip_output_reshape=skip_output_reshape, **kwargs)
    qn, kn, vn = normalize_attention_tensors(q, k, v, call)
    scale = kwargs.get("scale")
    sm_scale = float(scale) if scale is not None else -1.0  # <= 0: the op's default head_dim ** -0.5
    is_causal = bool(kwargs.get("is_causal", False))
    if kernel == "w8a8":
        tuning = attention_kernel_tuning(kwargs.get("transformer_options"))
        out = torch.ops.turing_utils.w8a8_attention(qn, kn, vn, call.tensor_layout, is_causal, sm_scale,
                                                    tuning.key_tile_tokens, tuning.rotate_qk, tuning.stabilize_k)
    else:
        out = torch.ops.turing_utils.sage_attention(qn, kn, vn, call.tensor_layout, is_causal, sm_scale)
    return finish_attention_output(out, call)


def w8a8_attention_override(*args, **kwargs):
    """``turing_w8a8_attention`` (stable.py:709-711)."""
    kwargs["_turing_kernel"] = "w8a8"
    return sage_attention_override(*args, **kwargs)
