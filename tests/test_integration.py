"""Plugin-side routing of the two hot-path callers (integration.py), on the CPU.

Meta tensors stand in for device tensors: with the device predicate forced
true, the registered ops run their fake implementations, so the routing,
layout normalisation and output restoration are exercised end to end without a
GPU.  The fallback cases mirror the reference's attention override contract
(comfyui_turing_utils/attention/stable.py:83-200)."""
from __future__ import annotations

import inspect

import pytest
import torch

from comfyui_turing_utils_kernel import integration

ALWAYS = staticmethod(lambda device: True)


def _fallback_recorder():
    calls = []

    def original(q, k, v, heads, **kwargs):
        calls.append(kwargs)
        return "fallback"

    return original, calls


def _nhd(b=2, lq=7, lk=9, heads=4, kv_heads=4, d=32, dtype=torch.bfloat16, device="meta"):
    q = torch.empty((b, lq, heads * d), dtype=dtype, device=device)
    k = torch.empty((b, lk, kv_heads * d), dtype=dtype, device=device)
    return q, k, torch.empty_like(k)


@pytest.mark.parametrize("case,kwargs,reason", [
    ("mask", {"mask": torch.zeros(1)}, "mask"),
    ("low_precision", {"low_precision_attention": False}, "low_precision"),
])
def test_fallback_reasons(case, kwargs, reason):
    q, k, v = _nhd()
    call, why = integration.inspect_attention_call(q, k, v, 4, device_predicate=lambda d: True, **kwargs)
    assert call is None and reason in why


def test_unsupported_device_falls_back_with_original_arguments():
    q, k, v = _nhd(device="cpu")
    original, calls = _fallback_recorder()
    out = integration.sage_attention_override(original, q, k, v, 4, skip_output_reshape=True, is_causal=True)
    assert out == "fallback"
    assert calls[0]["skip_output_reshape"] is True and calls[0]["is_causal"] is True


@pytest.mark.parametrize("mutate,reason", [
    (lambda q, k, v: (q, k, v.to(torch.float16)), "dtypes"),
    (lambda q, k, v: (q.to(torch.float64), k.to(torch.float64), v.to(torch.float64)), "unsupported"),
    (lambda q, k, v: (q, k, v[:, :3]), "incompatible"),
])
def test_shape_and_dtype_fallbacks(mutate, reason):
    q, k, v = mutate(*_nhd())
    call, why = integration.inspect_attention_call(q, k, v, 4, device_predicate=lambda d: True)
    assert call is None and reason in why


def test_head_dim_and_contiguity_fallbacks():
    q, k, v = _nhd(heads=2, kv_heads=2, d=160)
    call, why = integration.inspect_attention_call(q, k, v, 2, device_predicate=lambda d: True)
    assert call is None and "head_dim=160" in why
    q = torch.empty((1, 4, 9, 64), dtype=torch.bfloat16, device="meta").transpose(-1, -2)
    call, why = integration.inspect_attention_call(q, q, q, 4, skip_reshape=True, device_predicate=lambda d: True)
    assert call is None


def test_gqa_nhd_call_and_normalisation():
    q, k, v = _nhd(heads=8, kv_heads=2, d=64, dtype=torch.float32)
    call, why = integration.inspect_attention_call(q, k, v, 8, enable_gqa=True, device_predicate=lambda d: True)
    assert why is None
    assert (call.batch, call.heads, call.kv_heads, call.head_dim) == (2, 8, 2, 64)
    assert call.tensor_layout == "NHD" and call.input_dtype == torch.float32
    qn, kn, vn = integration.normalize_attention_tensors(q, k, v, call)
    assert qn.shape == (2, 7, 8, 64) and kn.shape == (2, 9, 2, 64) and qn.dtype == torch.bfloat16
    # without enable_gqa the K width must equal the Q width
    call, why = integration.inspect_attention_call(q, k, v, 8, device_predicate=lambda d: True)
    assert call is None and "head counts" in why


@pytest.mark.parametrize("skip_output_reshape", [False, True])
@pytest.mark.parametrize("skip_reshape", [False, True])
def test_override_routes_to_sage_and_restores_layout(skip_reshape, skip_output_reshape):
    heads, d = 4, 64
    if skip_reshape:
        q = torch.empty((2, heads, 7, d), dtype=torch.float32, device="meta")
        k = torch.empty((2, heads, 9, d), dtype=torch.float32, device="meta")
    else:
        q, k, _ = _nhd(heads=heads, kv_heads=heads, d=d, dtype=torch.float32)
    original, calls = _fallback_recorder()
    out = integration.sage_attention_override(original, q, k, torch.empty_like(k), heads, skip_reshape=skip_reshape,
                                              skip_output_reshape=skip_output_reshape,
                                              device_predicate=lambda dev: True)
    assert not calls
    assert out.dtype == torch.float32
    expect = (2, heads, 7, d) if skip_output_reshape else (2, 7, heads * d)
    assert out.shape == expect


def test_int8_linear_defaults_are_the_reference_defaults():
    """dispatch.py:618-627: out_dtype None, convrot False, convrot_groupsize
    256, input_act None.  A caller that omits them must not get G=128 rotation
    against G=256 weights, or rotated activations against unrotated weights."""
    params = inspect.signature(integration.int8_linear).parameters
    assert list(params) == ["x", "weight", "weight_scale", "bias", "out_dtype", "convrot", "convrot_groupsize",
                            "input_act"]
    assert params["bias"].default is None and params["out_dtype"].default is None
    assert params["convrot"].default is False
    assert params["convrot_groupsize"].default == 256
    assert params["input_act"].default is None


def test_int8_linear_contract(monkeypatch):
    monkeypatch.setattr(integration, "is_supported_device", lambda device: True)
    x = torch.empty((2, 5, 256), dtype=torch.bfloat16, device="meta")
    w = torch.empty((48, 256), dtype=torch.int8, device="meta")
    out = integration.int8_linear(x, w, torch.empty((), dtype=torch.float32, device="meta"), convrot=True)
    assert out.shape == (2, 5, 48) and out.dtype == torch.bfloat16
    out = integration.int8_linear(x, w, torch.empty((48,), device="meta"), convrot=True, convrot_groupsize=128,
                                  out_dtype=torch.float16)
    assert out.dtype == torch.float16
    with pytest.raises(ValueError, match="scalar or have 48"):
        integration.int8_linear(x, w, torch.empty((7,), device="meta"), convrot=True)
    out = integration.int8_linear(x, w, torch.empty((48,), device="meta"), convrot=True, input_act="gelu_tanh")
    assert out.shape == (2, 5, 48)
    xs = torch.empty((2, 5, 512), dtype=torch.bfloat16, device="meta")
    out = integration.int8_linear(xs, w, torch.empty((48,), device="meta"), convrot=True, input_act="swiglu")
    assert out.shape == (2, 5, 48)


# The keyword set comfy-kitchen's registry validates and forwards to a
# registered backend's int8_linear: the params of the plugin's "int8_linear"
# FunctionConstraints (comfyui_turing_utils/quantization/dispatch.py:879-898),
# which are the parameters of dispatch.int8_linear (dispatch.py:618-627).
KITCHEN_INT8_LINEAR_PARAMS = ("x", "weight", "weight_scale", "bias", "out_dtype", "convrot", "convrot_groupsize",
                              "input_act")


def _record_linear_ops(monkeypatch):
    """Wraps the quantizer and GEMM ops the linear path calls (their fake
    implementations on meta tensors) and records what each received."""
    import comfyui_turing_utils_kernel.integration as integ

    calls = []
    real = torch.ops.turing_utils

    class Ops:
        def __getattr__(self, name):
            op = getattr(real, name)

            def wrapped(*args, **kwargs):
                calls.append((name, args, kwargs))
                return op(*args, **kwargs)

            return wrapped

    class Torch:  # integration.torch with .ops.turing_utils recorded
        def __getattr__(self, name):
            return getattr(torch, name)

    fake_torch = Torch()
    fake_torch.ops = type("O", (), {"turing_utils": Ops()})()
    monkeypatch.setattr(integ, "torch", fake_torch)
    monkeypatch.setattr(integ, "is_supported_device", lambda device: True)
    return calls


def test_int8_linear_takes_the_plugin_call_forms(monkeypatch):
    """Every argument set through which the plugin reaches int8_linear, as
    literals, against integration.int8_linear (the function a gfx950 build
    registers or calls in dispatch.int8_linear's place):
      * Kitchen registry: all eight keywords (dispatch.py:879-898);
      * the W8A8 preflight's Kitchen calls (dispatch.py:245-252, :256-264):
        (x, weight, weight_scale) positional, then out_dtype, convrot,
        convrot_groupsize and input_act by keyword;
      * the fused-activation linear (fusions.py:80-89): (x, qdata, scale)
        positional, bias, out_dtype=x.dtype, convrot=True, convrot_groupsize
        and input_act by keyword.
    Each must reach the quantizer with the caller's group and activation and
    the GEMM op of the caller's out_dtype, without importing comfy_kitchen."""
    import sys

    assert tuple(inspect.signature(integration.int8_linear).parameters) == KITCHEN_INT8_LINEAR_PARAMS
    calls = _record_linear_ops(monkeypatch)
    x = torch.empty((2, 16, 256), dtype=torch.bfloat16, device="meta")
    w = torch.empty((64, 256), dtype=torch.int8, device="meta")
    ws = torch.empty((), dtype=torch.float32, device="meta")
    bias = torch.empty((64,), dtype=torch.bfloat16, device="meta")

    registry_kwargs = dict(x=x, weight=w, weight_scale=ws, bias=bias, out_dtype=torch.float16, convrot=True,
                           convrot_groupsize=256, input_act=None)
    assert tuple(registry_kwargs) == KITCHEN_INT8_LINEAR_PARAMS
    out = integration.int8_linear(**registry_kwargs)
    assert out.shape == (2, 16, 64) and out.dtype == torch.float16
    assert [c[0] for c in calls] == ["bf16_int8_convrot_quantize", "int8_linear_out"]
    assert calls[0][1][1] == 256 and calls[0][2] == {"swiglu": False}
    assert calls[1][1][5] is torch.float16

    calls.clear()  # preflight form, bf16 out
    out = integration.int8_linear(x, w, ws, out_dtype=torch.bfloat16, convrot=True, convrot_groupsize=256)
    assert out.dtype == torch.bfloat16 and [c[0] for c in calls] == ["bf16_int8_convrot_quantize", "int8_linear"]

    calls.clear()  # preflight SwiGLU form
    xs = torch.empty((2, 16, 512), dtype=torch.bfloat16, device="meta")
    out = integration.int8_linear(xs, w, ws, out_dtype=torch.bfloat16, convrot=True, convrot_groupsize=256,
                                  input_act="swiglu")
    assert out.shape == (2, 16, 64) and calls[0][2] == {"swiglu": True}

    calls.clear()  # fusions.py form, GELU folded, fp32 out
    out = integration.int8_linear(x, w, ws, bias=bias, out_dtype=torch.float32, convrot=True,
                                  convrot_groupsize=128, input_act="gelu_tanh")
    assert out.dtype == torch.float32
    assert [c[0] for c in calls] == ["bf16_gelu_int8_convrot_quantize", "int8_linear_out"]
    assert calls[0][1][1] == 128 and calls[1][1][5] is torch.float32
    assert "comfy_kitchen" not in sys.modules


def test_int8_linear_declines_what_it_cannot_serve():
    x = torch.zeros((3, 256), dtype=torch.bfloat16)
    w = torch.zeros((16, 256), dtype=torch.int8)
    s = torch.ones(16)
    with pytest.raises(NotImplementedError, match="gfx950"):
        integration.int8_linear(x, w, s, convrot=True)
    with pytest.raises(NotImplementedError, match="bfloat16"):
        integration.int8_linear(x.float(), w, s, convrot=True)
    with pytest.raises(NotImplementedError, match="ConvRot"):
        integration.int8_linear(x, w, s)  # the default convrot=False
    with pytest.raises(ValueError, match="activation"):
        integration.int8_linear(x, w, s, input_act="gelu")


def test_fallback_forwards_every_argument_as_received():
    """stable.py:611-618: the fallback gets (q, k, v, heads) and mask,
    attn_precision, skip_reshape, skip_output_reshape plus every other keyword
    (low_precision_attention, scale, transformer_options, ...), unchanged."""
    q, k, v = _nhd()
    original, calls = _fallback_recorder()
    opts = {"x": 1}
    out = integration.sage_attention_override(original, q, k, v, 4, attn_precision=torch.float32,
                                              low_precision_attention=False, scale=0.3, transformer_options=opts,
                                              enable_gqa=False, device_predicate=lambda d: True)
    assert out == "fallback"
    kw = calls[0]
    assert kw["low_precision_attention"] is False and kw["scale"] == 0.3 and kw["transformer_options"] is opts
    assert kw["attn_precision"] is torch.float32 and kw["mask"] is None and kw["enable_gqa"] is False
    assert "device_predicate" not in kw and "_turing_kernel" not in kw
    # the w8a8 entry (turing_w8a8_attention) falls back the same way
    integration.w8a8_attention_override(original, q, k, v, 4, mask=torch.zeros(1), device_predicate=lambda d: True)
    assert "_turing_kernel" not in calls[1] and calls[1]["mask"] is not None
    with pytest.raises(ValueError, match="kernel"):
        integration.sage_attention_override(original, q, k, v, 4, _turing_kernel="sol")


def test_attention_kernel_tuning_parsing():
    """tuning.py:18-32."""
    key = integration.ATTENTION_TUNING_KEY
    assert integration.attention_kernel_tuning(None) == integration.AttentionKernelTuning(0, True, True)
    assert integration.attention_kernel_tuning({key: "x"}) == integration.AttentionKernelTuning(0, True, True)
    t = integration.attention_kernel_tuning({key: {"key_tile_tokens": 128, "rotate_qk": True, "stabilize_k": False}})
    assert t == integration.AttentionKernelTuning(128, True, False)
    t = integration.attention_kernel_tuning({key: {"key_tile_tokens": 96, "rotate_qk": False, "stabilize_k": True}})
    assert t == integration.AttentionKernelTuning(0, False, False)


def test_w8a8_override_routes_to_the_w8a8_op(monkeypatch):
    seen = {}

    def fake_w8a8(q, k, v, layout, causal, sm_scale, tile, rotate, stabilize):
        seen.update(layout=layout, causal=causal, sm_scale=sm_scale, tile=tile, rotate=rotate, stabilize=stabilize)
        return torch.empty_like(q)

    monkeypatch.setattr(torch.ops.turing_utils, "w8a8_attention", fake_w8a8, raising=False)
    q, k, v = _nhd(d=64)
    opts = {integration.ATTENTION_TUNING_KEY: {"key_tile_tokens": 64, "rotate_qk": True, "stabilize_k": False}}
    out = integration.w8a8_attention_override(_not_called, q, k, v, 4, is_causal=True, scale=0.125,
                                              transformer_options=opts, device_predicate=lambda d: True)
    assert out.shape == (2, 7, 4 * 64)
    assert seen == dict(layout="NHD", causal=True, sm_scale=0.125, tile=64, rotate=True, stabilize=False)


def _not_called(*args, **kwargs):
    raise AssertionError("fell back")
