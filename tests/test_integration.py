"""Plugin-side routing of the two hot-path callers (integration.py), on the CPU.

Meta tensors stand in for device tensors: with the device predicate forced
true, the registered ops run their fake implementations, so the routing,
layout normalisation and output restoration are exercised end to end without a
GPU.  The fallback cases mirror the reference's attention override contract
(comfyui_turing_utils/attention/stable.py:83-200)."""
from __future__ import annotations

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


def test_int8_linear_contract(monkeypatch):
    monkeypatch.setattr(integration, "is_supported_device", lambda device: True)
    x = torch.empty((2, 5, 256), dtype=torch.bfloat16, device="meta")
    w = torch.empty((48, 256), dtype=torch.int8, device="meta")
    out = integration.int8_linear(x, w, torch.empty((), dtype=torch.float32, device="meta"))
    assert out.shape == (2, 5, 48) and out.dtype == torch.bfloat16
    out = integration.int8_linear(x, w, torch.empty((48,), device="meta"), convrot_groupsize=256,
                                  out_dtype=torch.float16)
    assert out.dtype == torch.float16
    with pytest.raises(ValueError, match="scalar or have 48"):
        integration.int8_linear(x, w, torch.empty((7,), device="meta"))
    out = integration.int8_linear(x, w, torch.empty((48,), device="meta"), input_act="gelu_tanh")
    assert out.shape == (2, 5, 48)
    xs = torch.empty((2, 5, 512), dtype=torch.bfloat16, device="meta")
    out = integration.int8_linear(xs, w, torch.empty((48,), device="meta"), input_act="swiglu")
    assert out.shape == (2, 5, 48)


def test_int8_linear_declines_what_it_cannot_serve():
    x = torch.zeros((3, 256), dtype=torch.bfloat16)
    w = torch.zeros((16, 256), dtype=torch.int8)
    s = torch.ones(16)
    with pytest.raises(NotImplementedError, match="gfx950"):
        integration.int8_linear(x, w, s)
    with pytest.raises(NotImplementedError, match="bfloat16"):
        integration.int8_linear(x.float(), w, s)
    with pytest.raises(NotImplementedError, match="ConvRot"):
        integration.int8_linear(x, w, s, convrot=False)
    with pytest.raises(ValueError, match="activation"):
        integration.int8_linear(x, w, s, input_act="gelu")
