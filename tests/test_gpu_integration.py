"""GPU parity of the two plugin-side callers on real device tensors.

* ``integration.int8_linear`` -- the capability path of
  ``comfyui_turing_utils/quantization/dispatch.py:618-670``: 3-D activations
  reshaped to rows, the ConvRot quantizer (none / tanh-GELU / SwiGLU input
  activation, ``_quantize_turing_int8_activation``, dispatch.py:326-393), the
  INT8 GEMM with the scale / bias epilogue, scalar or per-channel weight
  scales (dispatch.py:538-615), ``out_dtype``.  Checked bit for bit against the
  oracle chain convrot_quant -> int8_gemm_i32 -> epilogue_bf16 on sampled rows
  (every stage is row-independent, so a row subset is an exact check).
* ``integration.sage_attention_override`` -- ``turing_sage_attention``'s
  inspect / normalise / finish contract (comfyui_turing_utils/attention/
  stable.py:83-200, :593-706): NHD 3-D and HND 4-D inputs, GQA, fp32 inputs,
  ``skip_output_reshape``; outputs against the oracle's quantized attention
  within the north-star gate, and every fallback case returns the caller's
  own result untouched.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from comfyui_turing_utils_kernel import integration
from comfyui_turing_utils_kernel.turing_sage.correctness import (
    attention_error_metrics,
    require_attention_correctness,
)
from oracle import oracle
from tests import inputs

pytestmark = pytest.mark.gpu

GATE = dict(max_abs=2e-2, cosine=0.999)


def _oracle_linear(x2d: torch.Tensor, rows: np.ndarray, w: torch.Tensor, ws: torch.Tensor, bias, group: int,
                   act: int) -> np.ndarray:
    """bf16 bits [len(rows), N] of the reference chain on the given rows."""
    q, s = oracle.convrot_quant(inputs.bits(x2d[torch.from_numpy(rows)]), group, act=act)
    acc = oracle.int8_gemm_i32(q, w.numpy())
    b = None if bias is None else bias.float().numpy()
    return oracle.epilogue_bf16(acc, s, ws.float().numpy().reshape(-1), b)


def _rows(m: int, n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, n)])).astype(np.int64)


@pytest.mark.parametrize("ws_kind", ["per_channel", "scalar"])
def test_int8_linear_config1_3d(gpu_device, ws_kind):
    """C1 (M=4096, K=1536, N=8960, bias, G=128) as a [2, 2048, 1536] activation."""
    print(f"[integration linear] C1 3-D ws={ws_kind}", flush=True)
    x = inputs.activation(4096, 1536, 0)
    w, ws, bias = inputs.weights(8960, 1536, 0)
    if ws_kind == "scalar":
        ws = torch.tensor(3.0e-3)
    bias16 = bias.to(torch.bfloat16)  # a bf16 bias, as a ComfyUI checkpoint holds it
    out = integration.int8_linear(x.view(2, 2048, 1536).to(gpu_device), w.to(gpu_device), ws.to(gpu_device),
                                  bias16.to(gpu_device), convrot=True, convrot_groupsize=128)
    torch.cuda.synchronize(gpu_device)
    assert out.shape == (2, 2048, 8960) and out.dtype == torch.bfloat16
    rows = _rows(4096, 192, 1)
    ws_full = ws.expand(8960) if ws.numel() == 1 else ws
    ref = _oracle_linear(x, rows, w, ws_full, bias16, 128, oracle.ACT_NONE)
    got = inputs.bits(out.reshape(4096, 8960)[torch.from_numpy(rows).to(gpu_device)])
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"{len(bad)} outputs differ, first {bad[:5].tolist()}"


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_int8_linear_out_dtype_and_group_256(gpu_device, out_dtype):
    """out_dtype=float16 / float32: the epilogue's fp32 value rounded once to
    fp16 (no bf16 step), or kept in fp32; G=256 is the reference's own group
    (its default)."""
    print(f"[integration linear] out {out_dtype}, G=256", flush=True)
    x = inputs.activation(384, 1536, 5)
    w, ws, bias = inputs.weights(1024, 1536, 5)
    out = integration.int8_linear(x.view(3, 128, 1536).to(gpu_device), w.to(gpu_device), ws.to(gpu_device),
                                  bias.to(gpu_device), out_dtype=out_dtype, convrot=True)
    torch.cuda.synchronize(gpu_device)
    assert out.shape == (3, 128, 1024) and out.dtype == out_dtype
    q, s = oracle.convrot_quant(inputs.bits(x), 256)
    acc = oracle.int8_gemm_i32(q, w.numpy())
    got = out.reshape(384, 1024).cpu()
    if out_dtype == torch.float16:
        ref = oracle.epilogue_f16(acc, s, ws.numpy(), bias.numpy())
        np.testing.assert_array_equal(got.view(torch.int16).numpy().view(np.uint16), ref)
        # one rounding, not two: some values differ from the bf16 output cast to fp16
        via_bf16 = inputs.from_bits(oracle.epilogue_bf16(acc, s, ws.numpy(), bias.numpy())).to(torch.float16)
        assert not torch.equal(got, via_bf16)
    else:
        ref = oracle.epilogue_f32(acc, s, ws.numpy(), bias.numpy())
        np.testing.assert_array_equal(got.numpy().view(np.uint32), ref.view(np.uint32))


def test_int8_linear_ffn_down_gelu(gpu_device):
    """C4 FFN-down slice with the tanh-GELU folded into the quantizer
    (input_act="gelu_tanh": K=13824, N=5120, no bias)."""
    print("[integration linear] C4 ffn-down slice, gelu_tanh", flush=True)
    x = inputs.activation(512, 13824, 3)
    w, ws, _ = inputs.weights(5120, 13824, 3, with_bias=False)
    out = integration.int8_linear(x.view(1, 512, 13824).to(gpu_device), w.to(gpu_device), ws.to(gpu_device),
                                  convrot=True, convrot_groupsize=128, input_act="gelu_tanh")
    torch.cuda.synchronize(gpu_device)
    rows = _rows(512, 40, 3)
    ref = _oracle_linear(x, rows, w, ws, None, 128, oracle.ACT_GELU_TANH)
    got = inputs.bits(out.reshape(512, 5120)[torch.from_numpy(rows).to(gpu_device)])
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("act_name,act", [("swiglu", oracle.ACT_SWIGLU), ("none", oracle.ACT_NONE)])
def test_int8_linear_input_act(gpu_device, act_name, act):
    print(f"[integration linear] input_act={act_name}", flush=True)
    k = 1536
    x = inputs.activation(256, 2 * k if act == oracle.ACT_SWIGLU else k, 9)
    w, ws, bias = inputs.weights(2048, k, 9)
    out = integration.int8_linear(x.view(4, 64, -1).to(gpu_device), w.to(gpu_device), ws.to(gpu_device),
                                  bias.to(gpu_device), convrot=True, convrot_groupsize=128, input_act=act_name)
    torch.cuda.synchronize(gpu_device)
    assert out.shape == (4, 64, 2048)
    rows = np.arange(256, dtype=np.int64)
    ref = _oracle_linear(x, rows, w, ws, bias, 128, act)
    np.testing.assert_array_equal(inputs.bits(out.reshape(256, 2048)), ref)


# ---------------------------------------------------------------------------
# attention override
# ---------------------------------------------------------------------------
def _oracle_attention(q_hnd: torch.Tensor, k_hnd: torch.Tensor, v_hnd: torch.Tensor, rows: np.ndarray,
                      sm_scale: float, causal: bool = False) -> np.ndarray:
    """The Sage path's math (K smoothing, 128-token Q/K blocks, bf16 P) on
    bf16 HND inputs, padded to 128 channels as the kernel sees them (zero
    channels change neither the codes nor the result)."""
    d = q_hnd.size(-1)
    pad = 128 - d
    qp, kp, vp = (torch.nn.functional.pad(t, (0, pad)) if pad else t for t in (q_hnd, k_hnd, v_hnd))
    qp, kp, vp = (t.contiguous() for t in (qp, kp, vp))
    mean = oracle.sage_kmean(inputs.bits(kp))
    q8, qs = oracle.sage_quant(inputs.bits(qp), 128)
    k8, ks = oracle.sage_quant(inputs.bits(kp), 128, mean)
    return oracle.sage_attn_rows(q8, qs, 128, k8, ks, 128, inputs.bits(vp), sm_scale, rows, causal)[:, :d]


def _check(got: torch.Tensor, ref: np.ndarray):
    res = attention_error_metrics(got.float().cpu(), torch.from_numpy(ref), candidate_name="override",
                                  reference_name="oracle")
    print(f"  cos={res.cosine:.6f} max_abs={res.max_abs:.3e}", flush=True)
    require_attention_correctness(res, **GATE)


def _sample(b, h, l, n, seed):
    rng = np.random.default_rng(seed)
    rows = np.stack([rng.integers(0, b, n), rng.integers(0, h, n), rng.integers(0, l, n)], 1)
    rows[0, 2], rows[1, 2] = 0, l - 1
    return rows.astype(np.int64)


def _not_called(*args, **kwargs):
    raise AssertionError("the override fell back for a call Sage serves")


def test_override_nhd_40_heads(gpu_device):
    """ComfyUI's optimized_attention form: q/k/v [B, L, H*D] with 40 heads of
    128 (the Wan-14B head layout); output [B, L, H*D] bf16."""
    print("[integration attn] NHD 3-D, 40 heads", flush=True)
    b, h, l, d = 1, 40, 300, 128
    q, k, v = inputs.attention(b, h, l, d, 31)  # HND
    to_nhd = lambda t: t.transpose(1, 2).reshape(b, l, h * d).contiguous()  # noqa: E731
    out = integration.sage_attention_override(_not_called, to_nhd(q).to(gpu_device), to_nhd(k).to(gpu_device),
                                              to_nhd(v).to(gpu_device), h)
    torch.cuda.synchronize(gpu_device)
    assert out.shape == (b, l, h * d) and out.dtype == torch.bfloat16
    rows = _sample(b, h, l, 96, 31)
    ref = _oracle_attention(q, k, v, rows, d ** -0.5)
    got = out.view(b, l, h, d)[torch.from_numpy(rows[:, 0]), torch.from_numpy(rows[:, 2]), torch.from_numpy(rows[:, 1])]
    _check(got, ref)


@pytest.mark.parametrize("skip_output_reshape", [False, True])
def test_override_gqa_fp32_nhd(gpu_device, skip_output_reshape):
    """enable_gqa with 8 query heads over 2 KV heads of 64 channels, fp32
    inputs (cast to bf16 at the boundary, output cast back to fp32)."""
    print(f"[integration attn] GQA fp32 NHD skip_output_reshape={skip_output_reshape}", flush=True)
    b, h, hkv, lq, lk, d = 2, 8, 2, 257, 300, 64
    g = torch.Generator().manual_seed(41)
    q = torch.randn(b, lq, h * d, generator=g)
    k = torch.randn(b, lk, hkv * d, generator=g) + torch.randn(b, 1, hkv * d, generator=g) * 2
    v = torch.randn(b, lk, hkv * d, generator=g)
    out = integration.sage_attention_override(_not_called, q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), h,
                                              enable_gqa=True, skip_output_reshape=skip_output_reshape)
    torch.cuda.synchronize(gpu_device)
    assert out.dtype == torch.float32
    hnd = lambda t, heads, l: t.to(torch.bfloat16).view(b, l, heads, d).transpose(1, 2)  # noqa: E731
    qh, kh, vh = hnd(q, h, lq), hnd(k, hkv, lk), hnd(v, hkv, lk)
    kh, vh = kh.repeat_interleave(h // hkv, dim=1), vh.repeat_interleave(h // hkv, dim=1)
    rows = _sample(b, h, lq, 96, 41)
    ref = _oracle_attention(qh, kh, vh, rows, d ** -0.5)
    if skip_output_reshape:
        assert out.shape == (b, h, lq, d)
        got = out[torch.from_numpy(rows[:, 0]), torch.from_numpy(rows[:, 1]), torch.from_numpy(rows[:, 2])]
    else:
        assert out.shape == (b, lq, h * d)
        got = out.view(b, lq, h, d)[torch.from_numpy(rows[:, 0]), torch.from_numpy(rows[:, 2]),
                                    torch.from_numpy(rows[:, 1])]
    _check(got, ref)


@pytest.mark.parametrize("skip_output_reshape", [False, True])
def test_override_skip_reshape_hnd(gpu_device, skip_output_reshape):
    print(f"[integration attn] HND skip_reshape skip_output_reshape={skip_output_reshape}", flush=True)
    b, h, l, d = 1, 4, 200, 128
    q, k, v = inputs.attention(b, h, l, d, 51)
    out = integration.sage_attention_override(_not_called, q.to(gpu_device), k.to(gpu_device), v.to(gpu_device), h,
                                              skip_reshape=True, skip_output_reshape=skip_output_reshape)
    torch.cuda.synchronize(gpu_device)
    rows = _sample(b, h, l, 64, 51)
    ref = _oracle_attention(q, k, v, rows, d ** -0.5)
    if skip_output_reshape:
        assert out.shape == (b, h, l, d)
        got = out[torch.from_numpy(rows[:, 0]), torch.from_numpy(rows[:, 1]), torch.from_numpy(rows[:, 2])]
    else:
        assert out.shape == (b, l, h * d)
        got = out.view(b, l, h, d)[torch.from_numpy(rows[:, 0]), torch.from_numpy(rows[:, 2]),
                                   torch.from_numpy(rows[:, 1])]
    _check(got, ref)


def test_override_scale_and_causal(gpu_device):
    """The caller's ``scale`` and ``is_causal`` keywords reach the kernel
    (stable.py:684-700)."""
    print("[integration attn] scale=0.05, is_causal", flush=True)
    b, h, l, d = 1, 4, 333, 128
    q, k, v = inputs.attention(b, h, l, d, 61)
    to_nhd = lambda t: t.transpose(1, 2).reshape(b, l, h * d).contiguous()  # noqa: E731
    out = integration.sage_attention_override(_not_called, to_nhd(q).to(gpu_device), to_nhd(k).to(gpu_device),
                                              to_nhd(v).to(gpu_device), h, scale=0.05, is_causal=True)
    torch.cuda.synchronize(gpu_device)
    rows = _sample(b, h, l, 96, 61)
    ref = _oracle_attention(q, k, v, rows, 0.05, causal=True)
    got = out.view(b, l, h, d)[torch.from_numpy(rows[:, 0]), torch.from_numpy(rows[:, 2]), torch.from_numpy(rows[:, 1])]
    _check(got, ref)


@pytest.mark.parametrize("stabilize", [True, False])
def test_w8a8_override_nhd(gpu_device, stabilize):
    """``turing_w8a8_attention`` (the loader default): NHD 3-D inputs with the
    tuning read from ``transformer_options``, against the oracle's W8A8 rows
    (rotated Q/K, K anchor, per-channel V, u8 P)."""
    print(f"[integration attn] w8a8 NHD stabilize_k={stabilize}", flush=True)
    b, h, l, d = 1, 8, 300, 128
    q, k, v = inputs.attention(b, h, l, d, 71)
    to_nhd = lambda t: t.transpose(1, 2).reshape(b, l, h * d).contiguous()  # noqa: E731
    opts = {integration.ATTENTION_TUNING_KEY: {"rotate_qk": True, "stabilize_k": stabilize}}
    out = integration.w8a8_attention_override(_not_called, to_nhd(q).to(gpu_device), to_nhd(k).to(gpu_device),
                                              to_nhd(v).to(gpu_device), h, transformer_options=opts)
    torch.cuda.synchronize(gpu_device)
    assert out.shape == (b, l, h * d) and out.dtype == torch.bfloat16
    rows = _sample(b, h, l, 96, 71)
    q8, qs, k8, ks, _ = oracle.w8a8_quant_qk(inputs.bits(q), inputs.bits(k), oracle.DTYPE_BF16, True, stabilize)
    v8, vs = oracle.w8a8_quant_v(inputs.bits(v), oracle.DTYPE_BF16)
    ref = oracle.w8a8_attn_rows(q8, qs, k8, ks, v8, vs, l, d ** -0.5, rows, False)
    got = out.view(b, l, h, d)[torch.from_numpy(rows[:, 0]), torch.from_numpy(rows[:, 2]), torch.from_numpy(rows[:, 1])]
    _check(got, ref)


def _fallback_cases(dev):
    b, l, h, d = 1, 64, 2, 64
    x = torch.randn(b, l, h * d, device=dev).to(torch.bfloat16)
    wide = torch.randn(b, l, h * 160, device=dev).to(torch.bfloat16)
    strided = torch.randn(b, l, h * d * 2, device=dev).to(torch.bfloat16)[..., ::2]
    return {
        "mask": ((x, x, x), dict(mask=torch.zeros(l, l, device=dev))),
        "low_precision_off": ((x, x, x), dict(low_precision_attention=False)),
        "dtype_mismatch": ((x, x.half(), x), {}),
        "head_dim_160": ((wide, wide, wide), {}),
        "channels_not_contiguous": ((strided, strided, strided), {}),
        "cpu_tensors": ((x.cpu(), x.cpu(), x.cpu()), {}),
        "empty_sequence": ((x[:, :0], x[:, :0], x[:, :0]), {}),
    }


@pytest.mark.parametrize("case", ["mask", "low_precision_off", "dtype_mismatch", "head_dim_160",
                                  "channels_not_contiguous", "cpu_tensors", "empty_sequence"])
def test_override_fallbacks_return_the_callers_result(gpu_device, case):
    """Calls Sage cannot serve reach ``original`` with every argument unchanged,
    and its result is returned as is (stable.py:83-165's fallback contract)."""
    print(f"[integration attn] fallback {case}", flush=True)
    (q, k, v), extra = _fallback_cases(gpu_device)[case]
    heads = 2
    sentinel = torch.empty(1)
    seen = []

    def original(q_, k_, v_, heads_, **kwargs):
        seen.append((q_, k_, v_, heads_, kwargs))
        return sentinel

    out = integration.sage_attention_override(original, q, k, v, heads, **extra)
    assert out is sentinel
    assert len(seen) == 1
    q_, k_, v_, heads_, kwargs = seen[0]
    assert q_ is q and k_ is k and v_ is v and heads_ == heads
    for key, value in extra.items():
        assert kwargs[key] is value
