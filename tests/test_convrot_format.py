"""ConvRot checkpoint metadata and W8 loading (CPU, no kernel launches).

The classification cases follow the reference's own metadata tests
(tests/test_convrot_nodes.py:49-325, :376-486: legacy W8 normalisation,
rejections, conflicting duplicates, header vs tensor metadata, prefixes),
restated against this package's functions; the file cases write real
safetensors files and read them back.
"""
from __future__ import annotations

import json
import struct

import pytest
import torch

from comfyui_turing_utils_kernel import convrot_format as cf
from comfyui_turing_utils_kernel.wan_block import (W8A8Linear, WanBlockConfig, WanBlockW8A8, block_state,
                                                   load_block, load_text_embedding)


def w8(**extra):
    return {"format": "int8_tensorwise", "convrot": True, **extra}


# -- classification ------------------------------------------------------------

def test_w8_and_w4_kinds():
    assert cf.classify_config(w8(), "l", False) == ("w8", "int8")
    assert cf.classify_config({"format": "convrot_w4a4"}, "l", False) == ("w4", "int4")
    assert cf.classify_config({"format": "convrot_w4a4", "linear_dtype": "int8"}, "l", False) == ("w4", "int8")
    assert cf.classify_config({"format": "convrot_w4a4"}, "l", True) == ("w4", "int8")
    assert cf.classify_config({"format": "asym_w4a8_int8", "params": {"group_size": 32}}, "l", False) == \
        ("w4_codebook", "int8")


def test_params_object_is_consulted_after_the_top_level():
    assert cf.classify_config({"format": "int8_tensorwise", "params": {"convrot": True}}, "l", False) == ("w8", "int8")
    assert cf.classify_config({"format": "int8_tensorwise", "convrot": False, "params": {"convrot": True}},
                              "l", False) is None
    with pytest.raises(ValueError, match="non-object params"):
        cf.classify_config({"format": "int8_tensorwise", "params": [1]}, "l", False)


@pytest.mark.parametrize("fmt", [None, "int8_rowwise"])
def test_legacy_w8_is_normalised(fmt):
    config = {"convrot": True, "per_row": True}
    if fmt:
        config["format"] = fmt
    assert cf.classify_config(config, "l", False) == ("w8", "int8")
    assert config["format"] == "int8_tensorwise"


def test_legacy_w8_requires_per_row():
    with pytest.raises(ValueError, match="unsupported weight format"):
        cf.classify_config({"format": "int8_rowwise", "convrot": True}, "l", False)


def test_rejections():
    assert cf.classify_config({"format": "int8_tensorwise"}, "l", False) is None  # not ConvRot
    with pytest.raises(ValueError, match="non-boolean convrot"):
        cf.classify_config({"format": "int8_tensorwise", "convrot": 1}, "l", False)
    with pytest.raises(ValueError, match="unsupported weight format"):
        cf.classify_config({"format": "fp8_e4m3", "convrot": True}, "l", False)
    with pytest.raises(ValueError, match="INT8 activations only"):
        cf.classify_config(w8(linear_dtype="int4"), "l", False)
    assert cf.classify_config(w8(linear_dtype="int4"), "l", True) == ("w8", "int8")
    with pytest.raises(ValueError, match="unsupported linear_dtype"):
        cf.classify_config(w8(linear_dtype="fp8"), "l", True)
    with pytest.raises(ValueError, match="unsupported linear_dtype"):
        cf.classify_config({"format": "convrot_w4a4", "linear_dtype": "int2"}, "l", False)
    with pytest.raises(ValueError, match="must declare convrot=true"):
        cf.classify_config({"format": "asym_w4a8_int8", "convrot": False}, "l", False)
    with pytest.raises(ValueError, match="invalid group_size"):
        cf.classify_config({"format": "asym_w4a8_int8", "group_size": True}, "l", False)
    with pytest.raises(ValueError, match="convrot_groupsize=256"):
        cf.classify_config({"format": "asym_w4a8_int8", "convrot_groupsize": 128}, "l", False)
    with pytest.raises(ValueError, match="must be an object"):
        cf.classify_config([], "l", False)


def test_conflicting_duplicates_and_force_flag():
    recs = [("a", w8()), ("a", {"format": "convrot_w4a4"})]
    with pytest.raises(ValueError, match="Conflicting ConvRot metadata"):
        cf.classify_layers(recs)
    assert set(cf.classify_layers([("a", w8()), ("a", w8())])) == {"a"}
    with pytest.raises(ValueError, match="force_int8_gemm must be boolean"):
        cf.classify_layers([], force_int8_gemm="yes")
    summary = cf.summarize(cf.classify_layers([("a", w8()), ("b", {"format": "convrot_w4a4"}), ("c", {})]))
    assert summary == cf.ConvRotSummary(w4a4=1, w8a8=1)


def test_quant_tensor_round_trip():
    config = w8(convrot_groupsize=128)
    assert cf.decode_quant_tensor(cf.encode_quant_tensor(config), "k") == config
    with pytest.raises(ValueError, match="invalid quantization JSON"):
        cf.decode_quant_tensor(torch.tensor([123, 34], dtype=torch.uint8), "k")
    with pytest.raises(ValueError, match="must be an object"):
        cf.decode_quant_tensor(cf.encode_quant_tensor([1]), "k")  # type: ignore[arg-type]


# -- files ---------------------------------------------------------------------

def _linear(n, k, group=128, per_row=True, bias=True, seed=0):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    scale = torch.rand(n, generator=g) * 1e-3 + 1e-4 if per_row else torch.full((n,), 2e-3)
    b = torch.randn(n, generator=g) if bias else None
    return W8A8Linear(codes, scale, b, group)


def _same(a: W8A8Linear, b: W8A8Linear):
    assert torch.equal(a.weight, b.weight) and torch.equal(a.weight_scale, b.weight_scale) and a.group == b.group
    assert (a.bias is None) == (b.bias is None) and (a.bias is None or torch.equal(a.bias, b.bias))


@pytest.mark.parametrize("header", [False, True])
def test_save_load_round_trip(tmp_path, header):
    layers = {"m.a": _linear(64, 256, 128, True, True, 1), "m.b": _linear(32, 512, 256, False, False, 2),
              "other.c": _linear(16, 128, 128, True, True, 3)}
    path = tmp_path / "w.safetensors"
    cf.save_w8a8_linears(path, layers, {"m.norm": torch.ones(4)}, header_metadata=header)
    got = cf.load_w8a8_linears(path)
    assert set(got) == set(layers)
    for name in layers:
        _same(got[name], layers[name])
    assert set(cf.load_w8a8_linears(path, prefix="m.")) == {"m.a", "m.b"}
    assert cf.convrot_skip_reason(path) is None
    # a tensor-wise scale is stored as one value and widened on load
    from safetensors import safe_open
    with safe_open(str(path), framework="pt") as f:
        assert f.get_tensor("m.b.weight_scale").shape == ()
        assert f.get_tensor("m.a.weight_scale").shape == (64,)


def test_non_convrot_and_broken_files(tmp_path):
    from safetensors.torch import save_file

    plain = tmp_path / "plain.safetensors"
    save_file({"w": torch.zeros(2, 2)}, str(plain))
    assert "does not contain supported ConvRot" in cf.convrot_skip_reason(plain)
    with pytest.raises(ValueError, match="does not contain supported ConvRot"):
        cf.load_w8a8_linears(plain)
    assert "unsupported file extension" in cf.convrot_skip_reason(tmp_path / "x.ckpt")
    short = tmp_path / "short.safetensors"
    short.write_bytes(b"\x01\x02")
    assert "too short" in cf.convrot_skip_reason(short)
    huge = tmp_path / "huge.safetensors"
    huge.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    assert "invalid safetensors header size" in cf.convrot_skip_reason(huge)
    past = tmp_path / "past.safetensors"
    past.write_bytes(struct.pack("<Q", 100) + b"{}")
    assert "beyond file size" in cf.convrot_skip_reason(past)
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(struct.pack("<Q", 2) + b"{x")
    with pytest.raises(ValueError, match="invalid JSON"):
        cf.read_safetensors_header(bad)
    arr = tmp_path / "arr.safetensors"
    arr.write_bytes(struct.pack("<Q", 2) + b"[]")
    with pytest.raises(ValueError, match="must be an object"):
        cf.read_safetensors_header(arr)


def _write_raw(path, header: dict, data: bytes):
    text = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(text)) + text + data)


def test_quant_tensor_descriptor_checks(tmp_path):
    good = json.dumps(w8()).encode()
    cases = {
        "dtype": ({"dtype": "I8", "shape": [len(good)], "data_offsets": [0, len(good)]}, "must use U8"),
        "shape": ({"dtype": "U8", "shape": [len(good) + 1], "data_offsets": [0, len(good)]}, "does not match"),
        "offsets": ({"dtype": "U8", "shape": [len(good)], "data_offsets": [0, True]}, "invalid shape or data"),
        "outside": ({"dtype": "U8", "shape": [len(good) + 9], "data_offsets": [0, len(good) + 9]}, "outside"),
    }
    for name, (info, message) in cases.items():
        path = tmp_path / f"{name}.safetensors"
        _write_raw(path, {"l.comfy_quant": info}, good)
        with pytest.raises(ValueError, match=message):
            cf.layer_configs(path)
    path = tmp_path / "json.safetensors"
    _write_raw(path, {"l.comfy_quant": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}}, b"{x")
    with pytest.raises(ValueError, match="invalid quantization JSON"):
        cf.layer_configs(path)
    path = tmp_path / "meta.safetensors"
    _write_raw(path, {"__metadata__": {"_quantization_metadata": json.dumps({"layers": []})}}, b"")
    with pytest.raises(ValueError, match="layers object"):
        cf.layer_configs(path)


def test_w8_layer_without_tensors_is_refused(tmp_path):
    from safetensors.torch import save_file

    path = tmp_path / "m.safetensors"
    save_file({"l.comfy_quant": cf.encode_quant_tensor(w8()), "l.weight": torch.zeros(4, 128, dtype=torch.int8)},
              str(path))
    with pytest.raises(ValueError, match="l.weight_scale"):
        cf.load_w8a8_linears(path)
    save_file({"l.comfy_quant": cf.encode_quant_tensor(w8(convrot_groupsize=64)),
               "l.weight": torch.zeros(4, 128, dtype=torch.int8), "l.weight_scale": torch.ones(())}, str(path))
    with pytest.raises(ValueError, match="convrot_groupsize"):
        cf.load_w8a8_linears(path)


def test_concat_split_inverse():
    parts = [_linear(32, 256, seed=i) for i in range(3)]
    fused = W8A8Linear.concat(parts)
    assert fused.out_features == 96
    for a, b in zip(fused.split(3), parts):
        _same(a, b)
    with pytest.raises(ValueError, match="one K"):
        W8A8Linear.concat([_linear(8, 256), _linear(8, 128)])
    with pytest.raises(ValueError, match="bias"):
        W8A8Linear.concat([_linear(8, 256), _linear(8, 256, bias=False)])


def test_wan_block_checkpoint_round_trip(tmp_path):
    """A block written under Wan's parameter names (q / k / v as separate
    layers) loads back with the same fused weights."""
    c, f = 256, 512
    cfg = WanBlockConfig(dim=c, heads=2, ffn_dim=f, text_dim=128)
    g = torch.Generator().manual_seed(3)
    block = WanBlockW8A8(
        cfg, modulation=torch.randn(1, 6, c, generator=g),
        self_qkv=_linear(3 * c, c, seed=1), self_o=_linear(c, c, seed=2),
        self_norm_q=torch.rand(c, generator=g) + 0.5, self_norm_k=torch.rand(c, generator=g) + 0.5,
        norm3_weight=torch.randn(c, generator=g) * 0.5 + 1, norm3_bias=torch.randn(c, generator=g),
        cross_q=_linear(c, c, seed=4), cross_kv=_linear(2 * c, c, seed=5), cross_o=_linear(c, c, seed=6),
        cross_norm_q=torch.rand(c, generator=g) + 0.5, cross_norm_k=torch.rand(c, generator=g) + 0.5,
        ffn_up=_linear(f, c, seed=7), ffn_down=_linear(c, f, 256, seed=8))
    linears, tensors = block_state(block, 7, prefix="model.diffusion_model.")
    linears["model.diffusion_model.text_embedding.0"] = _linear(c, 128, seed=9)
    linears["model.diffusion_model.text_embedding.2"] = _linear(c, c, seed=10)
    path = tmp_path / "wan.safetensors"
    cf.save_w8a8_linears(path, linears, tensors)
    got = load_block(path, 7, cfg, prefix="model.diffusion_model.")
    for name in ("self_qkv", "self_o", "cross_q", "cross_kv", "cross_o", "ffn_up", "ffn_down"):
        _same(getattr(got, name), getattr(block, name))
    for name in ("modulation", "self_norm_q", "self_norm_k", "cross_norm_q", "cross_norm_k", "norm3_weight",
                 "norm3_bias"):
        assert torch.equal(getattr(got, name), getattr(block, name)), name
    text = load_text_embedding(path, prefix="model.diffusion_model.")
    _same(text.fc1, linears["model.diffusion_model.text_embedding.0"])
    with pytest.raises(ValueError, match="does not contain"):
        load_block(path, 3, cfg, prefix="model.diffusion_model.")
