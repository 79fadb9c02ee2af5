"""ConvRot checkpoints: the per-layer quantization metadata of a safetensors
file, and loading its W8A8 layers for this package's INT8 path.

Format (as the reference validates it, comfyui_turing_utils/quantization/
convrot.py:71-145, :163-245, :294-371).  A quantized layer ``name`` carries a
JSON object either in a U8 tensor ``name.comfy_quant`` or under
``layers[name]`` of the header's ``__metadata__._quantization_metadata``
string.  Keys are looked up on the object first, then under its ``params``
object.  Classification:
  * ``format == "convrot_w4a4"`` -> W4 (activations ``linear_dtype`` int4 or
    int8);
  * ``format == "asym_w4a8_int8"`` -> grouped-codebook W4A8 (must be
    ConvRot, ``group_size`` >= 4, ``convrot_groupsize`` 256);
  * otherwise ``convrot`` (default false) must be a boolean; false -> not a
    ConvRot layer; true -> the format must be ``"int8_tensorwise"``, with
    ``linear_dtype`` int8 (int4 only when INT8 GEMMs are forced).
  * Legacy W8 metadata -- no format or ``"int8_rowwise"``, with convrot and
    ``per_row`` true -- is read as ``"int8_tensorwise"``.
  A layer described twice must classify the same way both times.

W8 layers store ``name.weight`` (int8 [N, K], already ConvRot-rotated along
K), ``name.weight_scale`` (fp32, one value, or one per output channel for the
legacy per-row layout) and optionally ``name.bias``; the rotation group is
``convrot_groupsize`` (256 when absent).  Only W8 layers run on this path;
W4 and codebook layers are classified but not loaded.

Reading never unpickles: the header is parsed as JSON with size limits and
tensors come through ``safetensors.safe_open``.
"""
from __future__ import annotations

import dataclasses
import json
import math
import struct
from pathlib import Path
from typing import Optional

import torch

W4_FORMAT = "convrot_w4a4"
CODEBOOK_W4_FORMAT = "asym_w4a8_int8"
W8_FORMAT = "int8_tensorwise"
LEGACY_W8_FORMAT = "int8_rowwise"
MAX_SAFETENSORS_HEADER_SIZE = 128 * 1024 * 1024
MAX_QUANT_CONFIG_SIZE = 1024 * 1024
QUANT_SUFFIX = ".comfy_quant"
DEFAULT_W8_GROUP = 256


@dataclasses.dataclass(frozen=True)
class ConvRotSummary:
    w4a4: int = 0
    w4a8: int = 0
    codebook_w4a8: int = 0
    w8a8: int = 0


def _lookup(config: dict, name: str, default):
    """``config[name]``, else ``config["params"][name]``, else ``default``."""
    if name in config:
        return config[name]
    params = config.get("params", {})
    return params.get(name, default)


def _check_params(config: dict, layer: str) -> None:
    if not isinstance(config.get("params", {}), dict):
        raise ValueError(f"ConvRot layer {layer} has non-object params metadata")


def _strict_int(value) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def classify_config(config: dict, layer: str, force_int8_gemm: bool) -> Optional[tuple[str, str]]:
    """(weight kind, activation dtype) of one layer's metadata, or None when
    it is not a ConvRot layer; raises ValueError on metadata the reference
    refuses.  Legacy W8 metadata is rewritten in place to the current format."""
    if not isinstance(config, dict):
        raise ValueError(f"Quantization metadata for layer {layer} must be an object")
    _check_params(config, layer)
    fmt = config.get("format")
    if (fmt is None or fmt == LEGACY_W8_FORMAT) and _lookup(config, "convrot", False) is True \
            and _lookup(config, "per_row", False) is True:
        config["format"] = fmt = W8_FORMAT

    if fmt == W4_FORMAT:
        act = _lookup(config, "linear_dtype", "int4")
        if act not in ("int4", "int8"):
            raise ValueError(f"ConvRot W4 layer {layer} declares unsupported linear_dtype={act!r}; "
                             "expected 'int4' or 'int8'")
        return "w4", ("int8" if force_int8_gemm else act)

    if fmt == CODEBOOK_W4_FORMAT:
        if _lookup(config, "convrot", True) is not True:
            raise ValueError(f"Grouped-codebook W4A8 layer {layer} must declare convrot=true")
        group = _lookup(config, "group_size", 16)
        if not _strict_int(group) or group < 4:
            raise ValueError(f"Grouped-codebook W4A8 layer {layer} has invalid group_size={group!r}")
        if _lookup(config, "convrot_groupsize", 256) != 256:
            raise ValueError(f"Grouped-codebook W4A8 layer {layer} requires convrot_groupsize=256")
        return "w4_codebook", "int8"

    convrot = _lookup(config, "convrot", False)
    if not isinstance(convrot, bool):
        raise ValueError(f"Quantized layer {layer} has non-boolean convrot={convrot!r}")
    if not convrot:
        return None
    if fmt != W8_FORMAT:
        raise ValueError(f"ConvRot layer {layer} uses unsupported weight format {fmt!r}")
    act = _lookup(config, "linear_dtype", "int8")
    if act not in ("int4", "int8"):
        raise ValueError(f"ConvRot W8 layer {layer} declares unsupported linear_dtype={act!r}; expected 'int8'")
    if act != "int8" and not force_int8_gemm:
        raise ValueError(f"ConvRot W8 layer {layer} cannot use linear_dtype={act!r}; "
                         "W8 ConvRot supports INT8 activations only")
    return "w8", "int8"


def decode_quant_tensor(value: torch.Tensor, key: str) -> dict:
    """The JSON object held by a U8 ``.comfy_quant`` tensor."""
    if not isinstance(value, torch.Tensor):
        raise TypeError(f"{key} must be a JSON byte tensor")
    try:
        config = json.loads(value.detach().cpu().to(torch.uint8).numpy().tobytes())
    except (UnicodeDecodeError, json.JSONDecodeError) as exc:
        raise ValueError(f"{key} contains invalid quantization JSON") from exc
    if not isinstance(config, dict):
        raise ValueError(f"{key} quantization JSON must be an object")
    return config


def encode_quant_tensor(config: dict) -> torch.Tensor:
    return torch.frombuffer(bytearray(json.dumps(config).encode("utf-8")), dtype=torch.uint8).clone()


def read_safetensors_header(path) -> tuple[dict, int, int]:
    """(header JSON, first data byte, file size), with the size limits the
    reference applies before trusting a file."""
    path = Path(path)
    size = path.stat().st_size
    with path.open("rb") as handle:
        raw = handle.read(8)
        if len(raw) != 8:
            raise ValueError("file is too short to contain a safetensors header")
        (header_size,) = struct.unpack("<Q", raw)
        if header_size == 0 or header_size > MAX_SAFETENSORS_HEADER_SIZE:
            raise ValueError(f"invalid safetensors header size {header_size}")
        data_start = 8 + header_size
        if data_start > size:
            raise ValueError(f"safetensors header ends at byte {data_start}, beyond file size {size}")
        text = handle.read(header_size)
    try:
        header = json.loads(text)
    except (UnicodeDecodeError, json.JSONDecodeError) as exc:
        raise ValueError("safetensors header contains invalid JSON") from exc
    if not isinstance(header, dict):
        raise ValueError("safetensors header must be an object")
    return header, data_start, size


def read_quant_config(handle, info: dict, key: str, data_start: int, file_size: int) -> dict:
    """A ``.comfy_quant`` tensor's JSON read straight from the file, after
    checking its descriptor (U8, consistent shape and offsets, size cap)."""
    if not isinstance(info, dict):
        raise ValueError(f"{key} has an invalid safetensors tensor descriptor")
    if info.get("dtype") != "U8":
        raise ValueError(f"{key} must use U8 storage")
    shape, offsets = info.get("shape"), info.get("data_offsets")
    if (not isinstance(shape, list) or any(not _strict_int(d) or d < 0 for d in shape)
            or not isinstance(offsets, list) or len(offsets) != 2 or any(not _strict_int(o) for o in offsets)):
        raise ValueError(f"{key} has invalid shape or data offsets")
    begin, end = offsets
    length = end - begin
    if length != math.prod(shape):
        raise ValueError(f"{key} byte length does not match its U8 shape")
    if length > MAX_QUANT_CONFIG_SIZE:
        raise ValueError(f"{key} is too large to be quantization JSON")
    if begin < 0 or end < begin or data_start + end > file_size:
        raise ValueError(f"{key} data offsets are outside the safetensors file")
    handle.seek(data_start + begin)
    raw = handle.read(length)
    if len(raw) != length:
        raise ValueError(f"{key} tensor data is truncated")
    try:
        config = json.loads(raw)
    except (UnicodeDecodeError, json.JSONDecodeError) as exc:
        raise ValueError(f"{key} contains invalid quantization JSON") from exc
    if not isinstance(config, dict):
        raise ValueError(f"{key} quantization JSON must be an object")
    return config


def _header_layers(metadata: dict) -> Optional[dict]:
    raw = metadata.get("_quantization_metadata")
    if raw is None:
        return None
    try:
        parsed = json.loads(raw)
    except (TypeError, json.JSONDecodeError) as exc:
        raise ValueError("Safetensors _quantization_metadata contains invalid JSON") from exc
    if not isinstance(parsed, dict) or not isinstance(parsed.get("layers"), dict):
        raise ValueError("Safetensors _quantization_metadata must contain a layers object")
    return parsed


def layer_configs(path, prefix: Optional[str] = None) -> list[tuple[str, dict]]:
    """Every (layer, metadata) record of a file, header records first, then
    ``.comfy_quant`` tensors in header order; ``prefix`` keeps layers whose
    name starts with it."""
    header, data_start, size = read_safetensors_header(path)
    metadata = header.get("__metadata__", {})
    if not isinstance(metadata, dict):
        raise ValueError("safetensors __metadata__ must be an object")
    records = []
    parsed = _header_layers(metadata)
    if parsed is not None:
        records += [(n, c) for n, c in parsed["layers"].items() if prefix is None or n.startswith(prefix)]
    with Path(path).open("rb") as handle:
        for key, info in header.items():
            if key == "__metadata__" or not key.endswith(QUANT_SUFFIX):
                continue
            layer = key[: -len(QUANT_SUFFIX)]
            if prefix is not None and not layer.startswith(prefix):
                continue
            records.append((layer, read_quant_config(handle, info, key, data_start, size)))
    return records


def classify_layers(records, force_int8_gemm: bool = False) -> dict[str, tuple[str, str, dict]]:
    """layer -> (weight kind, activation dtype, metadata) for the ConvRot
    layers; a layer described twice must classify identically."""
    if not isinstance(force_int8_gemm, bool):
        raise ValueError(f"force_int8_gemm must be boolean, got {force_int8_gemm!r}")
    out: dict[str, tuple[str, str, dict]] = {}
    for layer, config in records:
        kind = classify_config(config, layer, force_int8_gemm)
        if kind is None:
            continue
        if layer in out and out[layer][:2] != kind:
            prev = out[layer]
            raise ValueError(f"Conflicting ConvRot metadata for layer {layer}: "
                             f"{prev[0]}/{prev[1]} versus {kind[0]}/{kind[1]}")
        out.setdefault(layer, (*kind, config))
    return out


def summarize(classified: dict) -> ConvRotSummary:
    kinds = [v[:2] for v in classified.values()]
    return ConvRotSummary(w4a4=kinds.count(("w4", "int4")), w4a8=kinds.count(("w4", "int8")),
                          codebook_w4a8=kinds.count(("w4_codebook", "int8")), w8a8=kinds.count(("w8", "int8")))


def convrot_skip_reason(path) -> Optional[str]:
    """None when the file holds at least one supported ConvRot layer, else
    why it is not a ConvRot model (never raises)."""
    path = Path(path)
    if path.suffix.lower() not in (".safetensors", ".sft"):
        return f"unsupported file extension {path.suffix!r}"
    try:
        for layer, config in layer_configs(path):
            if classify_config(config, layer, True) is not None:
                return None
    except Exception as exc:  # any unreadable file is a reason, not an error
        return f"could not read ConvRot metadata ({exc})"
    return "does not contain supported ConvRot quantization metadata"


def load_w8a8_linears(path, *, prefix: Optional[str] = None, device="cpu",
                      force_int8_gemm: bool = False) -> dict:
    """layer name -> W8A8Linear for every W8 ConvRot layer under ``prefix``.
    Raises ValueError when the file has no ConvRot layer there or names a W8
    layer without its tensors."""
    from safetensors import safe_open

    from .wan_block import W8A8Linear

    classified = classify_layers(layer_configs(path, prefix), force_int8_gemm)
    if not classified:
        raise ValueError("The selected model does not contain supported ConvRot quantization metadata")
    linears = {}
    with safe_open(str(path), framework="pt", device="cpu") as f:
        keys = set(f.keys())
        for layer, (kind, _act, config) in classified.items():
            if kind != "w8":
                continue
            for need in (".weight", ".weight_scale"):
                if layer + need not in keys:
                    raise ValueError(f"W8 ConvRot layer {layer} has no {layer + need} tensor")
            weight = f.get_tensor(layer + ".weight")
            if weight.dtype != torch.int8 or weight.dim() != 2:
                raise ValueError(f"{layer}.weight must be a 2D int8 tensor")
            scale = f.get_tensor(layer + ".weight_scale")
            bias = f.get_tensor(layer + ".bias") if layer + ".bias" in keys else None
            group = _lookup(config, "convrot_groupsize", DEFAULT_W8_GROUP)
            if group not in (128, 256):
                raise ValueError(f"W8 ConvRot layer {layer} has convrot_groupsize={group!r}; this path runs 128 or 256")
            linears[layer] = W8A8Linear(weight.to(device), scale.to(device),
                                        None if bias is None else bias.to(device), group)
    return linears


def save_w8a8_linears(path, linears: dict, tensors: Optional[dict] = None, *, header_metadata: bool = False) -> None:
    """Writes W8A8Linear layers in the format above (``.comfy_quant`` tensors,
    or one header ``_quantization_metadata`` object when ``header_metadata``),
    plus any plain ``tensors``.  Scales are written per output channel with
    ``per_row`` metadata when they differ across channels."""
    from safetensors.torch import save_file

    out = {k: v.detach().contiguous().cpu() for k, v in (tensors or {}).items()}
    layers = {}
    for name, lin in linears.items():
        scale = lin.weight_scale.detach().cpu()
        uniform = bool((scale == scale[0]).all())
        config = {"format": W8_FORMAT, "convrot": True, "convrot_groupsize": lin.group, "linear_dtype": "int8"}
        if not uniform:
            config["per_row"] = True
        out[name + ".weight"] = lin.weight.detach().cpu().contiguous()
        out[name + ".weight_scale"] = scale[:1].reshape(()).clone() if uniform else scale.contiguous()
        if lin.bias is not None:
            out[name + ".bias"] = lin.bias.detach().cpu().contiguous()
        if header_metadata:
            layers[name] = config
        else:
            out[name + QUANT_SUFFIX] = encode_quant_tensor(config)
    metadata = {"_quantization_metadata": json.dumps({"layers": layers})} if header_metadata else None
    save_file(out, str(path), metadata=metadata)
