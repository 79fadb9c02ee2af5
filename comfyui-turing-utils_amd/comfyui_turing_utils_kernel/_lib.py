"""ctypes binding of libtu_hip.so, the gfx950 C ABI declared in include/tu_hip.h.

This module is the only place that touches the shared library.  There is no
fallback: if the library is missing or fails to load, every op raises
``RuntimeError`` naming the build command.  ``torch`` is imported first so that
the library binds to the HIP runtime torch already loaded (both carry the
soname ``libamdhip64.so.7``).
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_NAME = "libtu_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
BUILD_HINT = (
    "build it with `make -C comfyui-turing-utils_amd/csrc` or "
    "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root"
)

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/tu_hip.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "tu_last_error": (ctypes.c_char_p, []),
    "tu_abi_version": (_i32, []),
    "tu_device_supported": (_i32, [_i32]),
    "tu_convrot_quant_i8": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _i32, _c_void_p]),
    "tu_int8_gemm_bf16": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p],
    ),
    "tu_int8_gemm_f16": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p],
    ),
    "tu_int8_gemm_f32": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p],
    ),
    "tu_int8_gemm_ex": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i64, _i64, _i32, _c_void_p],
    ),
    "tu_int8_gemm_tile_policy": (_i32, [_i64, _i64, _i32]),
    "tu_int8_gemm_bf16_residual": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _i64,
         _i64, _c_void_p],
    ),
    "tu_int8_gemm_i32": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p]),
    "tu_dequant_i32_bf16": (
        _i32,
        [_c_void_p, _i64, _c_void_p, _c_void_p, _i32, _c_void_p, _i64, _i64, _c_void_p],
    ),
    "tu_sage_kmean": (
        _i32,
        [_c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p, _c_void_p],
    ),
    "tu_sage_kmean_noalloc": (
        _i32,
        [_c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p, _c_void_p],
    ),
    "tu_sage_quant": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p],
    ),
    "tu_sage_v_prep": (
        _i32,
        [_c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _c_void_p],
    ),
    "tu_sage_attn_fwd": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _c_void_p,
         _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _f32, _i32, _c_void_p],
    ),
    "tu_sage_attn_fwd_split": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _c_void_p,
         _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _f32, _i32, _c_void_p, _i64, _c_void_p],
    ),
    "tu_sage_attn_kv_splits": (_i32, [_i64, _i64, _i64, _i64, _i32, _i32]),
    "tu_qk_rms_rope_int8": (
        _i32,
        [_c_void_p, _c_void_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, _i64, _i64,
         _c_void_p, _c_void_p, _i32, _f32, _c_void_p, _i64, _i32, _i64, _i64,
         _i64, _i64, _i64, _i64, _i64,
         _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _i64,
         _c_void_p, _c_void_p, _i32, _c_void_p, _c_void_p, _c_void_p],
    ),
    "tu_w8a8_quant_qk": (
        _i32,
        [_c_void_p, _c_void_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, _i64, _i64,
         _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _i64,
         _c_void_p, _c_void_p, _c_void_p, _i32, _c_void_p],
    ),
    "tu_w8a8_quant_v_workspace": (_i64, [_i64, _i64, _i64, _i64]),
    "tu_w8a8_quant_v": (
        _i32,
        [_c_void_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64,
         _c_void_p, _c_void_p, _i64, _c_void_p],
    ),
    "tu_w8a8_attn_fwd": (
        _i32,
        [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p,
         _i64, _c_void_p, _i32,
         _i64, _i64, _i64, _i64, _i64, _i64,
         _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
         _f32, _i32, _c_void_p],
    ),
    "tu_layer_norm_adaln": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i64, _i64, _i64, _f32, _c_void_p],
    ),
    "tu_layer_norm_affine": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i64, _f32, _c_void_p],
    ),
    "tu_layer_norm_adaln_convrot_quant_i8": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _f32, _c_void_p],
    ),
    "tu_layer_norm_affine_convrot_quant_i8": (
        _i32,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _f32, _c_void_p],
    ),
}

ABI_VERSION = 13

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Loads (once) and returns the library; raises RuntimeError if unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing; {BUILD_HINT}")
        try:
            lib = ctypes.CDLL(LIB_PATH)
        except OSError as exc:
            raise RuntimeError(f"failed to load {LIB_PATH}: {exc}; {BUILD_HINT}") from exc
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.tu_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Calls a tu_* entry point and raises RuntimeError with tu_last_error() on failure."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        message = lib.tu_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{name}: {message}")


def device_supported(device: torch.device) -> bool:
    """True when ``device`` is a CUDA/HIP device of the gfx950 family."""
    if device.type != "cuda":
        return False
    lib = load()
    index = device.index if device.index is not None else torch.cuda.current_device()
    result = lib.tu_device_supported(index)
    if result < 0:
        raise RuntimeError(f"tu_device_supported: {lib.tu_last_error().decode('utf-8', 'replace')}")
    return result == 1


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    """The current torch stream on ``device`` as a raw hipStream_t."""
    return torch.cuda.current_stream(device).cuda_stream
