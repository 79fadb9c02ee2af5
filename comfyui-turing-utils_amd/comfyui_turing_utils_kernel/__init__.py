"""comfyui-turing-utils kernel package for AMD MI355X (gfx950).

Drop-in for the reference kernel package ``comfyui_turing_utils_kernel``
(``kernel/comfyui_turing_utils_kernel/__init__.py``) on the quantized DiT hot
path: the attribute names the plugin looks up through ``load_kernel_package()``
(``comfyui_turing_utils/quantization/dispatch.py:63-67``) and
``load_turing_sage()`` (``comfyui_turing_utils/kernel_api.py:22-23``) resolve to
torch.library ops backed by hand-written HIP kernels in ``libtu_hip.so``.

Importing the package registers the ops; it does not load the shared library
(the first op call does, and raises RuntimeError if it is missing).
"""
from .ops import (
    turing_bf16_gelu_int8_convrot_quantize,
    turing_bf16_int8_convrot_quantize,
    turing_dequantize_int8_bf16,
    turing_gelu_int8_convrot_quantize,
    turing_int8_gemm_i32,
    turing_int8_linear,
    turing_int8_linear_out,
    turing_layer_norm_adaln,
    turing_layer_norm_adaln_int8_convrot_quantize,
    turing_layer_norm_affine,
    turing_layer_norm_affine_int8_convrot_quantize,
    turing_swiglu_int8_convrot_quantize,
)
from . import turing_sage

# Version gates of the plugin compare against the reference's 0.29.1 ABI
# (comfyui_turing_utils/attention/stable.py:343-385); this build keeps the op
# contract of that version.
__version__ = "0.29.1"

__all__ = [
    "turing_bf16_gelu_int8_convrot_quantize",
    "turing_bf16_int8_convrot_quantize",
    "turing_dequantize_int8_bf16",
    "turing_gelu_int8_convrot_quantize",
    "turing_int8_gemm_i32",
    "turing_int8_linear",
    "turing_int8_linear_out",
    "turing_layer_norm_adaln",
    "turing_layer_norm_adaln_int8_convrot_quantize",
    "turing_layer_norm_affine",
    "turing_layer_norm_affine_int8_convrot_quantize",
    "turing_sage",
    "turing_swiglu_int8_convrot_quantize",
]
