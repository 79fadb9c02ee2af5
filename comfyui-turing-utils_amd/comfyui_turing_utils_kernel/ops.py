"""torch.library ops of the ConvRot W8A8 linear path, backed by libtu_hip.so.

Names, signatures, fake (meta) implementations and error types follow the
reference package's ``kernel/comfyui_turing_utils_kernel/ops.py`` so callers
that dispatch through ``torch.ops.turing_utils.*`` or the package attributes
(``comfyui_turing_utils/quantization/dispatch.py:63-67``) run unchanged.

Differences from the reference, by design of this MI355X build:
  * the device predicate is gfx950 instead of sm75;
  * the ConvRot quantizers accept ``group_size`` 128 (this build's
    block-Hadamard extension) as well as 256 (the reference's only size);
  * tanh and exp inside the fused GELU / SwiGLU activations are this
    build's fixed fp32 sequences (bit-identical to the CPU oracle), not
    CUDA's tanhf / expf;
  * ``int8_gemm_i32`` is an extra op exposing the raw INT32 accumulator of
    the same GEMM kernel, used for bit-exact parity checks;
  * ``int8_linear_out`` is an extra op writing the same epilogue in fp16 or
    fp32 (the output_dtype the plugin hands comfy-kitchen's fused linear).
"""
from __future__ import annotations

import torch

from . import _lib


def _require_device(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} requires CUDA (HIP) tensors")
    if not _lib.device_supported(t.device):
        raise RuntimeError(f"{what} requires a gfx950 (MI355X-class) GPU")


# ---------------------------------------------------------------------------
# INT8 linear (reference ops.py:96-126, bindings.cpp:371-421)
# ---------------------------------------------------------------------------
def _linear_args(activation, weight, activation_scale, weight_scale, bias):
    """int8_linear's checks and layouts; returns the normalized tensors and (m, n, k)."""
    _require_device(activation, "INT8 linear")
    activation = activation.contiguous()
    weight = weight.contiguous()
    activation_scale = activation_scale.reshape(-1).to(torch.float32).contiguous()
    weight_scale = weight_scale.reshape(-1).to(torch.float32).contiguous()
    if bias is not None:
        bias = bias.reshape(-1).to(torch.float32).contiguous()
    if activation.dim() != 2 or weight.dim() != 2:
        raise ValueError("INT8 linear activation and weight must be 2D")
    if activation.dtype != torch.int8 or weight.dtype != torch.int8:
        raise TypeError("INT8 linear activation and weight must be int8")
    devices = {activation.device, weight.device, activation_scale.device, weight_scale.device}
    if bias is not None:
        devices.add(bias.device)
    if len(devices) != 1:
        raise ValueError("INT8 linear tensors must use the same CUDA device")
    m, k = activation.shape
    n = weight.shape[0]
    if weight.shape[1] != k:
        raise ValueError("INT8 linear K dimensions must match")
    if k % 16 != 0 or n % 8 != 0:
        raise ValueError("INT8 linear requires K%16=0 and N%8=0")
    if activation_scale.numel() != m:
        raise ValueError("activation_scale must contain one value per row")
    if weight_scale.numel() != n:
        raise ValueError("weight_scale must contain one value per output channel")
    if bias is not None and bias.numel() != n:
        raise ValueError("bias must contain one value per output channel")
    return activation, weight, activation_scale, weight_scale, bias, m, n, k


@torch.library.custom_op("turing_utils::int8_linear", mutates_args=())
def turing_int8_linear(
    activation: torch.Tensor,
    weight: torch.Tensor,
    activation_scale: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """W8A8 contraction with the fused per-token x per-channel scale + bias epilogue."""
    activation, weight, activation_scale, weight_scale, bias, m, n, k = _linear_args(
        activation, weight, activation_scale, weight_scale, bias)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=activation.device)
    if m == 0:
        return out
    with torch.cuda.device(activation.device):
        _lib.call(
            "tu_int8_gemm_bf16",
            activation.data_ptr(), weight.data_ptr(), activation_scale.data_ptr(), weight_scale.data_ptr(),
            _lib.ptr(bias), out.data_ptr(), m, n, k, _lib.stream_of(activation.device),
        )
    return out


@turing_int8_linear.register_fake
def _turing_int8_linear_fake(activation, weight, activation_scale, weight_scale, bias=None):
    return torch.empty((activation.size(0), weight.size(0)), dtype=torch.bfloat16, device=activation.device)


_OUT_ENTRY = {torch.bfloat16: "tu_int8_gemm_bf16", torch.float16: "tu_int8_gemm_f16",
              torch.float32: "tu_int8_gemm_f32"}


@torch.library.custom_op("turing_utils::int8_linear_out", mutates_args=())
def turing_int8_linear_out(
    activation: torch.Tensor,
    weight: torch.Tensor,
    activation_scale: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None,
    out_dtype: torch.dtype,
) -> torch.Tensor:
    """int8_linear with the epilogue value ((acc * as) * ws) + bias written in
    ``out_dtype``: bf16 (int8_linear itself), fp16 rounded once from fp32
    (NaN as 0x7e00), or fp32 unrounded.  The output_dtype of the plugin's
    GEMM call (comfyui_turing_utils/quantization/dispatch.py:538-615), which
    the reference serves through comfy-kitchen; no counterpart among the
    reference package's ops."""
    if out_dtype not in _OUT_ENTRY:
        raise TypeError(f"INT8 linear out_dtype must be bfloat16, float16 or float32, got {out_dtype}")
    activation, weight, activation_scale, weight_scale, bias, m, n, k = _linear_args(
        activation, weight, activation_scale, weight_scale, bias)
    out = torch.empty((m, n), dtype=out_dtype, device=activation.device)
    if m == 0:
        return out
    with torch.cuda.device(activation.device):
        _lib.call(
            _OUT_ENTRY[out_dtype],
            activation.data_ptr(), weight.data_ptr(), activation_scale.data_ptr(), weight_scale.data_ptr(),
            _lib.ptr(bias), out.data_ptr(), m, n, k, _lib.stream_of(activation.device),
        )
    return out


@turing_int8_linear_out.register_fake
def _turing_int8_linear_out_fake(activation, weight, activation_scale, weight_scale, bias, out_dtype):
    if out_dtype not in _OUT_ENTRY:
        raise TypeError(f"INT8 linear out_dtype must be bfloat16, float16 or float32, got {out_dtype}")
    return torch.empty((activation.size(0), weight.size(0)), dtype=out_dtype, device=activation.device)


def _check_residual(residual, gate, gate_rows, m, n) -> None:
    if residual.dtype != torch.bfloat16 or tuple(residual.shape) != (m, n):
        raise ValueError(f"residual must be bf16 [{m}, {n}], got {residual.dtype} {tuple(residual.shape)}")
    if gate is not None:
        rows = (m + gate_rows - 1) // gate_rows if gate_rows > 0 else -1
        if gate.numel() != rows * n:
            raise ValueError(f"gate must hold one row of {n} values per {gate_rows} output rows, "
                             f"got {tuple(gate.shape)}")


@torch.library.custom_op("turing_utils::int8_linear_residual", mutates_args=())
def turing_int8_linear_residual(
    activation: torch.Tensor,
    weight: torch.Tensor,
    activation_scale: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None,
    residual: torch.Tensor,
    gate: torch.Tensor | None = None,
    gate_rows: int = 1,
) -> torch.Tensor:
    """int8_linear with a gated residual add fused into the epilogue:
    bf16_rn(fma(y, gate[row // gate_rows], residual)), y the int8_linear
    output, gate 1 when None.  residual: bf16 [M, N]; gate: bf16 [G, N]
    (one row per gate_rows consecutive rows, e.g. [B, N] with gate_rows = L).
    No counterpart in the reference's ops (it fuses a DiT block's residual
    add / addcmul into the projection)."""
    activation, weight, activation_scale, weight_scale, bias, m, n, k = _linear_args(
        activation, weight, activation_scale, weight_scale, bias)
    _check_residual(residual, gate, gate_rows, m, n)
    residual = residual.contiguous()
    if gate is not None:
        gate = gate.to(torch.bfloat16).reshape(-1, n).contiguous()
    devices = {activation.device, residual.device} | ({gate.device} if gate is not None else set())
    if len(devices) != 1:
        raise ValueError("INT8 linear tensors must use the same CUDA device")
    out = torch.empty((m, n), dtype=torch.bfloat16, device=activation.device)
    if m == 0:
        return out
    with torch.cuda.device(activation.device):
        _lib.call(
            "tu_int8_gemm_bf16_residual",
            activation.data_ptr(), weight.data_ptr(), activation_scale.data_ptr(), weight_scale.data_ptr(),
            _lib.ptr(bias), residual.data_ptr(), _lib.ptr(gate), int(gate_rows) if gate is not None else 1,
            out.data_ptr(), m, n, k, _lib.stream_of(activation.device),
        )
    return out


@turing_int8_linear_residual.register_fake
def _turing_int8_linear_residual_fake(activation, weight, activation_scale, weight_scale, bias, residual, gate=None,
                                      gate_rows=1):
    _check_residual(residual, gate, gate_rows, activation.size(0), weight.size(0))
    return torch.empty((activation.size(0), weight.size(0)), dtype=torch.bfloat16, device=activation.device)


@torch.library.custom_op("turing_utils::int8_gemm_i32", mutates_args=())
def turing_int8_gemm_i32(activation: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """INT32 accumulator ``activation @ weight.T`` of the same MFMA GEMM kernel."""
    _require_device(activation, "INT8 GEMM")
    activation = activation.contiguous()
    weight = weight.contiguous()
    if activation.dtype != torch.int8 or weight.dtype != torch.int8:
        raise TypeError("INT8 GEMM operands must be int8")
    if activation.dim() != 2 or weight.dim() != 2 or weight.shape[1] != activation.shape[1]:
        raise ValueError("INT8 GEMM operands must be [M, K] and [N, K]")
    if activation.device != weight.device:
        raise ValueError("INT8 GEMM operands must share one device")
    m, k = activation.shape
    n = weight.shape[0]
    if k % 16 != 0 or n % 8 != 0:
        raise ValueError("INT8 GEMM requires K%16=0 and N%8=0")
    out = torch.empty((m, n), dtype=torch.int32, device=activation.device)
    if m == 0:
        return out
    with torch.cuda.device(activation.device):
        _lib.call("tu_int8_gemm_i32", activation.data_ptr(), weight.data_ptr(), out.data_ptr(), m, n, k,
                  _lib.stream_of(activation.device))
    return out


@turing_int8_gemm_i32.register_fake
def _turing_int8_gemm_i32_fake(activation, weight):
    return torch.empty((activation.size(0), weight.size(0)), dtype=torch.int32, device=activation.device)


# ---------------------------------------------------------------------------
# INT32 -> BF16 epilogue (reference ops.py:129-160, bindings.cpp:423-472)
# ---------------------------------------------------------------------------
@torch.library.custom_op("turing_utils::dequantize_int8_bf16", mutates_args=())
def turing_dequantize_int8_bf16(
    accumulator: torch.Tensor,
    activation_scale: torch.Tensor,
    weight_scale: torch.Tensor,
    output_columns: int = -1,
) -> torch.Tensor:
    """Dequantize an INT32 GEMM workspace directly into packed BF16 stores."""
    _require_device(accumulator, "BF16 epilogue")
    if accumulator.dtype != torch.int32 or accumulator.ndim != 2:
        raise TypeError("accumulator must be a 2D int32 tensor")
    accumulator = accumulator.contiguous()
    activation_scale = activation_scale.reshape(-1).to(torch.float32).contiguous()
    weight_scale = weight_scale.reshape(-1).to(torch.float32).contiguous()
    if accumulator.device != activation_scale.device or accumulator.device != weight_scale.device:
        raise ValueError("accumulator and scales must use the same CUDA device")
    rows, acc_cols = accumulator.shape
    cols = acc_cols if output_columns < 0 else output_columns
    if rows <= 0 or acc_cols <= 0:
        raise ValueError("INT8 BF16 epilogue dimensions must be positive")
    if not 0 < cols <= acc_cols:
        raise ValueError("output_columns must be positive and no larger than the accumulator width")
    if activation_scale.numel() != rows:
        raise ValueError("activation_scale must contain one value per accumulator row")
    if weight_scale.numel() not in (1, cols):
        raise ValueError("weight_scale must be scalar or contain one value per output column")
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=accumulator.device)
    with torch.cuda.device(accumulator.device):
        _lib.call(
            "tu_dequant_i32_bf16", accumulator.data_ptr(), acc_cols, activation_scale.data_ptr(),
            weight_scale.data_ptr(), int(weight_scale.numel() == 1), out.data_ptr(), rows, cols,
            _lib.stream_of(accumulator.device),
        )
    return out


@turing_dequantize_int8_bf16.register_fake
def _turing_dequantize_int8_bf16_fake(accumulator, activation_scale, weight_scale, output_columns=-1):
    columns = accumulator.size(1) if output_columns < 0 else output_columns
    return torch.empty((accumulator.size(0), columns), dtype=torch.bfloat16, device=accumulator.device)


# ---------------------------------------------------------------------------
# ConvRot INT8 activation quantizer (reference ops.py:257-282, :313-331)
# ---------------------------------------------------------------------------
SUPPORTED_GROUP_SIZES = (128, 256)
ACT_NONE, ACT_GELU_TANH, ACT_SWIGLU = 0, 1, 2
STAGED_SCALE = 0x100  # scale = absmax * (1/127), the two-pass kernels' formula
FP16_INPUT = 0x200  # x holds float16 (the two-pass kernels' InputType = half)
MAX_CONVROT_COLUMNS = 65536  # activated width; the kernel keeps a whole row in registers


def _convrot_quantize(x: torch.Tensor, group_size: int, act: int, what: str,
                      staged: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """staged=True is the two-pass ops' contract: staged scale formula and
    float16 or bfloat16 input (ops.py:163-186, :215-233); the row-buffer ops
    take bfloat16 only (ops.py:257-282, :313-331)."""
    _require_device(x, what)
    if staged:
        if x.dtype not in (torch.float16, torch.bfloat16):
            raise TypeError(f"{what} input must be float16 or bfloat16")
    elif x.dtype != torch.bfloat16:
        raise TypeError(f"{what} input must be bfloat16")
    if x.ndim != 2:
        raise ValueError(f"{what} input must be 2D")
    if group_size not in SUPPORTED_GROUP_SIZES:
        raise ValueError(f"{what} supports group_size {SUPPORTED_GROUP_SIZES}, got {group_size}")
    x = x.contiguous()
    rows, width = x.shape
    if act == ACT_SWIGLU and width % 2:
        raise ValueError(f"{what} SwiGLU input width must be even")
    hidden = width // 2 if act == ACT_SWIGLU else width
    if rows <= 0 or hidden <= 0 or hidden % group_size:
        raise ValueError(f"{what} width must be positive and divisible by {group_size}")
    if hidden > MAX_CONVROT_COLUMNS:
        raise ValueError(f"{what} width {hidden} exceeds the {MAX_CONVROT_COLUMNS}-column limit")
    if x.data_ptr() % 16:
        x = x.clone()  # the kernel reads 16-byte vectors
    q = torch.empty((rows, hidden), dtype=torch.int8, device=x.device)
    scales = torch.empty((rows, 1), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        flags = (STAGED_SCALE if staged else 0) | (FP16_INPUT if x.dtype == torch.float16 else 0)
        _lib.call("tu_convrot_quant_i8", x.data_ptr(), q.data_ptr(), scales.data_ptr(), rows, hidden,
                  group_size, act | flags, _lib.stream_of(x.device))
    return q, scales


@torch.library.custom_op("turing_utils::bf16_int8_convrot_quantize", mutates_args=())
def turing_bf16_int8_convrot_quantize(
    x: torch.Tensor,
    group_size: int = 256,
    *,
    swiglu: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Whole-row BF16 ConvRot rotation + per-token symmetric INT8 quantization.
    swiglu=True folds SwiGLU over the [gate | up] halves of each row first."""
    return _convrot_quantize(x, group_size, ACT_SWIGLU if swiglu else ACT_NONE, "BF16 row-buffer ConvRot")


@turing_bf16_int8_convrot_quantize.register_fake
def _turing_bf16_int8_convrot_quantize_fake(x, group_size=256, *, swiglu=False):
    hidden = x.size(1) // 2 if swiglu else x.size(1)
    return (
        torch.empty((x.size(0), hidden), dtype=torch.int8, device=x.device),
        torch.empty((x.size(0), 1), dtype=torch.float32, device=x.device),
    )


@torch.library.custom_op("turing_utils::bf16_gelu_int8_convrot_quantize", mutates_args=())
def turing_bf16_gelu_int8_convrot_quantize(
    x: torch.Tensor,
    group_size: int = 256,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Whole-row BF16 tanh-GELU + ConvRot INT8 quantization (reference ops.py:313-331):
    GELU is applied on load and rounded to bf16 before the rotation."""
    return _convrot_quantize(x, group_size, ACT_GELU_TANH, "BF16 GELU ConvRot")


@turing_bf16_gelu_int8_convrot_quantize.register_fake
def _turing_bf16_gelu_int8_convrot_quantize_fake(x, group_size=256):
    return (
        torch.empty(x.shape, dtype=torch.int8, device=x.device),
        torch.empty((x.size(0), 1), dtype=torch.float32, device=x.device),
    )


# ---------------------------------------------------------------------------
# Two-pass ("staged") fused-activation quantizers (reference ops.py:163-186,
# :215-233; bindings.cpp:474-510, :550-600).  The reference computes these in
# two kernels through a global bf16 / fp16 copy of the rotated rows; here the
# same single-pass kernel runs with the staged scale formula (and fp16
# elements for float16 input), so codes and scales equal the reference's
# two-pass results.
# ---------------------------------------------------------------------------
@torch.library.custom_op("turing_utils::swiglu_int8_convrot_quantize", mutates_args=())
def turing_swiglu_int8_convrot_quantize(
    x: torch.Tensor,
    group_size: int = 256,
) -> tuple[torch.Tensor, torch.Tensor]:
    """SwiGLU over the [gate | up] halves of each row (float16 or bfloat16),
    then ConvRot INT8 quantization."""
    return _convrot_quantize(x, group_size, ACT_SWIGLU, "SwiGLU ConvRot", staged=True)


@turing_swiglu_int8_convrot_quantize.register_fake
def _turing_swiglu_int8_convrot_quantize_fake(x, group_size=256):
    return (
        torch.empty((x.size(0), x.size(1) // 2), dtype=torch.int8, device=x.device),
        torch.empty((x.size(0), 1), dtype=torch.float32, device=x.device),
    )


@torch.library.custom_op("turing_utils::gelu_int8_convrot_quantize", mutates_args=())
def turing_gelu_int8_convrot_quantize(
    x: torch.Tensor,
    group_size: int = 256,
) -> tuple[torch.Tensor, torch.Tensor]:
    """tanh-GELU (rounded to the input type, float16 or bfloat16), then
    ConvRot INT8 quantization."""
    return _convrot_quantize(x, group_size, ACT_GELU_TANH, "GELU ConvRot", staged=True)


@turing_gelu_int8_convrot_quantize.register_fake
def _turing_gelu_int8_convrot_quantize_fake(x, group_size=256):
    return (
        torch.empty(x.shape, dtype=torch.int8, device=x.device),
        torch.empty((x.size(0), 1), dtype=torch.float32, device=x.device),
    )


# ---------------------------------------------------------------------------
# LayerNorm + AdaLN (reference ops.py:399-418, segmented_rms_adaln.cu:236-409)
# ---------------------------------------------------------------------------
_LN_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


@torch.library.custom_op("turing_utils::layer_norm_adaln", mutates_args=())
def turing_layer_norm_adaln(
    x: torch.Tensor,
    scale: torch.Tensor,
    shift: torch.Tensor,
    epsilon: float = 1.0e-5,
) -> torch.Tensor:
    """Fused FP32-reduction LayerNorm and Wan AdaLN modulation:
    LayerNorm(x) * (1 + scale) + shift with x [B, L, H] and scale / shift
    [B, steps, H] (token t of L uses modulation row t // ceil(L / steps))."""
    _require_device(x, "LayerNorm+AdaLN")
    if x.dtype not in _LN_DTYPES or x.ndim != 3:
        raise TypeError("LayerNorm+AdaLN input must be 3D float16, bfloat16, or float32")
    scale = scale.to(device=x.device, dtype=x.dtype).contiguous()
    shift = shift.to(device=x.device, dtype=x.dtype).contiguous()
    batch, length, hidden = x.shape
    if scale.ndim != 3 or scale.shape != shift.shape or scale.size(0) != batch or scale.size(2) != hidden:
        raise ValueError("LayerNorm+AdaLN scale / shift must be [B, steps, H] and match")
    x = x.contiguous()
    out = torch.empty_like(x)
    with torch.cuda.device(x.device):
        _lib.call("tu_layer_norm_adaln", x.data_ptr(), scale.data_ptr(), shift.data_ptr(), out.data_ptr(),
                  _LN_DTYPES[x.dtype], batch, length, hidden, scale.size(1), float(epsilon),
                  _lib.stream_of(x.device))
    return out


@turing_layer_norm_adaln.register_fake
def _turing_layer_norm_adaln_fake(x, scale, shift, epsilon=1.0e-5):
    return torch.empty_like(x)


# ---------------------------------------------------------------------------
# LayerNorm with an elementwise affine weight / bias (no reference op: ComfyUI's
# torch LayerNorm runs the Wan block's norm3, which the reference leaves alone)
# ---------------------------------------------------------------------------
@torch.library.custom_op("turing_utils::layer_norm_affine", mutates_args=())
def turing_layer_norm_affine(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    epsilon: float = 1.0e-5,
) -> torch.Tensor:
    """layer_norm(x, (H,), weight, bias, epsilon) over the last dimension of
    x [..., H]: fp32 statistics in the order of layer_norm_adaln, one rounding
    of fma(normalized, weight, bias) to x's dtype."""
    _require_device(x, "LayerNorm")
    if x.dtype not in _LN_DTYPES or x.ndim < 1:
        raise TypeError("LayerNorm input must be float16, bfloat16, or float32")
    hidden = x.shape[-1]
    weight = weight.to(device=x.device, dtype=x.dtype).reshape(-1).contiguous()
    bias = bias.to(device=x.device, dtype=x.dtype).reshape(-1).contiguous()
    if weight.numel() != hidden or bias.numel() != hidden:
        raise ValueError(f"LayerNorm weight and bias must hold {hidden} values")
    x = x.contiguous()
    out = torch.empty_like(x)
    rows = x.numel() // hidden if hidden else 0
    with torch.cuda.device(x.device):
        _lib.call("tu_layer_norm_affine", x.data_ptr(), weight.data_ptr(), bias.data_ptr(), out.data_ptr(),
                  _LN_DTYPES[x.dtype], rows, hidden, float(epsilon), _lib.stream_of(x.device))
    return out


@turing_layer_norm_affine.register_fake
def _turing_layer_norm_affine_fake(x, weight, bias, epsilon=1.0e-5):
    return torch.empty_like(x)


# ---------------------------------------------------------------------------
# LayerNorm fused with the ConvRot INT8 quantizer (no reference op: the
# reference runs the norm, ops.py:399-418, and the linear's activation
# quantizer, quantization/dispatch.py:538-615, as two ops)
# ---------------------------------------------------------------------------
LN_CONVROT_MAX_HIDDEN = 5120  # rows and rotated values stay in registers


def _ln_convrot_fused(x: torch.Tensor, hidden: int, group_size: int) -> bool:
    """The one-kernel path: bf16, G = 128, hidden a multiple of 256 up to 5120."""
    return (x.dtype == torch.bfloat16 and group_size == 128 and hidden % 256 == 0
            and 256 <= hidden <= LN_CONVROT_MAX_HIDDEN)


def _aligned16(*tensors: torch.Tensor) -> bool:
    return all(t.data_ptr() % 16 == 0 for t in tensors)


@torch.library.custom_op("turing_utils::layer_norm_adaln_int8_convrot_quantize", mutates_args=())
def turing_layer_norm_adaln_int8_convrot_quantize(
    x: torch.Tensor,
    scale: torch.Tensor,
    shift: torch.Tensor,
    epsilon: float = 1.0e-5,
    group_size: int = 128,
) -> tuple[torch.Tensor, torch.Tensor]:
    """ConvRot INT8 codes [B*L, H] and row scales [B*L, 1] of
    layer_norm_adaln(x, scale, shift, epsilon), bit for bit those of
    bf16_int8_convrot_quantize(layer_norm_adaln(...).reshape(-1, H), group_size).
    bf16 x with group 128 and H a multiple of 256 up to 5120 runs as one
    kernel (the normalized rows never reach memory); anything else runs the
    two ops."""
    _require_device(x, "LayerNorm+AdaLN ConvRot")
    if x.dtype not in _LN_DTYPES or x.ndim != 3:
        raise TypeError("LayerNorm+AdaLN input must be 3D float16, bfloat16, or float32")
    batch, length, hidden = x.shape
    if not _ln_convrot_fused(x, hidden, group_size):
        normed = turing_layer_norm_adaln(x, scale, shift, epsilon)
        return _convrot_quantize(normed.reshape(batch * length, hidden), group_size, ACT_NONE,
                                 "BF16 row-buffer ConvRot")
    scale = scale.to(device=x.device, dtype=x.dtype).contiguous()
    shift = shift.to(device=x.device, dtype=x.dtype).contiguous()
    if scale.ndim != 3 or scale.shape != shift.shape or scale.size(0) != batch or scale.size(2) != hidden:
        raise ValueError("LayerNorm+AdaLN scale / shift must be [B, steps, H] and match")
    x = x.contiguous()
    if not _aligned16(x, scale, shift):  # the kernel reads 16-byte vectors
        x, scale, shift = x.clone(), scale.clone(), shift.clone()
    q = torch.empty((batch * length, hidden), dtype=torch.int8, device=x.device)
    scales = torch.empty((batch * length, 1), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("tu_layer_norm_adaln_convrot_quant_i8", x.data_ptr(), scale.data_ptr(), shift.data_ptr(),
                  q.data_ptr(), scales.data_ptr(), batch, length, hidden, scale.size(1), float(epsilon),
                  _lib.stream_of(x.device))
    return q, scales


@turing_layer_norm_adaln_int8_convrot_quantize.register_fake
def _turing_layer_norm_adaln_int8_convrot_quantize_fake(x, scale, shift, epsilon=1.0e-5, group_size=128):
    rows = x.size(0) * x.size(1)
    return (torch.empty((rows, x.size(2)), dtype=torch.int8, device=x.device),
            torch.empty((rows, 1), dtype=torch.float32, device=x.device))


@torch.library.custom_op("turing_utils::layer_norm_affine_int8_convrot_quantize", mutates_args=())
def turing_layer_norm_affine_int8_convrot_quantize(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    epsilon: float = 1.0e-5,
    group_size: int = 128,
) -> tuple[torch.Tensor, torch.Tensor]:
    """ConvRot INT8 codes [rows, H] and row scales [rows, 1] of
    layer_norm_affine(x, weight, bias, epsilon) over x [..., H], bit for bit
    those of bf16_int8_convrot_quantize on that output; one kernel under the
    conditions of layer_norm_adaln_int8_convrot_quantize, else the two ops."""
    _require_device(x, "LayerNorm ConvRot")
    if x.dtype not in _LN_DTYPES or x.ndim < 1:
        raise TypeError("LayerNorm input must be float16, bfloat16, or float32")
    hidden = x.shape[-1]
    rows = x.numel() // hidden if hidden else 0
    if not _ln_convrot_fused(x, hidden, group_size) or rows == 0:
        normed = turing_layer_norm_affine(x, weight, bias, epsilon)
        return _convrot_quantize(normed.reshape(rows, hidden), group_size, ACT_NONE, "BF16 row-buffer ConvRot")
    weight = weight.to(device=x.device, dtype=x.dtype).reshape(-1).contiguous()
    bias = bias.to(device=x.device, dtype=x.dtype).reshape(-1).contiguous()
    if weight.numel() != hidden or bias.numel() != hidden:
        raise ValueError(f"LayerNorm weight and bias must hold {hidden} values")
    x = x.contiguous()
    if not _aligned16(x, weight, bias):
        x, weight, bias = x.clone(), weight.clone(), bias.clone()
    q = torch.empty((rows, hidden), dtype=torch.int8, device=x.device)
    scales = torch.empty((rows, 1), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.call("tu_layer_norm_affine_convrot_quant_i8", x.data_ptr(), weight.data_ptr(), bias.data_ptr(),
                  q.data_ptr(), scales.data_ptr(), rows, hidden, float(epsilon), _lib.stream_of(x.device))
    return q, scales


@turing_layer_norm_affine_int8_convrot_quantize.register_fake
def _turing_layer_norm_affine_int8_convrot_quantize_fake(x, weight, bias, epsilon=1.0e-5, group_size=128):
    hidden = x.shape[-1]
    rows = x.numel() // hidden if hidden else 0
    return (torch.empty((rows, hidden), dtype=torch.int8, device=x.device),
            torch.empty((rows, 1), dtype=torch.float32, device=x.device))
