"""Wan 2.1 DiT block forward on this package's W8A8 linears and INT8 attention.

The reference plugin does not own the block: ComfyUI's WanAttentionBlock does,
and the plugin swaps in its kernels at the self-attention site
(comfyui_turing_utils/adapters/wan.py:55-137: q / k / v projections, row-scope
RMSNorm + interleaved RoPE + INT8 through turing_utils::qk_rms_rope_int8, Sage
attention, o projection), at the linears (the ConvRot W8A8 layout,
quantization/dispatch.py) and at the norms (turing_utils::layer_norm_adaln,
kernel/scripts/validate_wan_fusions.py:80-119).  This module composes the same
ops into the whole block so that it can be run and timed without ComfyUI:

    e = modulation + e_t                     [B, 6, C]: shift, scale, gate (attention),
                                                         shift, scale, gate (FFN)
    x = x + SelfAttn(LN(x) * (1 + e1) + e0) * e2
    x = x + CrossAttn(LN_affine(x), context)
    x = x + FFN(LN(x) * (1 + e4) + e3) * e5

* norm1 / norm2: ``turing_utils::layer_norm_adaln``.  norm3, LayerNorm with
  an elementwise weight and bias (ComfyUI's own LayerNorm in the reference's
  setting): ``turing_utils::layer_norm_affine``, any weight values.  In the
  forward each norm's output has one consumer, the next projection's ConvRot
  quantizer, so norm and quantizer run as one kernel
  (``turing_utils::layer_norm_adaln_int8_convrot_quantize`` /
  ``layer_norm_affine_int8_convrot_quantize``) and the normalized rows are
  never written; the codes are those of the two ops, bit for bit.
* SelfAttn: q, k and v come from one W8A8 GEMM (N = 3C).  q and k go through
  one fused RMSNorm + RoPE + INT8 kernel.  Then Sage INT8 attention, and the
  o projection.
* CrossAttn: q from x; k and v from the text context through one GEMM
  (N = 2C).  RMSNorm + INT8 of q and k, no RoPE.  Then Sage attention over the
  text tokens.
* FFN: W8A8 up projection; the tanh-GELU is fused into the down projection's
  ConvRot quantizer (``turing_utils::bf16_gelu_int8_convrot_quantize``).
* Text embedding (once per model forward, not per block): Linear(4096, C),
  tanh-GELU, Linear(C, C), all W8A8 the same way.

Every linear is ConvRot W8A8 at group 128: the weights are rotated and
quantized per output channel by the same kernel that quantizes activations
per token (the rotation is orthogonal, so rot(x) . rot(w) = x . w).  The
residual stream x is bf16; each residual add, x + y * gate, runs in the
epilogue of the projection that produces y (``turing_utils::int8_linear_residual``):
bf16_rn(fma(y, gate, x)) with y the bf16 projection output.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import ops  # noqa: F401  (registers torch.ops.turing_utils.*)
from .turing_sage import core as sage_core

GROUP = 128


@dataclass
class QuantizedActivation:
    """ConvRot INT8 codes [B*L, C] and row scales [B*L, 1] (group ``group``)
    of a bf16 activation [B, L, C], as a fused norm + quantizer makes them."""
    codes: torch.Tensor
    scale: torch.Tensor
    batch: int
    length: int
    group: int

    @property
    def shape(self) -> tuple[int, int, int]:
        return (self.batch, self.length, self.codes.shape[1])


def _token_rows(h):
    """[B*L, C] rows of a bf16 activation [B, L, C], or its codes as they are."""
    if isinstance(h, QuantizedActivation):
        return h
    b, l, c = h.shape
    return h.reshape(b * l, c)


class W8A8Linear:
    """y = x W^T + b with W stored as ConvRot-rotated INT8 codes and a
    per-output-channel fp32 scale; x is quantized per token by the ConvRot
    quantizer (optionally with the tanh-GELU applied first)."""

    def __init__(self, weight_int8: torch.Tensor, weight_scale: torch.Tensor, bias: Optional[torch.Tensor],
                 group: int = GROUP):
        if weight_int8.dtype != torch.int8 or weight_int8.dim() != 2:
            raise TypeError("W8A8 weight must be a 2D int8 tensor")
        if group not in (128, 256) or weight_int8.shape[1] % group:
            raise ValueError(f"ConvRot group {group} must be 128 or 256 and divide K={weight_int8.shape[1]}")
        self.weight = weight_int8.contiguous()
        self.out_features, self.in_features = self.weight.shape
        scale = weight_scale.reshape(-1).to(torch.float32)
        if scale.numel() == 1:  # tensor-wise scale
            scale = scale.expand(self.out_features)
        if scale.numel() != self.out_features:
            raise ValueError(f"weight scale has {scale.numel()} values for {self.out_features} output channels")
        self.weight_scale = scale.contiguous()
        self.bias = None if bias is None else bias.reshape(-1).to(torch.float32).contiguous()
        if self.bias is not None and self.bias.numel() != self.out_features:
            raise ValueError("bias length must equal the output channels")
        self.group = group

    @classmethod
    def from_float(cls, weight: torch.Tensor, bias: Optional[torch.Tensor] = None, group: int = GROUP) -> "W8A8Linear":
        """Quantizes a dense weight [N, K] (rounded to bf16 first) on its device."""
        codes, scale = torch.ops.turing_utils.bf16_int8_convrot_quantize(
            weight.to(torch.bfloat16).contiguous(), group)
        return cls(codes, scale, bias, group)

    def __call__(self, x, gelu: bool = False, residual: Optional[torch.Tensor] = None,
                 gate: Optional[torch.Tensor] = None, gate_rows: int = 1) -> torch.Tensor:
        """y = x W^T + b, or residual + y * gate[row // gate_rows] (gate 1 when
        None) fused into the GEMM epilogue when ``residual`` [M, N] is given.
        x: bf16 [M, K], or a QuantizedActivation of this linear's group."""
        if isinstance(x, QuantizedActivation):
            if gelu or x.group != self.group or x.codes.shape[1] != self.in_features:
                raise ValueError(f"W8A8 linear expects codes of [M, {self.in_features}] at group {self.group} "
                                 f"without an activation, got {tuple(x.codes.shape)} at group {x.group}")
            codes, scale = x.codes, x.scale
        else:
            if x.dim() != 2 or x.shape[1] != self.in_features:
                raise ValueError(f"W8A8 linear expects [M, {self.in_features}], got {tuple(x.shape)}")
            quantize = (torch.ops.turing_utils.bf16_gelu_int8_convrot_quantize if gelu
                        else torch.ops.turing_utils.bf16_int8_convrot_quantize)
            codes, scale = quantize(x.contiguous(), self.group)
        if residual is None:
            return torch.ops.turing_utils.int8_linear(codes, self.weight, scale, self.weight_scale, self.bias)
        return torch.ops.turing_utils.int8_linear_residual(codes, self.weight, scale, self.weight_scale, self.bias,
                                                           residual, gate, gate_rows)

    @staticmethod
    def concat(parts: "list[W8A8Linear]") -> "W8A8Linear":
        """One linear whose output is the parts' outputs side by side (same K
        and group): codes, scales and biases stacked along N."""
        if len({(p.in_features, p.group) for p in parts}) != 1:
            raise ValueError("concatenated linears need one K and one ConvRot group")
        if len({p.bias is None for p in parts}) != 1:
            raise ValueError("concatenated linears must all have a bias or none")
        bias = None if parts[0].bias is None else torch.cat([p.bias for p in parts])
        return W8A8Linear(torch.cat([p.weight for p in parts]), torch.cat([p.weight_scale for p in parts]), bias,
                          parts[0].group)

    def split(self, n: int) -> "list[W8A8Linear]":
        """The inverse of ``concat`` for ``n`` equal parts."""
        if self.out_features % n:
            raise ValueError(f"{self.out_features} output channels do not split into {n} equal parts")
        size = self.out_features // n
        return [W8A8Linear(self.weight[i * size:(i + 1) * size], self.weight_scale[i * size:(i + 1) * size],
                           None if self.bias is None else self.bias[i * size:(i + 1) * size], self.group)
                for i in range(n)]


def rope_freqs(grid: tuple[int, int, int], head_dim: int = 128, theta: float = 10000.0,
               device=None) -> torch.Tensor:
    """Wan's 3D rotary table as rotation matrices, [1, F*H*W, 1, D/2, 2, 2]
    ([[cos, -sin], [sin, cos]] per channel pair, interleaved pairs): the
    head_dim splits into D - 4*(D//6) temporal and 2*(D//6) + 2*(D//6)
    spatial channels, each axis with frequencies theta^(-2i/d)."""
    f, h, w = grid
    dims = (head_dim - 4 * (head_dim // 6), 2 * (head_dim // 6), 2 * (head_dim // 6))
    angles = []
    for n, d, shape in zip((f, h, w), dims, ((f, 1, 1), (1, h, 1), (1, 1, w))):
        inv = theta ** (-torch.arange(0, d, 2, dtype=torch.float64) / d)
        a = torch.arange(n, dtype=torch.float64)[:, None] * inv[None, :]
        angles.append(a.view(*shape, d // 2).expand(f, h, w, d // 2))
    ang = torch.cat(angles, -1).reshape(1, f * h * w, 1, head_dim // 2)
    cos, sin = ang.cos(), ang.sin()
    rot = torch.stack([torch.stack([cos, -sin], -1), torch.stack([sin, cos], -1)], -2)
    return rot.to(torch.float32).to(device)


@dataclass
class WanBlockConfig:
    dim: int = 5120
    heads: int = 40
    ffn_dim: int = 13824
    text_dim: int = 4096
    eps: float = 1e-6

    @property
    def head_dim(self) -> int:
        return self.dim // self.heads


class WanTextEmbeddingW8A8:
    """Linear(text_dim, C), tanh-GELU, Linear(C, C) on the text context."""

    def __init__(self, fc1: W8A8Linear, fc2: W8A8Linear):
        self.fc1, self.fc2 = fc1, fc2

    def __call__(self, context: torch.Tensor) -> torch.Tensor:
        b, l, d = context.shape
        hidden = self.fc1(context.reshape(b * l, d))
        return self.fc2(hidden, gelu=True).view(b, l, -1)


class WanBlockW8A8:
    """One Wan 2.1 attention block; see the module docstring for the math."""

    def __init__(self, cfg: WanBlockConfig, *, modulation: torch.Tensor,
                 self_qkv: W8A8Linear, self_o: W8A8Linear, self_norm_q: torch.Tensor, self_norm_k: torch.Tensor,
                 norm3_weight: torch.Tensor, norm3_bias: torch.Tensor,
                 cross_q: W8A8Linear, cross_kv: W8A8Linear, cross_o: W8A8Linear,
                 cross_norm_q: torch.Tensor, cross_norm_k: torch.Tensor,
                 ffn_up: W8A8Linear, ffn_down: W8A8Linear):
        c = cfg.dim
        if cfg.head_dim not in (64, 128) or cfg.head_dim * cfg.heads != c:
            raise ValueError("Wan block needs head_dim 64 or 128 and heads * head_dim == dim")
        for lin, k, n in ((self_qkv, c, 3 * c), (self_o, c, c), (cross_q, c, c), (cross_kv, c, 2 * c),
                          (cross_o, c, c), (ffn_up, c, cfg.ffn_dim), (ffn_down, cfg.ffn_dim, c)):
            if (lin.in_features, lin.out_features) != (k, n):
                raise ValueError(f"linear shape {(lin.out_features, lin.in_features)} != {(n, k)}")
        self.cfg = cfg
        self.modulation = modulation.to(torch.float32).reshape(1, 6, c)
        self.self_qkv, self.self_o = self_qkv, self_o
        self.self_norm_q = self_norm_q.to(torch.bfloat16).contiguous()
        self.self_norm_k = self_norm_k.to(torch.bfloat16).contiguous()
        self.cross_q, self.cross_kv, self.cross_o = cross_q, cross_kv, cross_o
        self.cross_norm_q = cross_norm_q.to(torch.bfloat16).contiguous()
        self.cross_norm_k = cross_norm_k.to(torch.bfloat16).contiguous()
        self.ffn_up, self.ffn_down = ffn_up, ffn_down
        self.norm3_weight = norm3_weight.to(torch.bfloat16).reshape(c).contiguous()
        self.norm3_bias = norm3_bias.to(torch.bfloat16).reshape(c).contiguous()

    # -- sublayers (each takes and returns bf16 [B, L, C]) ---------------------

    # (h: bf16 [B, L, C] or its QuantizedActivation for the first projection)

    def self_attention(self, h, freqs: torch.Tensor, residual: Optional[torch.Tensor] = None,
                       gate: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The attention output projected by o; with ``residual`` [B, L, C],
        residual + that * gate (gate [B, 1, C] or None) from one epilogue."""
        cfg = self.cfg
        b, l, c = h.shape
        qkv = self.self_qkv(_token_rows(h)).view(b, l, 3, cfg.heads, cfg.head_dim)
        q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
        qk = sage_core.prequantize_rms_rope_qk(
            q, k, self.self_norm_q, self.self_norm_k, freqs, epsilon=cfg.eps, rot_dim=cfg.head_dim,
            tensor_layout="NHD", norm_scope="row")
        state = sage_core.prequantize_sageattn_from_qk(qk, v, sm_scale=cfg.head_dim ** -0.5)
        del qkv, q, k, qk
        out = sage_core.sageattn_from_prequantized(state)
        return self._project(self.self_o, out.reshape(b * l, c), residual, gate).view(b, l, c)

    def _project(self, lin: W8A8Linear, x2d: torch.Tensor, residual, gate, gelu: bool = False) -> torch.Tensor:
        if residual is None:
            return lin(x2d, gelu=gelu)
        b, l, c = residual.shape
        g = None if gate is None else gate.reshape(b, c)
        return lin(x2d, gelu=gelu, residual=residual.reshape(b * l, c), gate=g, gate_rows=l)

    def cross_attention(self, h, context: torch.Tensor,
                        residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        cfg = self.cfg
        b, l, c = h.shape
        lc = context.shape[1]
        q = self.cross_q(_token_rows(h)).view(b, l, cfg.heads, cfg.head_dim)
        kv = self.cross_kv(context.reshape(b * lc, c)).view(b, lc, 2, cfg.heads, cfg.head_dim)
        k, v = kv[:, :, 0], kv[:, :, 1]
        qk = sage_core.prequantize_rms_rope_qk(
            q, k, self.cross_norm_q, self.cross_norm_k, None, epsilon=cfg.eps, rot_dim=0,
            tensor_layout="NHD", norm_scope="row")
        state = sage_core.prequantize_sageattn_from_qk(qk, v, sm_scale=cfg.head_dim ** -0.5)
        del q, kv, k, qk
        out = sage_core.sageattn_from_prequantized(state)
        return self._project(self.cross_o, out.reshape(b * l, c), residual, None).view(b, l, c)

    def ffn(self, h, residual: Optional[torch.Tensor] = None,
            gate: Optional[torch.Tensor] = None) -> torch.Tensor:
        b, l, c = h.shape
        up = self.ffn_up(_token_rows(h))
        return self._project(self.ffn_down, up, residual, gate, gelu=True).view(b, l, c)

    def modulation_chunks(self, e: torch.Tensor) -> list[torch.Tensor]:
        """(modulation + e) split into the six [B, 1, C] bf16 rows."""
        mod = (self.modulation + e.to(torch.float32)).to(torch.bfloat16)
        return [mod[:, i:i + 1] for i in range(6)]

    def forward(self, x: torch.Tensor, e: torch.Tensor, context: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
        """x bf16 [B, L, C]; e [B, 6, C] time modulation; context bf16 [B, Lc, C]
        (after the text embedding); freqs [1|B, L, 1, D/2, 2, 2]."""
        cfg = self.cfg
        if x.dtype != torch.bfloat16 or x.dim() != 3 or x.shape[2] != cfg.dim:
            raise TypeError(f"Wan block input must be bf16 [B, L, {cfg.dim}]")
        if context.dtype != torch.bfloat16 or context.dim() != 3 or context.shape[2] != cfg.dim:
            raise TypeError(f"Wan block context must be bf16 [B, Lc, {cfg.dim}]")
        e0, e1, e2, e3, e4, e5 = self.modulation_chunks(e)
        x = x.contiguous()
        b, l, _ = x.shape

        def adaln_codes(x, scale, shift, group):
            codes, rs = torch.ops.turing_utils.layer_norm_adaln_int8_convrot_quantize(x, scale, shift, cfg.eps, group)
            return QuantizedActivation(codes, rs, b, l, group)

        # each norm runs with the next projection's quantizer, each residual
        # add in the epilogue of the projection before it
        x = self.self_attention(adaln_codes(x, e1, e0, self.self_qkv.group), freqs, residual=x, gate=e2)
        codes, rs = torch.ops.turing_utils.layer_norm_affine_int8_convrot_quantize(
            x, self.norm3_weight, self.norm3_bias, cfg.eps, self.cross_q.group)
        x = self.cross_attention(QuantizedActivation(codes, rs, b, l, self.cross_q.group), context, residual=x)
        return self.ffn(adaln_codes(x, e4, e3, self.ffn_up.group), residual=x, gate=e5)

    __call__ = forward


def random_block(cfg: WanBlockConfig, seed: int, device) -> tuple[WanBlockW8A8, WanTextEmbeddingW8A8]:
    """Random-init block and text embedding: every linear weight and bias
    N(0, 0.02) (generated in fp32 on ``device`` with a seeded generator), then
    quantized; RMSNorm weights 1 + N(0, 0.05); norm3 weight 1 + N(0, 0.05) and
    bias N(0, 0.02);
    the modulation table N(0, 1) / sqrt(C) as in Wan's initialisation."""
    device = torch.device(device)
    g = torch.Generator(device=device).manual_seed(seed)
    c, f = cfg.dim, cfg.ffn_dim

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=device)

    def linear(n, k):
        w = randn(n, k) * 0.02
        b = randn(n) * 0.02
        return W8A8Linear.from_float(w, b.to(torch.bfloat16))

    def norm_weight():
        return (1 + 0.05 * randn(c)).to(torch.bfloat16)

    block = WanBlockW8A8(
        cfg,
        modulation=randn(1, 6, c) / math.sqrt(c),
        self_qkv=linear(3 * c, c), self_o=linear(c, c),
        self_norm_q=norm_weight(), self_norm_k=norm_weight(),
        norm3_weight=norm_weight(),
        norm3_bias=randn(c) * 0.02,
        cross_q=linear(c, c), cross_kv=linear(2 * c, c), cross_o=linear(c, c),
        cross_norm_q=norm_weight(), cross_norm_k=norm_weight(),
        ffn_up=linear(f, c), ffn_down=linear(c, f),
    )
    text = WanTextEmbeddingW8A8(linear(c, cfg.text_dim), linear(c, c))
    return block, text


# Wan 2.1 parameter names of one block (the official checkpoint's and
# ComfyUI's): quantized linears and plain tensors, relative to "blocks.{i}.".
_BLOCK_LINEARS = ("self_attn.q", "self_attn.k", "self_attn.v", "self_attn.o", "cross_attn.q", "cross_attn.k",
                  "cross_attn.v", "cross_attn.o", "ffn.0", "ffn.2")
_BLOCK_TENSORS = ("modulation", "self_attn.norm_q.weight", "self_attn.norm_k.weight", "cross_attn.norm_q.weight",
                  "cross_attn.norm_k.weight", "norm3.weight", "norm3.bias")


def block_state(block: WanBlockW8A8, index: int, prefix: str = "") -> tuple[dict, dict]:
    """(W8 linears, plain tensors) of ``block`` under Wan's names for block
    ``index``: the fused q / k / v and k / v GEMMs split back into layers."""
    p = f"{prefix}blocks.{index}."
    q, k, v = block.self_qkv.split(3)
    ck, cv = block.cross_kv.split(2)
    linears = dict(zip((p + n for n in _BLOCK_LINEARS),
                       (q, k, v, block.self_o, block.cross_q, ck, cv, block.cross_o, block.ffn_up, block.ffn_down)))
    tensors = dict(zip((p + n for n in _BLOCK_TENSORS),
                       (block.modulation, block.self_norm_q, block.self_norm_k, block.cross_norm_q,
                        block.cross_norm_k, block.norm3_weight, block.norm3_bias)))
    return linears, tensors


def load_block(path, index: int, cfg: Optional[WanBlockConfig] = None, *, prefix: str = "",
               device="cpu") -> WanBlockW8A8:
    """Block ``index`` of a Wan 2.1 ConvRot W8A8 safetensors checkpoint (its
    W8 layers as the ConvRot metadata describes them, the norms and the
    modulation table as plain tensors), with q / k / v and cross k / v fused."""
    from safetensors import safe_open

    from .convrot_format import load_w8a8_linears

    cfg = cfg or WanBlockConfig()
    p = f"{prefix}blocks.{index}."
    lin = load_w8a8_linears(path, prefix=p, device=device)
    missing = [p + n for n in _BLOCK_LINEARS if p + n not in lin]
    if missing:
        raise ValueError(f"checkpoint has no W8 ConvRot layers {missing}")
    with safe_open(str(path), framework="pt", device="cpu") as f:
        keys = set(f.keys())
        absent = [p + n for n in _BLOCK_TENSORS if p + n not in keys]
        if absent:
            raise ValueError(f"checkpoint has no tensors {absent}")
        t = {n: f.get_tensor(p + n).to(device) for n in _BLOCK_TENSORS}
    L = {n: lin[p + n] for n in _BLOCK_LINEARS}
    return WanBlockW8A8(
        cfg, modulation=t["modulation"],
        self_qkv=W8A8Linear.concat([L["self_attn.q"], L["self_attn.k"], L["self_attn.v"]]), self_o=L["self_attn.o"],
        self_norm_q=t["self_attn.norm_q.weight"], self_norm_k=t["self_attn.norm_k.weight"],
        norm3_weight=t["norm3.weight"], norm3_bias=t["norm3.bias"],
        cross_q=L["cross_attn.q"], cross_kv=W8A8Linear.concat([L["cross_attn.k"], L["cross_attn.v"]]),
        cross_o=L["cross_attn.o"], cross_norm_q=t["cross_attn.norm_q.weight"],
        cross_norm_k=t["cross_attn.norm_k.weight"], ffn_up=L["ffn.0"], ffn_down=L["ffn.2"])


def load_text_embedding(path, *, prefix: str = "", device="cpu") -> WanTextEmbeddingW8A8:
    """Wan's ``text_embedding.0`` / ``text_embedding.2`` W8 layers."""
    from .convrot_format import load_w8a8_linears

    lin = load_w8a8_linears(path, prefix=f"{prefix}text_embedding.", device=device)
    try:
        return WanTextEmbeddingW8A8(lin[f"{prefix}text_embedding.0"], lin[f"{prefix}text_embedding.2"])
    except KeyError as exc:
        raise ValueError(f"checkpoint has no W8 ConvRot layer {exc}") from None


def c5_inputs(text: WanTextEmbeddingW8A8, device, seed: int = 4, grid=(21, 30, 52), text_tokens: int = 512):
    """Synthetic C5 inputs: x bf16 [1, F*H*W, 5120] ~ N(0, 1), the time
    modulation e fp32 [1, 6, 5120] ~ N(0, 0.01), the text context bf16
    [1, 512, 4096] ~ N(0, 1) passed through the text embedding, and the
    rotary table of the latent grid (Wan 2.1 480p, 81 frames: 21 x 30 x 52)."""
    g = torch.Generator(device=device).manual_seed(seed)
    tokens = grid[0] * grid[1] * grid[2]
    x = torch.randn(1, tokens, 5120, generator=g, device=device).to(torch.bfloat16)
    e = 0.1 * torch.randn(1, 6, 5120, generator=g, device=device)
    context = text(torch.randn(1, text_tokens, 4096, generator=g, device=device).to(torch.bfloat16))
    return x, e, context, rope_freqs(grid, 128, device=device)


def block_ops(cfg: WanBlockConfig, tokens: int, text_tokens: int) -> float:
    """Multiply-adds x 2 of one block forward: the seven projections and the
    self / cross attention (4 H L Lk D each)."""
    c, f, m = cfg.dim, cfg.ffn_dim, tokens
    linears = 2.0 * m * c * (3 * c + c + c + c + 2 * f) + 2.0 * text_tokens * c * 2 * c
    attention = 4.0 * cfg.heads * m * (m + text_tokens) * cfg.head_dim
    return linears + attention


def main(argv=None) -> int:
    """Runs the random-init C5 block forward on cuda:0 and prints one JSON
    line (ms per forward, TOPS) -- the workload profiled with rocprofv3."""
    import argparse
    import json

    p = argparse.ArgumentParser(description=main.__doc__)
    p.add_argument("--iters", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    args = p.parse_args(argv)
    dev = torch.device("cuda", 0)
    cfg = WanBlockConfig()
    block, text = random_block(cfg, seed=4, device=dev)
    x, e, context, freqs = c5_inputs(text, dev)
    for _ in range(args.warmup):
        block(x, e, context, freqs)
    torch.cuda.synchronize(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.iters):
        block(x, e, context, freqs)
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end) / args.iters
    ops_ = block_ops(cfg, x.shape[1], context.shape[1])
    print(json.dumps({"workload": "wan14b_block_c5", "ms": ms, "tops": ops_ / ms / 1e9, "iters": args.iters}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
