"""fp32 PyTorch reference of the Wan block harness (test infrastructure).

Same block as comfyui_turing_utils_kernel.wan_block, computed in fp32 with
dequantized weights (codes x per-channel scale, rotated back to the original
basis with the dense ConvRot group matrix built from the CPU oracle),
unquantized activations and exact softmax attention.  Cross-token work is
confined to the self-attention, so the block output of any subset of rows can
be computed from keys / values of all tokens plus the rows' own queries --
which is how the full 32760-token shape is checked.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle

_ROT = {}


def rotation(device, group: int = 128) -> torch.Tensor:
    """M with rot(v) = v @ M for one group (orthogonal and symmetric)."""
    key = (str(device), group)
    if key not in _ROT:
        m = np.stack([oracle.rotate_group(r, group) for r in np.eye(group, dtype=np.float32)])
        _ROT[key] = torch.from_numpy(m).to(device)
    return _ROT[key]


def dense_weight(lin) -> torch.Tensor:
    """fp32 W [N, K] in the original basis: rot(W) = codes * scale, so W = (codes * scale) @ M^T."""
    if getattr(lin, "_ref_dense", None) is None:
        w = lin.weight.float() * lin.weight_scale[:, None]
        n, k = w.shape
        m = rotation(w.device, lin.group)
        lin._ref_dense = (w.view(n, k // lin.group, lin.group) @ m.T).reshape(n, k)
    return lin._ref_dense


def linear(x: torch.Tensor, lin, gelu: bool = False) -> torch.Tensor:
    if gelu:
        x = torch.nn.functional.gelu(x, approximate="tanh")
    y = x @ dense_weight(lin).T
    return y if lin.bias is None else y + lin.bias


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w.float()


def rope(x: torch.Tensor, freqs: torch.Tensor) -> torch.Tensor:
    """x [B, L, H, D]; freqs [1|B, L, 1, D/2, 2, 2]: each interleaved pair times its matrix."""
    b, l, h, d = x.shape
    pairs = x.reshape(b, l, h, d // 2, 2)
    f = freqs.float()
    out = f[..., 0] * pairs[..., 0:1] + f[..., 1] * pairs[..., 1:2]
    return out.reshape(b, l, h, d)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, chunk: int = 1024) -> torch.Tensor:
    """q [B, Lq, H, D], k / v [B, Lk, H, D] fp32 -> [B, Lq, H, D], exact softmax."""
    scale = q.shape[-1] ** -0.5
    kt = k.permute(0, 2, 3, 1)  # B H D Lk
    vh = v.permute(0, 2, 1, 3)  # B H Lk D
    outs = []
    for s in range(0, q.shape[1], chunk):
        qc = q[:, s:s + chunk].permute(0, 2, 1, 3)  # B H c D
        p = torch.softmax((qc @ kt) * scale, dim=-1)
        outs.append((p @ vh).permute(0, 2, 1, 3))
    return torch.cat(outs, 1)


def layer_norm(x: torch.Tensor, eps: float) -> torch.Tensor:
    return torch.nn.functional.layer_norm(x.float(), (x.shape[-1],), eps=eps)


def modulation(block, e: torch.Tensor) -> list[torch.Tensor]:
    mod = block.modulation + e.float()
    return [mod[:, i:i + 1] for i in range(6)]


def self_attention(block, h: torch.Tensor, freqs: torch.Tensor, rows=None) -> torch.Tensor:
    """h fp32 [B, L, C] (all tokens); output rows ``rows`` (all when None)."""
    cfg = block.cfg
    b, l, c = h.shape
    w = dense_weight(block.self_qkv)
    bias = block.self_qkv.bias
    hq = h if rows is None else h[:, rows]
    fq = freqs if rows is None else freqs[:, rows]
    q = hq @ w[:c].T + bias[:c]
    k = h @ w[c:2 * c].T + bias[c:2 * c]
    v = h @ w[2 * c:].T + bias[2 * c:]
    q = rope(rms_norm(q, block.self_norm_q, cfg.eps).view(b, -1, cfg.heads, cfg.head_dim), fq)
    k = rope(rms_norm(k, block.self_norm_k, cfg.eps).view(b, l, cfg.heads, cfg.head_dim), freqs)
    o = attention(q, k, v.view(b, l, cfg.heads, cfg.head_dim))
    return linear(o.reshape(b, -1, c), block.self_o)


def cross_attention(block, h: torch.Tensor, context: torch.Tensor) -> torch.Tensor:
    cfg = block.cfg
    b, l, c = h.shape
    lc = context.shape[1]
    q = rms_norm(linear(h, block.cross_q), block.cross_norm_q, cfg.eps).view(b, l, cfg.heads, cfg.head_dim)
    kv = linear(context.float(), block.cross_kv)
    k = rms_norm(kv[..., :c], block.cross_norm_k, cfg.eps).view(b, lc, cfg.heads, cfg.head_dim)
    v = kv[..., c:].reshape(b, lc, cfg.heads, cfg.head_dim)
    return linear(attention(q, k, v).reshape(b, l, c), block.cross_o)


def ffn(block, h: torch.Tensor) -> torch.Tensor:
    return linear(linear(h, block.ffn_up), block.ffn_down, gelu=True)


def text_embedding(text, context: torch.Tensor) -> torch.Tensor:
    return linear(linear(context.float(), text.fc1), text.fc2, gelu=True)


def block_rows(block, x: torch.Tensor, e: torch.Tensor, context: torch.Tensor, freqs: torch.Tensor,
               rows=None) -> torch.Tensor:
    """The block output at ``rows`` (fp32), every intermediate unrounded."""
    cfg = block.cfg
    e0, e1, e2, e3, e4, e5 = modulation(block, e)
    xf = x.float()
    h = layer_norm(xf, cfg.eps) * (1 + e1) + e0
    xr = xf if rows is None else xf[:, rows]
    xr = xr + self_attention(block, h, freqs, rows) * e2
    xr = xr + cross_attention(block, layer_norm(xr, cfg.eps) * block.norm3_weight.float() + block.norm3_bias.float(),
                              context)
    return xr + ffn(block, layer_norm(xr, cfg.eps) * (1 + e4) + e3) * e5


def metrics(got: torch.Tensor, ref: torch.Tensor) -> dict:
    g, r = got.double().flatten(), ref.double().flatten()
    return {
        "cos": float(torch.nn.functional.cosine_similarity(g, r, dim=0)),
        "rel_l2": float((g - r).norm() / r.norm()),
        "max_abs": float((g - r).abs().max()),
    }
