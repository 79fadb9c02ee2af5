"""Host-side checks of the Wan block harness (no GPU: nothing here launches)."""
from __future__ import annotations

import pytest
import torch

from comfyui_turing_utils_kernel.wan_block import W8A8Linear, WanBlockConfig, WanBlockW8A8, rope_freqs


def _kwargs(c=256, f=512):
    def lin(n, k):
        return W8A8Linear(torch.zeros(n, k, dtype=torch.int8), torch.ones(n), None)

    ones = torch.ones(c)
    return dict(modulation=torch.zeros(1, 6, c), self_qkv=lin(3 * c, c), self_o=lin(c, c), self_norm_q=ones,
                self_norm_k=ones, norm3_bias=ones * 0, cross_q=lin(c, c), cross_kv=lin(2 * c, c), cross_o=lin(c, c),
                cross_norm_q=ones, cross_norm_k=ones, ffn_up=lin(f, c), ffn_down=lin(c, f))


CFG = WanBlockConfig(dim=256, heads=2, ffn_dim=512, text_dim=256)


def test_norm3_takes_any_affine_weight():
    """norm3 is a plain affine LayerNorm: weights below 0.5, negative or
    not of the form 1 + a bf16 value (129 / 512 is one) are kept as given."""
    w = torch.tensor([0.251953125, -0.3, 0.01, -3.5, 1.25, 0.0] * 43)[:256]
    block = WanBlockW8A8(CFG, norm3_weight=w, **_kwargs())
    assert torch.equal(block.norm3_weight, w.to(torch.bfloat16))
    assert block.norm3_bias.shape == (256,)


def test_linear_shapes_and_inputs_are_checked():
    kw = _kwargs()
    kw["ffn_down"] = W8A8Linear(torch.zeros(256, 256, dtype=torch.int8), torch.ones(256), None)
    with pytest.raises(ValueError, match="linear shape"):
        WanBlockW8A8(CFG, norm3_weight=torch.ones(256), **kw)
    block = WanBlockW8A8(CFG, norm3_weight=torch.ones(256), **_kwargs())
    x = torch.zeros(1, 8, 256, dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="input"):
        block(x.float(), torch.zeros(1, 6, 256), x, rope_freqs((1, 2, 4), 128))
    with pytest.raises(TypeError, match="context"):
        block(x, torch.zeros(1, 6, 256), x[..., :128], rope_freqs((1, 2, 4), 128))


def test_rope_table():
    """Wan's split of 128 channels: 44 temporal, 42 + 42 spatial (22 + 21 + 21
    pairs); rotation matrices with cos on the diagonal; token (0, 0, 0) is the
    identity; the temporal angle of frame f pair 0 is f."""
    t = rope_freqs((3, 2, 5), 128).double()
    assert t.shape == (1, 30, 1, 64, 2, 2)
    assert torch.allclose(t[0, 0, 0], torch.eye(2, dtype=torch.float64).expand(64, 2, 2))
    assert torch.allclose(t[..., 0, 0], t[..., 1, 1]) and torch.allclose(t[..., 0, 1], -t[..., 1, 0])
    det = t[..., 0, 0] * t[..., 1, 1] - t[..., 0, 1] * t[..., 1, 0]
    assert torch.allclose(det, torch.ones_like(det), atol=1e-6)
    # token index = (f * 2 + h) * 5 + w
    frame2 = t[0, 2 * 10, 0]
    assert abs(frame2[0, 1, 0] - torch.sin(torch.tensor(2.0, dtype=torch.float64))) < 1e-6
    assert torch.allclose(frame2[22:], torch.eye(2, dtype=torch.float64).expand(42, 2, 2))
    w3 = t[0, 3, 0]  # f 0, h 0, w 3: only the last 21 pairs rotate
    assert torch.allclose(w3[:43], torch.eye(2, dtype=torch.float64).expand(43, 2, 2))
    assert abs(w3[43, 1, 0] - torch.sin(torch.tensor(3.0, dtype=torch.float64))) < 1e-6


def test_quantized_activation_must_match_the_linear():
    """A projection fed the codes of a fused norm + quantizer refuses codes of
    another width or ConvRot group, and a GELU request (the codes are already
    made), before any launch."""
    from comfyui_turing_utils_kernel.wan_block import QuantizedActivation

    lin = W8A8Linear(torch.zeros(512, 256, dtype=torch.int8), torch.ones(512), None)
    codes, scale = torch.zeros(8, 256, dtype=torch.int8), torch.ones(8, 1)
    assert QuantizedActivation(codes, scale, 1, 8, 128).shape == (1, 8, 256)
    for bad, kw in ((QuantizedActivation(codes, scale, 1, 8, 256), {}),
                    (QuantizedActivation(codes[:, :128], scale, 1, 8, 128), {}),
                    (QuantizedActivation(codes, scale, 1, 8, 128), {"gelu": True})):
        with pytest.raises(ValueError, match="expects codes"):
            lin(bad, **kw)
