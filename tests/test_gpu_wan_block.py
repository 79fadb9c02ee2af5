"""GPU: the Wan 2.1 14B block harness (comfyui_turing_utils_kernel.wan_block)
against an fp32 PyTorch reference of the same block (tests/wan_reference.py:
dequantized weights, unquantized activations, exact softmax).

Each op inside the block is bit-exact or within the attention bar against the
CPU oracle in its own test file; what this file checks is the composition --
modulation chunk order, gates, norm3's affine form, the q / k / v and k / v
splits of the fused GEMMs, the RoPE table and layout, the NHD views fed to the
fused Q/K producer and the attention -- at the C5 dimensions (C 5120, 40 heads
of 128, FFN 13824, text 4096 -> 5120).

Bars.  The remaining error is the activation quantization (INT8 per token in
each W8A8 linear, INT8 Q / K per 16 / 64 tokens, bf16 P.V).  Measured on
MI355X: sublayer rel-L2 0.013-0.014 (cos >= 0.99990), block update rel-L2
0.0126 (1024 tokens) and 0.0121 (C5 rows).  Planted in the fp32 reference,
wiring mistakes give at the sublayer level: RoPE inverted 0.29, RoPE pair
order flipped 0.35; at the block level: norm3 weight dropped 0.0225,
attention shift / scale swapped 0.027, FFN shift / scale swapped 0.039, gates
swapped 0.26, cross k / v swapped 1.42.  Hence the bars: sublayers rel-L2 <=
0.025, the block update rel-L2 <= 0.018 (with the cosines those imply).
"""
from __future__ import annotations

import pytest
import torch

from tests import wan_reference as ref

pytestmark = pytest.mark.gpu

SUBLAYER_REL_MAX = 0.025
BLOCK_REL_MAX = 0.018


@pytest.fixture(scope="module")
def harness(gpu_device):
    from comfyui_turing_utils_kernel.wan_block import WanBlockConfig, random_block

    print("building random-init Wan block (seed 4)", flush=True)
    block, text = random_block(WanBlockConfig(), seed=4, device=gpu_device)
    torch.cuda.synchronize(gpu_device)
    return block, text


def _inputs(block, text, grid, lc, seed, dev):
    from comfyui_turing_utils_kernel.wan_block import rope_freqs

    g = torch.Generator(device=dev).manual_seed(seed)
    l = grid[0] * grid[1] * grid[2]
    x = torch.randn(1, l, 5120, generator=g, device=dev).to(torch.bfloat16)
    e = 0.1 * torch.randn(1, 6, 5120, generator=g, device=dev)
    context_raw = torch.randn(1, lc, 4096, generator=g, device=dev).to(torch.bfloat16)
    context = text(context_raw)
    # bf16 rotation tables, as the fused producer consumes them, for both sides
    freqs = rope_freqs(grid, 128, device=dev).to(torch.bfloat16).float()
    return x, e, context_raw, context, freqs


def _check(name, got, want, rel_max):
    m = ref.metrics(got, want)
    print(f"{name}: {m}", flush=True)
    # cos >= 1 - rel^2 / 2 when the error is uncorrelated with the signal
    assert m["rel_l2"] <= rel_max and m["cos"] >= 1 - rel_max ** 2, (name, m)


def test_sublayers_teacher_forced(harness, gpu_device):
    block, text = harness
    x, e, context_raw, context, freqs = _inputs(block, text, (2, 16, 32), 77, 11, gpu_device)
    lnadaln = torch.ops.turing_utils.layer_norm_adaln
    e0, e1, *_ = block.modulation_chunks(e)
    h = lnadaln(x, e1, e0, 1e-6)
    r = SUBLAYER_REL_MAX
    _check("text_embedding", context, ref.text_embedding(text, context_raw), r)
    _check("self_attention", block.self_attention(h, freqs), ref.self_attention(block, h.float(), freqs), r)
    _check("cross_attention", block.cross_attention(h, context), ref.cross_attention(block, h.float(), context), r)
    _check("ffn", block.ffn(h), ref.ffn(block, h.float()), r)


def test_block_small(harness, gpu_device):
    block, text = harness
    x, e, _, context, freqs = _inputs(block, text, (2, 16, 32), 77, 12, gpu_device)
    out = block(x, e, context, freqs)
    assert out.dtype == torch.bfloat16 and out.shape == x.shape
    want = ref.block_rows(block, x, e, context, freqs)
    _check("block update", out.float() - x.float(), want - x.float(), BLOCK_REL_MAX)


def test_block_c5_sampled_rows(harness, gpu_device):
    """C5: 32760 tokens (grid 21 x 30 x 52), 512 text tokens; the fp32
    reference at 64 sampled rows (first, last, random) with keys / values of
    all tokens."""
    block, text = harness
    print("C5 block forward L=32760 Lc=512", flush=True)
    x, e, _, context, freqs = _inputs(block, text, (21, 30, 52), 512, 13, gpu_device)
    out = block(x, e, context, freqs)
    torch.cuda.synchronize(gpu_device)
    assert torch.isfinite(out).all()
    rows = torch.cat([torch.tensor([0, 32759]),
                      torch.randperm(32760, generator=torch.Generator().manual_seed(5))[:62]]).to(gpu_device)
    want = ref.block_rows(block, x, e, context, freqs, rows)
    _check("C5 block update (rows)", out[:, rows].float() - x[:, rows].float(), want - x[:, rows].float(),
           BLOCK_REL_MAX)


def test_checkpoint_round_trip_forward(harness, gpu_device, tmp_path):
    """The block written as a ConvRot W8A8 checkpoint under Wan's names and
    loaded back runs the same forward, bit for bit."""
    from comfyui_turing_utils_kernel import convrot_format
    from comfyui_turing_utils_kernel.wan_block import block_state, load_block

    block, text = harness
    linears, tensors = block_state(block, 0)
    path = tmp_path / "wan_block0.safetensors"
    convrot_format.save_w8a8_linears(path, linears, tensors)
    loaded = load_block(path, 0, block.cfg, device=gpu_device)
    x, e, _, context, freqs = _inputs(block, text, (2, 16, 32), 77, 14, gpu_device)
    assert torch.equal(loaded(x, e, context, freqs), block(x, e, context, freqs))


def test_batch_of_two(harness, gpu_device):
    """B = 2 with per-sample modulation and text: every view, stride and
    broadcast of the block holds beyond batch 1, and each sample equals the
    block run on it alone."""
    from comfyui_turing_utils_kernel.wan_block import rope_freqs

    block, text = harness
    g = torch.Generator(device=gpu_device).manual_seed(21)
    grid = (1, 16, 16)
    x = torch.randn(2, 256, 5120, generator=g, device=gpu_device).to(torch.bfloat16)
    e = 0.1 * torch.randn(2, 6, 5120, generator=g, device=gpu_device)
    context = text(torch.randn(2, 40, 4096, generator=g, device=gpu_device).to(torch.bfloat16))
    freqs = rope_freqs(grid, 128, device=gpu_device).to(torch.bfloat16).float()
    out = block(x, e, context, freqs)
    want = ref.block_rows(block, x, e, context, freqs)
    _check("block update, B=2", out.float() - x.float(), want - x.float(), BLOCK_REL_MAX)
    for i in range(2):
        alone = block(x[i:i + 1].contiguous(), e[i:i + 1], context[i:i + 1].contiguous(), freqs)
        assert torch.equal(alone, out[i:i + 1]), i


def test_block_norm3_wide_affine_weights(harness, gpu_device):
    """norm3 weights drawn from N(1, 0.5) (negative and sub-0.5 channels, which
    the AdaLN form cannot express) and bias N(0, 0.3): the block still meets
    the composition bar, and dropping norm3's weight in the reference is far
    outside it."""
    import copy

    block, text = harness
    g = torch.Generator(device=gpu_device).manual_seed(31)
    wide = copy.copy(block)
    wide.norm3_weight = (1 + 0.5 * torch.randn(5120, generator=g, device=gpu_device)).to(torch.bfloat16)
    wide.norm3_bias = (0.3 * torch.randn(5120, generator=g, device=gpu_device)).to(torch.bfloat16)
    assert (wide.norm3_weight < 0).any()
    x, e, _, context, freqs = _inputs(block, text, (2, 16, 32), 77, 15, gpu_device)
    out = wide(x, e, context, freqs)
    want = ref.block_rows(wide, x, e, context, freqs)
    _check("block update, wide norm3", out.float() - x.float(), want - x.float(), BLOCK_REL_MAX)
    dropped = copy.copy(wide)
    dropped.norm3_weight = torch.ones_like(wide.norm3_weight)
    bad = ref.metrics(out.float() - x.float(), ref.block_rows(dropped, x, e, context, freqs) - x.float())
    assert bad["rel_l2"] > 2 * BLOCK_REL_MAX, bad
