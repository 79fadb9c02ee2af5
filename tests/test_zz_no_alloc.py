"""tu_sage_kmean_noalloc, the K-mean entry point that allocates nothing (its
chunk sums live in a static device array), against tu_sage_kmean with caller
scratch: bit-identical means on two calls in a row, the second smaller, and
the size limit refused before any launch."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from comfyui_turing_utils_kernel import _lib
from oracle import oracle
from tests import inputs

pytestmark = pytest.mark.gpu

MAX_FLOATS = 1 << 22


def _k(b, h, l, d, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn(b, h, l, d, generator=g, device=dev) + 2 * torch.randn(b, h, 1, d, generator=g, device=dev)
    return k.to(torch.bfloat16)


def _with_scratch(k: torch.Tensor) -> torch.Tensor:
    b, h, l, d = k.shape
    scratch = torch.empty(b * h * ((l + 127) // 128) * d, dtype=torch.float32, device=k.device)
    mean = torch.empty(b, h, d, dtype=torch.bfloat16, device=k.device)
    _lib.call("tu_sage_kmean", k.data_ptr(), b, h, l, d, k.stride(0), k.stride(1), k.stride(2), scratch.data_ptr(),
              mean.data_ptr(), _lib.stream_of(k.device))
    return mean


def _no_alloc(k: torch.Tensor, mean: torch.Tensor) -> None:
    b, h, l, d = k.shape
    _lib.call("tu_sage_kmean_noalloc", k.data_ptr(), b, h, l, d, k.stride(0), k.stride(1), k.stride(2),
              mean.data_ptr(), _lib.stream_of(k.device))


def test_no_alloc_kmean_matches_the_scratch_entry_point(gpu_device):
    # first call: Wan-14B's self-attention K (B1 H40 L32760 D128, 1310720
    # chunk sums); second: a smaller ragged one (B2 H3 L300 D64, NHD view)
    print("[kmean noalloc] B1 H40 L32760 D128, then B2 H3 L300 D64 (NHD)", flush=True)
    big = _k(1, 40, 32760, 128, 1, gpu_device)
    small = _k(2, 300, 3, 64, 2, gpu_device).transpose(1, 2)  # [B, H, L, D] view of NHD storage
    out_big = torch.full((1, 40, 128), -1.0, dtype=torch.bfloat16, device=gpu_device)
    out_small = torch.full((2, 3, 64), -1.0, dtype=torch.bfloat16, device=gpu_device)
    _no_alloc(big, out_big)
    _no_alloc(small, out_small)
    ref_big, ref_small = _with_scratch(big), _with_scratch(small)
    torch.cuda.synchronize(gpu_device)
    assert torch.equal(out_big.view(torch.int16), ref_big.view(torch.int16))
    assert torch.equal(out_small.view(torch.int16), ref_small.view(torch.int16))
    np.testing.assert_array_equal(inputs.bits(out_small), oracle.sage_kmean(inputs.bits(small.contiguous())))
    # the large input again after the small one: the shared array keeps no
    # state that a later call depends on
    again = torch.empty_like(out_big)
    _no_alloc(big, again)
    torch.cuda.synchronize(gpu_device)
    assert torch.equal(again.view(torch.int16), ref_big.view(torch.int16))


def test_no_alloc_kmean_refuses_inputs_beyond_its_scratch(gpu_device):
    k = torch.zeros(1, 1, 64, 128, dtype=torch.bfloat16, device=gpu_device)
    mean = torch.zeros(1, 1, 128, dtype=torch.bfloat16, device=gpu_device)
    # 41 heads x 800 chunks x 128 channels = 4198400 > 2^22 floats: refused on
    # the host before anything is launched (the tiny tensor is never read)
    with pytest.raises(RuntimeError, match="exceeds"):
        _lib.call("tu_sage_kmean_noalloc", k.data_ptr(), 1, 41, 800 * 128, 128, 41 * 800 * 128 * 128,
                  800 * 128 * 128, 128, mean.data_ptr(), _lib.stream_of(gpu_device))
    assert 41 * 800 * 128 > MAX_FLOATS
