"""GPU parity: INT8 GEMM accumulators (bit-exact), the BF16 epilogue (bit-exact
vs the oracle's operation order) and dequantize_int8_bf16.

Oracle: or_int8_gemm_i32 (exact integer sum) and or_int8_epilogue_bf16
(w4a8.cu:480-525 operation order: ((acc * as) * ws) + bias, bf16 RNE).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle
from tests import inputs

pytestmark = pytest.mark.gpu


def _rand_i8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-128, 128, shape, generator=g, dtype=torch.int8)


@pytest.mark.parametrize(
    "m,n,k",
    [(1, 8, 16), (7, 24, 48), (256, 256, 64), (300, 264, 192), (513, 520, 1040), (64, 8960, 1536), (40, 512, 13824),
     # 1, 2 and 3 full 128-byte K steps with and without a partial last step (the
     # main loop's last two steps reload the final step), ragged M and N tiles
     (257, 264, 128), (129, 8, 256), (520, 272, 320), (65, 264, 384), (33, 1024, 448), (600, 512, 5120)],
)
def test_gemm_i32_exact(gpu_device, m, n, k):
    print(f"[gemm-i32] m={m} n={n} k={k}", flush=True)
    a = _rand_i8((m, k), m * 7 + n)
    w = _rand_i8((n, k), k * 3 + 1)
    acc = torch.ops.turing_utils.int8_gemm_i32(a.to(gpu_device), w.to(gpu_device))
    torch.cuda.synchronize(gpu_device)
    ref = oracle.int8_gemm_i32(a.numpy(), w.numpy())
    np.testing.assert_array_equal(acc.cpu().numpy(), ref)


def test_gemm_i32_extremes(gpu_device):
    """All -128 times -128 at K=13824: the largest accumulator this path can see."""
    m, n, k = 32, 16, 13824
    a = torch.full((m, k), -128, dtype=torch.int8)
    w = torch.full((n, k), -128, dtype=torch.int8)
    acc = torch.ops.turing_utils.int8_gemm_i32(a.to(gpu_device), w.to(gpu_device)).cpu()
    assert int(acc.min()) == int(acc.max()) == 16384 * k


def test_gemm_i32_activation_past_2gib(gpu_device):
    """An activation of more than 2^31 bytes (160000 x 13824, about 2.2 GB):
    every operand offset the kernel forms is relative to a 256-row panel, so
    nothing overflows 32 bits.  Rows across the whole range (first, last,
    panel edges) are checked bit-exact against the oracle."""
    m, n, k = 160000, 264, 13824
    assert m * k > 2**31
    print(f"[gemm-i32 >2GiB] m={m} n={n} k={k}", flush=True)
    g = torch.Generator(device=gpu_device).manual_seed(11)
    a = torch.randint(-128, 128, (m, k), generator=g, dtype=torch.int8, device=gpu_device)
    w = _rand_i8((n, k), 12)
    acc = torch.ops.turing_utils.int8_gemm_i32(a, w.to(gpu_device))
    rows = torch.tensor([0, 1, 255, 256, 77777, 155391, 155392, m - 257, m - 2, m - 1])
    a_rows = a[rows.to(gpu_device)].cpu()
    got = acc[rows.to(gpu_device)].cpu().numpy()
    del a, acc
    torch.cuda.synchronize(gpu_device)
    np.testing.assert_array_equal(got, oracle.int8_gemm_i32(a_rows.numpy(), w.numpy()))


@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("m,n,k", [(300, 264, 192), (96, 8960, 1536)])
def test_int8_linear_epilogue_exact(gpu_device, m, n, k, with_bias):
    print(f"[int8_linear] m={m} n={n} k={k} bias={with_bias}", flush=True)
    a = _rand_i8((m, k), 5 + m)
    w, ws, bias = inputs.weights(n, k, 9, with_bias)
    g = torch.Generator().manual_seed(3)
    as_ = torch.empty(m).uniform_(1e-3, 1e-1, generator=g)
    out = torch.ops.turing_utils.int8_linear(
        a.to(gpu_device), w.to(gpu_device), as_.to(gpu_device), ws.to(gpu_device),
        None if bias is None else bias.to(gpu_device),
    )
    torch.cuda.synchronize(gpu_device)
    acc = oracle.int8_gemm_i32(a.numpy(), w.numpy())
    ref = oracle.epilogue_bf16(acc, as_.numpy(), ws.numpy(), None if bias is None else bias.numpy())
    got = inputs.bits(out)
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"{len(bad)} outputs differ, first {bad[:5].tolist()}"


def test_int8_linear_epilogue_nonfinite_scales(gpu_device):
    """Waves whose scales and bias are finite (with nonzero column scales)
    round on the hardware conversion, the others in software; both must give
    the oracle's bits, canonical 0x7fff NaN included.  Row 70's scale
    overflows the product to +-inf (a finite-scale wave: inf stays inf); row
    200's meets a zero and a -0 column scale (inf * 0 = NaN); NaN and inf
    sit in a row scale, a column scale and the bias."""
    m, n, k = 300, 520, 192
    print(f"[int8_linear nonfinite] m={m} n={n} k={k}", flush=True)
    a = _rand_i8((m, k), 41)
    w, ws, bias = inputs.weights(n, k, 43, True)
    g = torch.Generator().manual_seed(5)
    as_ = torch.empty(m).uniform_(1e-3, 1e-1, generator=g)
    as_[5] = float("nan")
    as_[70] = 3.0e38
    as_[200] = 1.0e37
    as_[260] = float("-inf")
    ws[300] = 0.0
    ws[301] = -0.0
    ws[400] = float("inf")
    ws[513] = float("nan")
    bias = bias.clone()
    bias[450] = float("nan")
    bias[460] = float("-inf")
    for b in (bias, None):
        out = torch.ops.turing_utils.int8_linear(
            a.to(gpu_device), w.to(gpu_device), as_.to(gpu_device), ws.to(gpu_device),
            None if b is None else b.to(gpu_device))
        torch.cuda.synchronize(gpu_device)
        acc = oracle.int8_gemm_i32(a.numpy(), w.numpy())
        ref = oracle.epilogue_bf16(acc, as_.numpy(), ws.numpy(), None if b is None else b.numpy())
        got = inputs.bits(out)
        assert (ref == 0x7FFF).any() and ((ref & 0x7FFF) == 0x7F80).any()
        bad = np.argwhere(got != ref)
        assert bad.size == 0, f"bias={b is not None}: {len(bad)} outputs differ, first {bad[:5].tolist()}"


@pytest.mark.parametrize("gate_rows", [None, 1, 37])
@pytest.mark.parametrize("m,n,k,with_bias", [(300, 264, 192, True), (257, 520, 1040, False), (96, 5120, 1536, True)])
def test_int8_linear_residual_exact(gpu_device, m, n, k, with_bias, gate_rows):
    """The gated residual epilogue: bf16_rn(fma(y, gate[i // gate_rows], residual)) with
    y the bf16 epilogue output; ragged M and N tiles, ungated and per-row / per-block gates."""
    print(f"[int8_linear_residual] m={m} n={n} k={k} bias={with_bias} gate_rows={gate_rows}", flush=True)
    a = _rand_i8((m, k), 11 + m)
    w, ws, bias = inputs.weights(n, k, 4, with_bias)
    g = torch.Generator().manual_seed(8)
    as_ = torch.empty(m).uniform_(1e-3, 1e-1, generator=g)
    residual = (torch.randn(m, n, generator=g) * 4).to(torch.bfloat16)
    gate = None
    if gate_rows is not None:
        gate = torch.empty((m + gate_rows - 1) // gate_rows, n).uniform_(-2, 2, generator=g).to(torch.bfloat16)
    dev = gpu_device
    res_dev = residual.to(dev)
    out = torch.ops.turing_utils.int8_linear_residual(
        a.to(dev), w.to(dev), as_.to(dev), ws.to(dev), None if bias is None else bias.to(dev),
        res_dev, None if gate is None else gate.to(dev), 1 if gate_rows is None else gate_rows,
    )
    torch.cuda.synchronize(dev)
    acc = oracle.int8_gemm_i32(a.numpy(), w.numpy())
    y = oracle.epilogue_bf16(acc, as_.numpy(), ws.numpy(), None if bias is None else bias.numpy())
    ref = oracle.residual_gate_bf16(y, inputs.bits(residual), None if gate is None else inputs.bits(gate),
                                    1 if gate_rows is None else gate_rows)
    got = inputs.bits(out)
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"{len(bad)} outputs differ, first {bad[:5].tolist()}"
    np.testing.assert_array_equal(inputs.bits(res_dev), inputs.bits(residual))


def test_residual_and_bf16_on_192_wide_tiles(gpu_device):
    """A grid that the tile policy runs on 256 x 192 tiles (2048 x 8968: two
    rounds of them on 256 CUs, a ragged last 192-wide tile): the bf16 output
    and the gated residual epilogue, 96 sampled rows bit-exact against the
    oracle."""
    from comfyui_turing_utils_kernel import _lib

    m, n, k, gate_rows = 2048, 8968, 256, 16
    print(f"[gemm 256x192] m={m} n={n} k={k} policy={_lib.load().tu_int8_gemm_tile_policy(m, n, 256)}", flush=True)
    assert _lib.load().tu_int8_gemm_tile_policy(m, n, 256) == 3
    a = _rand_i8((m, k), 5)
    w, ws, bias = inputs.weights(n, k, 6, True)
    g = torch.Generator().manual_seed(9)
    as_ = torch.empty(m).uniform_(1e-3, 1e-1, generator=g)
    residual = (torch.randn(m, n, generator=g) * 4).to(torch.bfloat16)
    gate = torch.empty(m // gate_rows, n).uniform_(-2, 2, generator=g).to(torch.bfloat16)
    dev = gpu_device
    ad, wd, asd, wsd, bd = a.to(dev), w.to(dev), as_.to(dev), ws.to(dev), bias.to(dev)
    y_dev = torch.ops.turing_utils.int8_linear(ad, wd, asd, wsd, bd)
    out = torch.ops.turing_utils.int8_linear_residual(ad, wd, asd, wsd, bd, residual.to(dev), gate.to(dev), gate_rows)
    torch.cuda.synchronize(dev)
    rows = np.sort(np.random.default_rng(4).choice(m, 96, replace=False))
    acc = oracle.int8_gemm_i32(a.numpy()[rows], w.numpy())
    y = oracle.epilogue_bf16(acc, as_.numpy()[rows], ws.numpy(), bias.numpy())
    np.testing.assert_array_equal(inputs.bits(y_dev)[rows], y)
    ref = oracle.residual_gate_bf16(y, inputs.bits(residual)[rows], inputs.bits(gate)[rows // gate_rows], 1)
    np.testing.assert_array_equal(inputs.bits(out)[rows], ref)


@pytest.mark.parametrize("gate_rows", [None, 37])
@pytest.mark.parametrize("m,n,k", [(300, 264, 192), (257, 520, 1040), (513, 776, 1536)])
def test_residual_in_place_through_the_c_abi(gpu_device, m, n, k, gate_rows):
    """tu_int8_gemm_bf16_residual with out == residual (the header allows it):
    bit-exact against the oracle on ragged M / N tiles."""
    from comfyui_turing_utils_kernel import _lib

    print(f"[int8_gemm_bf16_residual in place] m={m} n={n} k={k} gate_rows={gate_rows}", flush=True)
    a = _rand_i8((m, k), 21 + m)
    w, ws, bias = inputs.weights(n, k, 6, True)
    g = torch.Generator().manual_seed(9)
    as_ = torch.empty(m).uniform_(1e-3, 1e-1, generator=g)
    residual = (torch.randn(m, n, generator=g) * 4).to(torch.bfloat16)
    gate = None
    if gate_rows is not None:
        gate = torch.empty((m + gate_rows - 1) // gate_rows, n).uniform_(-2, 2, generator=g).to(torch.bfloat16)
    dev = gpu_device
    ad, wd, asd, wsd, bd = a.to(dev), w.to(dev), as_.to(dev), ws.to(dev), bias.to(dev)
    buf = residual.to(dev)
    gd = None if gate is None else gate.to(dev)
    with torch.cuda.device(dev):
        _lib.call("tu_int8_gemm_bf16_residual", ad.data_ptr(), wd.data_ptr(), asd.data_ptr(), wsd.data_ptr(),
                  bd.data_ptr(), buf.data_ptr(), _lib.ptr(gd), 1 if gate_rows is None else gate_rows,
                  buf.data_ptr(), m, n, k, _lib.stream_of(dev))
    torch.cuda.synchronize(dev)
    y = oracle.epilogue_bf16(oracle.int8_gemm_i32(a.numpy(), w.numpy()), as_.numpy(), ws.numpy(), bias.numpy())
    ref = oracle.residual_gate_bf16(y, inputs.bits(residual), None if gate is None else inputs.bits(gate),
                                    1 if gate_rows is None else gate_rows)
    bad = np.argwhere(inputs.bits(buf) != ref)
    assert bad.size == 0, f"{len(bad)} outputs differ, first {bad[:5].tolist()}"


def test_int8_linear_config1_rows(gpu_device):
    """BASELINE config 1 through the drop-in ops (quantize G=128, then int8_linear);
    128 sampled rows checked bit-exact against the oracle chain."""
    x = inputs.activation(4096, 1536, 0)
    w, ws, bias = inputs.weights(8960, 1536, 0)
    dev = gpu_device
    q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(x.to(dev), 128)
    out = torch.ops.turing_utils.int8_linear(q, w.to(dev), s, ws.to(dev), bias.to(dev))
    torch.cuda.synchronize(dev)
    rows = np.sort(np.random.default_rng(0).choice(4096, 128, replace=False))
    q_ref, s_ref = oracle.convrot_quant(inputs.bits(x[rows]), 128)
    np.testing.assert_array_equal(q.cpu().numpy()[rows], q_ref)
    acc = oracle.int8_gemm_i32(q_ref, w.numpy())
    ref = oracle.epilogue_bf16(acc, s_ref, ws.numpy(), bias.numpy())
    np.testing.assert_array_equal(inputs.bits(out)[rows], ref)


@pytest.mark.parametrize("cols,scalar", [(264, False), (200, False), (264, True), (131, False)])
def test_dequantize_exact(gpu_device, cols, scalar):
    m, ld = 37, 264
    g = torch.Generator().manual_seed(cols)
    acc = torch.randint(-(2**30), 2**30, (m, ld), generator=g, dtype=torch.int32)
    as_ = torch.empty(m).uniform_(1e-4, 1e-2, generator=g)
    ws = torch.empty(1 if scalar else cols).uniform_(1e-3, 5e-3, generator=g)
    out = torch.ops.turing_utils.dequantize_int8_bf16(acc.to(gpu_device), as_.to(gpu_device), ws.to(gpu_device), cols)
    ref = oracle.epilogue_bf16(acc.numpy(), as_.numpy(), ws.numpy(), None, cols=cols)
    np.testing.assert_array_equal(inputs.bits(out), ref)


def _linear_out_check(got: torch.Tensor, acc, as_, ws, bias, out_dtype):
    """Bit-exact comparison of int8_linear_out against the oracle's fp16 / fp32
    epilogue (fp32: NaN positions, bits elsewhere)."""
    b = None if bias is None else bias.numpy()
    if out_dtype == torch.float16:
        ref = oracle.epilogue_f16(acc, as_.numpy(), ws.numpy(), b)
        g = got.cpu().view(torch.int16).numpy().view(np.uint16)
        bad = np.argwhere(g != ref)
    else:
        ref = oracle.epilogue_f32(acc, as_.numpy(), ws.numpy(), b)
        g = got.cpu().numpy()
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(g), nan)
        bad = np.argwhere((g.view(np.uint32) != ref.view(np.uint32)) & ~nan)
    assert bad.size == 0, f"{len(bad)} outputs differ, first {bad[:5].tolist()}"


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("with_bias", [True, False])
@pytest.mark.parametrize("m,n,k", [(300, 264, 192), (96, 8960, 1536), (513, 520, 1040)])
def test_int8_linear_out_exact(gpu_device, m, n, k, with_bias, out_dtype):
    """int8_linear_out: the epilogue value rounded once to fp16 (not through
    bf16), or kept in fp32, bit-exact against the oracle on ragged tiles."""
    print(f"[int8_linear_out] m={m} n={n} k={k} bias={with_bias} {out_dtype}", flush=True)
    a = _rand_i8((m, k), 15 + m)
    w, ws, bias = inputs.weights(n, k, 19, with_bias)
    g = torch.Generator().manual_seed(13)
    as_ = torch.empty(m).uniform_(1e-3, 1e-1, generator=g)
    dev = gpu_device
    out = torch.ops.turing_utils.int8_linear_out(a.to(dev), w.to(dev), as_.to(dev), ws.to(dev),
                                                 None if bias is None else bias.to(dev), out_dtype)
    torch.cuda.synchronize(dev)
    assert out.dtype == out_dtype and out.shape == (m, n)
    _linear_out_check(out, oracle.int8_gemm_i32(a.numpy(), w.numpy()), as_, ws, bias, out_dtype)


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_int8_linear_out_edges(gpu_device, out_dtype):
    """fp16 overflow to +-inf, the 65504 rounding boundary, fp16 subnormals,
    and non-finite scales and bias (NaN written as 0x7e00 in fp16), on both
    the hardware-rounding waves and the guarded ones."""
    m, n, k = 300, 520, 192
    print(f"[int8_linear_out edges] {out_dtype}", flush=True)
    a = _rand_i8((m, k), 47)
    w, ws, bias = inputs.weights(n, k, 53, True)
    g = torch.Generator().manual_seed(7)
    as_ = torch.empty(m).uniform_(1e-3, 1e-1, generator=g)
    as_[10] = 40.0        # |y| in the thousands to past 65520: fp16 +-inf
    as_[11] = 1e-7        # fp16 subnormals and zeros
    as_[12] = 4e-9
    as_[100] = float("nan")
    as_[200] = float("inf")
    ws[30] = 0.0
    ws[300] = float("-inf")
    bias = bias.clone()
    bias[40] = float("nan")
    dev = gpu_device
    acc = oracle.int8_gemm_i32(a.numpy(), w.numpy())
    for b in (None, bias):
        out = torch.ops.turing_utils.int8_linear_out(a.to(dev), w.to(dev), as_.to(dev), ws.to(dev),
                                                     None if b is None else b.to(dev), out_dtype)
        torch.cuda.synchronize(dev)
        _linear_out_check(out, acc, as_, ws, b, out_dtype)
    if out_dtype == torch.float16:
        h = out.cpu().float()
        assert torch.isinf(h).any() and (h[11].abs() < 6.1e-5).any() and torch.isnan(h).any()


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.float32])
def test_int8_linear_out_config1_rows(gpu_device, out_dtype):
    """Config 1 (4096 x 1536 -> 8960 with bias) in fp16 and fp32: 128 sampled
    rows bit-exact; the bf16 op's output equals the fp32 output rounded to
    bf16 everywhere."""
    x = inputs.activation(4096, 1536, 0)
    w, ws, bias = inputs.weights(8960, 1536, 0)
    dev = gpu_device
    q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(x.to(dev), 128)
    out = torch.ops.turing_utils.int8_linear_out(q, w.to(dev), s, ws.to(dev), bias.to(dev), out_dtype)
    bf = torch.ops.turing_utils.int8_linear(q, w.to(dev), s, ws.to(dev), bias.to(dev))
    torch.cuda.synchronize(dev)
    rows = np.sort(np.random.default_rng(1).choice(4096, 128, replace=False))
    acc = oracle.int8_gemm_i32(q.cpu().numpy()[rows], w.numpy())
    _linear_out_check(out[torch.from_numpy(rows).to(dev)], acc, s.cpu().reshape(-1)[rows], ws, bias, out_dtype)
    if out_dtype == torch.float32:
        assert torch.equal(out.to(torch.bfloat16), bf)


OUT_TYPES = {"bf16": (0, torch.bfloat16), "f16": (1, torch.float16), "f32": (2, torch.float32), "i32": (3, torch.int32)}


@pytest.mark.parametrize("policy", [1, 2, 3])
@pytest.mark.parametrize("out", sorted(OUT_TYPES))
@pytest.mark.parametrize("m,n,k", [(1, 8, 16), (129, 8, 256), (300, 264, 192), (513, 520, 1040), (257, 264, 384),
                                   (200, 1024, 5120)])
def test_gemm_tile_policies_exact(gpu_device, m, n, k, out, policy):
    """tu_int8_gemm_ex with each tile policy forced (1: 256 x 256 tiles, 2:
    128 x 256, 3: 256 x 192) and each output type: bit-exact against the
    oracle on ragged M and N tiles (N 264 and 1024 leave a 192-wide tile
    partly or one wave's half of it wholly empty), partial last K steps and
    one-tile grids."""
    from comfyui_turing_utils_kernel import _lib

    print(f"[gemm ex] m={m} n={n} k={k} out={out} policy={policy}", flush=True)
    code, dtype = OUT_TYPES[out]
    a = _rand_i8((m, k), 3 * m + k)
    w, ws, bias = inputs.weights(n, k, 23, True)
    g = torch.Generator().manual_seed(m)
    as_ = torch.empty(m).uniform_(1e-3, 1e-1, generator=g)
    dev = gpu_device
    ad, wd, asd, wsd, bd = a.to(dev), w.to(dev), as_.to(dev), ws.to(dev), bias.to(dev)
    res = torch.empty((m, n), dtype=dtype, device=dev)
    with torch.cuda.device(dev):
        _lib.call("tu_int8_gemm_ex", ad.data_ptr(), wd.data_ptr(), asd.data_ptr(), wsd.data_ptr(), bd.data_ptr(),
                  res.data_ptr(), code, m, n, k, policy, _lib.stream_of(dev))
    torch.cuda.synchronize(dev)
    acc = oracle.int8_gemm_i32(a.numpy(), w.numpy())
    if out == "i32":
        np.testing.assert_array_equal(res.cpu().numpy(), acc)
    elif out == "bf16":
        np.testing.assert_array_equal(inputs.bits(res), oracle.epilogue_bf16(acc, as_.numpy(), ws.numpy(), bias.numpy()))
    else:
        _linear_out_check(res, acc, as_, ws, bias, dtype)


@pytest.mark.parametrize("policy", [1, 2, 3])
def test_gemm_tile_policies_config1(gpu_device, policy):
    """Config 1 (4096 x 1536 -> 8960, bias) with each tile policy: identical
    bf16 output, 128 sampled rows bit-exact against the oracle."""
    from comfyui_turing_utils_kernel import _lib

    x = inputs.activation(4096, 1536, 0)
    w, ws, bias = inputs.weights(8960, 1536, 0)
    dev = gpu_device
    q, s = torch.ops.turing_utils.bf16_int8_convrot_quantize(x.to(dev), 128)
    wd, wsd, bd = w.to(dev), ws.to(dev), bias.to(dev)
    out = torch.empty((4096, 8960), dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        _lib.call("tu_int8_gemm_ex", q.data_ptr(), wd.data_ptr(), s.data_ptr(), wsd.data_ptr(), bd.data_ptr(),
                  out.data_ptr(), 0, 4096, 8960, 1536, policy, _lib.stream_of(dev))
    ref_op = torch.ops.turing_utils.int8_linear(q, wd, s, wsd, bd)
    torch.cuda.synchronize(dev)
    assert torch.equal(out, ref_op)
    rows = np.sort(np.random.default_rng(2).choice(4096, 128, replace=False))
    acc = oracle.int8_gemm_i32(q.cpu().numpy()[rows], w.numpy())
    ref = oracle.epilogue_bf16(acc, s.cpu().numpy().reshape(-1)[rows], ws.numpy(), bias.numpy())
    np.testing.assert_array_equal(inputs.bits(out)[rows], ref)
