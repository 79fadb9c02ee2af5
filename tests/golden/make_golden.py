"""Writes tests/golden/kat.npz: known-answer vectors for every hot-path function,
derived here in plain numpy/torch, independently of the C oracle.

Inputs are chosen so that each derivation is exact where the specification is
exact: activations and K are small multiples of powers of two, so the
block-Hadamard butterflies, the K channel sums and the int8 products carry no
rounding and any summation order gives the same bits.  The rotation is taken
from the dense Kronecker matrix of R4 (convrot_quant.cu:104-116), not from the
staged butterflies the oracle and the kernel use.

Run from the repository root:  python tests/golden/make_golden.py
The reference package is neither imported nor read.
"""
from __future__ import annotations

import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kat.npz")

R4 = 0.5 * np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], np.float64)
C = np.float64(np.float32(0.70710678118654752440))
BF16_MAX = np.float32(3.38953139e38)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bf16_val(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def rotate(x: np.ndarray, group: int) -> np.ndarray:
    """fp32 rotation of the rows of x (exact for the chosen inputs)."""
    r3 = np.kron(R4, np.kron(R4, R4))  # digits of stride 16, 4, 1
    m, k = x.shape
    g = x.astype(np.float64).reshape(m, k // group, group)
    if group == 256:
        y = g @ np.kron(R4, r3).T
        return y.astype(np.float32).reshape(m, k)
    z = g.reshape(m, k // group, 2, 64) @ r3.T  # R4 (x) R4 (x) R4 on the low 64
    top = np.stack([z[:, :, 0] + z[:, :, 1], z[:, :, 0] - z[:, :, 1]], axis=2)  # exact
    return (top.astype(np.float32).astype(np.float64) * C).astype(np.float32).reshape(m, k)


def convrot_quant(x_bits: np.ndarray, group: int):
    y = rotate(bf16_val(x_bits), group)
    absmax = np.abs(y).max(axis=1)
    scale = np.maximum(np.minimum(absmax, BF16_MAX) / np.float32(127), np.float32(1e-30)).astype(np.float32)
    yb = bf16_val(bf16_bits(y))
    sb = bf16_val(bf16_bits(scale))
    r = bf16_val(bf16_bits((yb / sb[:, None]).astype(np.float32)))
    return np.clip(np.rint(r), -128, 127).astype(np.int8), scale


def epilogue(acc, a_scale, w_scale, bias):
    v = (acc.astype(np.float32) * a_scale[:, None]).astype(np.float32)
    v = (v * w_scale[None, :]).astype(np.float32)
    if bias is not None:
        v = (v + bias[None, :]).astype(np.float32)
    return bf16_bits(v)


def kmean(k_bits):
    tot = bf16_val(k_bits).astype(np.float64).sum(axis=2)  # exact: small multiples of 1/8
    return bf16_bits((tot.astype(np.float32) / np.float32(k_bits.shape[2])).astype(np.float32))


def block_quant(x_bits, blk, mean_bits=None):
    b, h, l, d = x_bits.shape
    v = bf16_val(x_bits)
    if mean_bits is not None:
        v = (v - bf16_val(mean_bits)[:, :, None, :]).astype(np.float32)
    nblk = -(-l // blk)
    q = np.zeros(x_bits.shape, np.int8)
    s = np.zeros((b, h, nblk), np.float32)
    for i in range(nblk):
        blkv = v[:, :, i * blk:(i + 1) * blk]
        amax = np.maximum(np.abs(blkv).max(axis=(2, 3)), np.float32(1e-7)).astype(np.float32)
        s[:, :, i] = amax / np.float32(127)
        mult = (np.float32(127) / amax).astype(np.float32)
        q[:, :, i * blk:(i + 1) * blk] = np.clip(np.rint((blkv * mult[:, :, None, None]).astype(np.float32)),
                                                 -128, 127).astype(np.int8)
    return q, s


def attention(q8, qs, blkq, k8, ks, blkk, v_bits, sm, causal):
    b, hq, lq, d = q8.shape
    hkv, lk = k8.shape[1], k8.shape[2]
    g = hq // hkv
    out = np.zeros((b, hq, lq, d), np.float64)
    qsc = np.repeat(qs, blkq, axis=2)[:, :, :lq].astype(np.float64)
    ksc = np.repeat(ks, blkk, axis=2)[:, :, :lk].astype(np.float64)
    v = bf16_val(v_bits).astype(np.float64)
    for bi in range(b):
        for h in range(hq):
            acc = q8[bi, h].astype(np.int64) @ k8[bi, h // g].astype(np.int64).T
            s = acc * (float(sm) * 1.4426950408889634) * qsc[bi, h][:, None] * ksc[bi, h // g][None, :]
            if causal:
                s = np.where(np.arange(lk)[None, :] > np.arange(lq)[:, None], -np.inf, s)
            p = np.exp2(s - s.max(axis=1, keepdims=True))
            p = bf16_val(bf16_bits(p.astype(np.float32))).astype(np.float64)
            out[bi, h] = (p @ v[bi, h // g]) / p.sum(axis=1, keepdims=True)
    return out.astype(np.float32)


def main():
    rng = np.random.default_rng(20260)
    kat = {}
    # ConvRot: multiples of 1/4 in [-8, 8], one outlier channel x16, one zero row
    x = rng.integers(-32, 33, (6, 512)).astype(np.float32) / 4
    x[:, 37] *= 16
    x[4] = 0
    xb = bf16_bits(x)
    kat["convrot_x"] = xb
    for group in (128, 256):
        q, s = convrot_quant(xb, group)
        kat[f"convrot_q_g{group}"], kat[f"convrot_scale_g{group}"] = q, s
    # GEMM + epilogue
    a = rng.integers(-128, 128, (37, 256), dtype=np.int8)
    w = rng.integers(-128, 128, (40, 256), dtype=np.int8)
    a[0] = -128
    w[0] = -128
    acc = (a.astype(np.int64) @ w.astype(np.int64).T).astype(np.int32)
    a_scale = rng.uniform(1e-4, 1e-2, 37).astype(np.float32)
    w_scale = rng.uniform(1e-3, 5e-3, 40).astype(np.float32)
    bias = bf16_val(bf16_bits((rng.standard_normal(40) * 0.02).astype(np.float32)))
    kat.update(gemm_a=a, gemm_w=w, gemm_acc=acc, gemm_a_scale=a_scale, gemm_w_scale=w_scale, gemm_bias=bias,
               gemm_out_bias=epilogue(acc, a_scale, w_scale, bias), gemm_out=epilogue(acc, a_scale, w_scale, None))
    # Sage: GQA 2:1, ragged length, multiples of 1/8 plus a per-head channel bias
    b, hq, hkv, l, d = 1, 2, 1, 80, 128
    qv = rng.integers(-24, 25, (b, hq, l, d)).astype(np.float32) / 8
    kv = rng.integers(-24, 25, (b, hkv, l, d)).astype(np.float32) / 8
    kv += rng.integers(-16, 17, (b, hkv, 1, d)).astype(np.float32) / 8
    vv = rng.standard_normal((b, hkv, l, d)).astype(np.float32)
    qb, kb, vb = bf16_bits(qv), bf16_bits(kv), bf16_bits(vv)
    mean = kmean(kb)
    sm = np.float32(d ** -0.5)
    kat.update(sage_q=qb, sage_k=kb, sage_v=vb, sage_kmean=mean)
    for blkq, blkk in ((16, 64), (128, 128)):
        q8, qs = block_quant(qb, blkq)
        k8, ks = block_quant(kb, blkk, mean)
        kat[f"sage_q8_b{blkq}"], kat[f"sage_qs_b{blkq}"] = q8, qs
        kat[f"sage_k8_b{blkk}"], kat[f"sage_ks_b{blkk}"] = k8, ks
        for causal in ((False, True) if blkq == 16 else (False,)):
            kat[f"sage_out_q{blkq}_k{blkk}_c{int(causal)}"] = attention(q8, qs, blkq, k8, ks, blkk, vb, sm, causal)
    np.savez_compressed(OUT, **kat)
    print(f"wrote {OUT}: {len(kat)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
