"""numpy/ctypes front end of the C oracle (oracle/tu_oracle.c).

TEST INFRASTRUCTURE ONLY: a CPU restatement of the reference's arithmetic used
to check the HIP kernels.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it.  See tu_oracle.c for the reference citations
and for how each function is pinned.

bf16 tensors cross this interface as numpy uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lock = threading.Lock()
_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int


def build() -> str:
    """Compiles liboracle.so with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                build()
            L = ctypes.CDLL(LIB_PATH)
            for fn in ("or_exp_det", "or_tanh_det", "or_gelu_tanh_bf16", "or_gelu_tanh_f16"):
                getattr(L, fn).restype = ctypes.c_float
                getattr(L, fn).argtypes = [ctypes.c_float]
            L.or_swiglu.restype = ctypes.c_float
            L.or_swiglu.argtypes = [ctypes.c_float, ctypes.c_float]
            L.or_num_threads.restype = _i32
            L.or_num_threads.argtypes = []
            L.or_f32_to_bf16_rne.restype = ctypes.c_uint16
            L.or_f32_to_bf16_rne.argtypes = [ctypes.c_float]
            L.or_bf16_to_f32.restype = ctypes.c_float
            L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
            L.or_f32_to_bf16_n.restype = None
            L.or_f32_to_bf16_n.argtypes = [_p, _p, _i64]
            L.or_convrot_rotate_group.restype = _i32
            L.or_convrot_rotate_group.argtypes = [_p, _p, _i32]
            L.or_convrot_quant_i8.restype = _i32
            L.or_convrot_quant_i8.argtypes = [_p, _i64, _i64, _i32, _i32, _i32, _p, _p]
            L.or_convrot_quant_i8_t.restype = _i32
            L.or_convrot_quant_i8_t.argtypes = [_p, _i64, _i64, _i32, _i32, _i32, _i32, _p, _p]
            L.or_check_recip_quant.restype = _i64
            L.or_check_recip_quant.argtypes = [_p, _p]
            L.or_int8_gemm_i32.restype = _i32
            L.or_int8_gemm_i32.argtypes = [_p, _p, _i64, _i64, _i64, _p]
            L.or_int8_epilogue_bf16.restype = _i32
            L.or_int8_epilogue_bf16.argtypes = [_p, _i64, _p, _p, _i32, _p, _i64, _i64, _p]
            L.or_int8_epilogue_f32.restype = _i32
            L.or_int8_epilogue_f32.argtypes = [_p, _i64, _p, _p, _i32, _p, _i64, _i64, _p]
            L.or_int8_epilogue_f16.restype = _i32
            L.or_int8_epilogue_f16.argtypes = [_p, _i64, _p, _p, _i32, _p, _i64, _i64, _p]
            L.or_residual_gate_bf16.restype = _i32
            L.or_residual_gate_bf16.argtypes = [_p, _p, _p, _i64, _i64, _i64, _p]
            L.or_sage_kmean.restype = _i32
            L.or_sage_kmean.argtypes = [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p]
            L.or_sage_quant.restype = _i32
            L.or_sage_quant.argtypes = [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                        _p, _i64, _i64, _i64, _p]
            L.or_sage_attn_rows.restype = _i32
            L.or_sage_attn_rows.argtypes = [_p, _i64, _i64, _i64, _p, _i64,
                                            _p, _i64, _i64, _i64, _p, _i64,
                                            _p, _i64, _i64, _i64,
                                            _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _i32, _i32,
                                            _p, _i64, _p]
            L.or_f32_to_f16_rne.restype = ctypes.c_uint16
            L.or_f32_to_f16_rne.argtypes = [ctypes.c_float]
            L.or_f16_to_f32.restype = ctypes.c_float
            L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
            L.or_qk_rms_rope_int8.restype = _i32
            L.or_qk_rms_rope_int8.argtypes = [_p, _i32, _i64, _i64, _i64, _i64, _p, _i32, ctypes.c_float,
                                              _p, _i64, _i64, _i64, _i32, _i64, _i64, _p, _p]
            L.or_qk_rms_rope_int8_ex.restype = _i32
            L.or_qk_rms_rope_int8_ex.argtypes = [_p, _i32, _i64, _i64, _i64, _i64, _p, _i32, ctypes.c_float,
                                                 _p, _i64, _i64, _i64, _i32, _i64, _i64, _i32, _p, _p, _p, _p]
            L.or_qk_fused_anchor.restype = _i32
            L.or_qk_fused_anchor.argtypes = [_p, _i32, _i64, _i64, _i64, _i64, _p, _i32, ctypes.c_float, _p,
                                             _i64, _i64, _i64, _i32, _p, _p]
            L.or_qk_processed.restype = _i32
            L.or_qk_processed.argtypes = [_p, _i32, _i64, _i64, _i64, _i64, _p, _i32, ctypes.c_float, _p,
                                          _i64, _i64, _i64, _i32, _p]
            L.or_layer_norm_adaln.restype = _i32
            L.or_layer_norm_adaln.argtypes = [_p, _i32, _i64, _i64, _i64, _p, _p, _i64, ctypes.c_float, _p]
            L.or_layer_norm_affine.restype = _i32
            L.or_layer_norm_affine.argtypes = [_p, _i32, _i64, _i64, _p, _p, ctypes.c_float, _p]
            L.or_w8a8_sign_negative.restype = _i32
            L.or_w8a8_sign_negative.argtypes = [_i32]
            L.or_w8a8_hadamard.restype = None
            L.or_w8a8_hadamard.argtypes = [_p, _i32]
            L.or_w8a8_detect_anchor.restype = ctypes.c_int32
            L.or_w8a8_detect_anchor.argtypes = [_p, _i32, _i64, _i64, _i64]
            L.or_w8a8_quant_tiles.restype = _i32
            L.or_w8a8_quant_tiles.argtypes = [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                              _i32, _p, _p, _p]
            L.or_w8a8_quant_v.restype = _i32
            L.or_w8a8_quant_v.argtypes = [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p]
            L.or_w8a8_attn_rows.restype = _i32
            L.or_w8a8_attn_rows.argtypes = [_p, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _i64, _p, _i64,
                                            _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, ctypes.c_float, _i32,
                                            _p, _i64, _p]
            _lib = L
    return _lib


def num_threads() -> int:
    """OpenMP threads the oracle's parallel loops run on."""
    return int(lib().or_num_threads())


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _check(status: int, what: str) -> None:
    if status != 0:
        raise ValueError(f"oracle {what} rejected its arguments (status {status})")


# --- bf16 ------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_bf16_n(_ptr(x), _ptr(out), x.size)
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --- ConvRot ---------------------------------------------------------------

def rotate_group(x: np.ndarray, group: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape == (group,)
    y = np.empty(group, dtype=np.float32)
    _check(lib().or_convrot_rotate_group(_ptr(x), _ptr(y), group), "rotate_group")
    return y


ACT_NONE, ACT_GELU_TANH, ACT_SWIGLU = 0, 1, 2


def convrot_quant(x_bits: np.ndarray, group: int, staged: bool = False,
                  act: int = ACT_NONE, fp16: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """(int8 codes [M, K], fp32 scales [M]) of the row-buffer quantizer.
    act: 0 none, 1 tanh-GELU, 2 SwiGLU (input [M, 2K] = [gate | up]).
    fp16: x_bits are IEEE fp16 patterns (the two-pass ops' float16 input)."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    m, width = x_bits.shape
    k = width // 2 if act == ACT_SWIGLU else width
    q = np.empty((m, k), dtype=np.int8)
    s = np.empty(m, dtype=np.float32)
    _check(lib().or_convrot_quant_i8_t(_ptr(x_bits), m, k, group, act, int(staged), int(fp16), _ptr(q), _ptr(s)),
           "convrot_quant")
    return q, s


def exp_det(v: float) -> float:
    return float(lib().or_exp_det(v))


def tanh_det(u: float) -> float:
    return float(lib().or_tanh_det(u))


def gelu_tanh_bf16(x: float) -> float:
    return float(lib().or_gelu_tanh_bf16(x))


def gelu_tanh_f16(x: float) -> float:
    return float(lib().or_gelu_tanh_f16(x))


def swiglu(gate: float, up: float) -> float:
    return float(lib().or_swiglu(gate, up))


def check_recip_quant() -> tuple[int, int, int]:
    """(code mismatches, pairs checked, fp32 quotient mismatches)."""
    pairs = ctypes.c_int64(0)
    fp32 = ctypes.c_int64(0)
    bad = lib().or_check_recip_quant(ctypes.byref(pairs), ctypes.byref(fp32))
    return int(bad), int(pairs.value), int(fp32.value)


# --- GEMM ------------------------------------------------------------------

def int8_gemm_i32(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    m, k = a.shape
    n = w.shape[0]
    assert w.shape[1] == k
    acc = np.empty((m, n), dtype=np.int32)
    _check(lib().or_int8_gemm_i32(_ptr(a), _ptr(w), m, n, k, _ptr(acc)), "int8_gemm_i32")
    return acc


def epilogue_bf16(acc: np.ndarray, a_scale: np.ndarray, w_scale: np.ndarray,
                  bias: np.ndarray | None = None, cols: int | None = None) -> np.ndarray:
    """bf16 bits [M, cols] of bf16_rn(((acc * as) * ws) + bias)."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    m, ld = acc.shape
    cols = ld if cols is None else cols
    a_scale = np.ascontiguousarray(a_scale, dtype=np.float32).reshape(-1)
    w_scale = np.ascontiguousarray(w_scale, dtype=np.float32).reshape(-1)
    scalar = int(w_scale.size == 1)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    out = np.empty((m, cols), dtype=np.uint16)
    _check(lib().or_int8_epilogue_bf16(_ptr(acc), ld, _ptr(a_scale), _ptr(w_scale), scalar,
                                       None if b is None else _ptr(b), m, cols, _ptr(out)), "epilogue")
    return out


def _epilogue_out(fn: str, dtype, acc, a_scale, w_scale, bias, cols):
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    m, ld = acc.shape
    cols = ld if cols is None else cols
    a_scale = np.ascontiguousarray(a_scale, dtype=np.float32).reshape(-1)
    w_scale = np.ascontiguousarray(w_scale, dtype=np.float32).reshape(-1)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    out = np.empty((m, cols), dtype=dtype)
    _check(getattr(lib(), fn)(_ptr(acc), ld, _ptr(a_scale), _ptr(w_scale), int(w_scale.size == 1),
                              None if b is None else _ptr(b), m, cols, _ptr(out)), "epilogue")
    return out


def epilogue_f32(acc: np.ndarray, a_scale: np.ndarray, w_scale: np.ndarray, bias: np.ndarray | None = None,
                 cols: int | None = None) -> np.ndarray:
    """fp32 [M, cols] of ((acc * as) * ws) + bias, step by step (the fp32
    output_dtype of the W8A8 GEMM)."""
    return _epilogue_out("or_int8_epilogue_f32", np.float32, acc, a_scale, w_scale, bias, cols)


def epilogue_f16(acc: np.ndarray, a_scale: np.ndarray, w_scale: np.ndarray, bias: np.ndarray | None = None,
                 cols: int | None = None) -> np.ndarray:
    """fp16 bits [M, cols] of that value rounded once (RNE; NaN as 0x7e00)."""
    return _epilogue_out("or_int8_epilogue_f16", np.uint16, acc, a_scale, w_scale, bias, cols)


def residual_gate_bf16(y_bits: np.ndarray, residual_bits: np.ndarray, gate_bits: np.ndarray | None = None,
                       gate_rows: int = 1) -> np.ndarray:
    """bf16 bits of bf16_rn(fma(y, gate[i // gate_rows][j] or 1, residual))."""
    y = np.ascontiguousarray(y_bits, dtype=np.uint16)
    r = np.ascontiguousarray(residual_bits, dtype=np.uint16)
    m, n = y.shape
    assert r.shape == (m, n)
    g = None if gate_bits is None else np.ascontiguousarray(gate_bits, dtype=np.uint16)
    if g is not None:
        assert g.shape == ((m + gate_rows - 1) // gate_rows, n)
    out = np.empty((m, n), dtype=np.uint16)
    _check(lib().or_residual_gate_bf16(_ptr(y), _ptr(r), None if g is None else _ptr(g), gate_rows, m, n,
                                       _ptr(out)), "residual_gate")
    return out


# --- Sage --------------------------------------------------------------------

def _hnd(x: np.ndarray) -> tuple[int, int, int, int, int, int, int]:
    b, h, l, d = x.shape
    return b, h, l, d, h * l * d, l * d, d


def sage_kmean(k_bits: np.ndarray) -> np.ndarray:
    """bf16 bits [B, H, D] of the K channel mean; k is HND [B, H, L, D]."""
    k_bits = np.ascontiguousarray(k_bits, dtype=np.uint16)
    b, h, l, d, sb, sh, sl = _hnd(k_bits)
    mean = np.empty((b, h, d), dtype=np.uint16)
    _check(lib().or_sage_kmean(_ptr(k_bits), b, h, l, d, sb, sh, sl, _ptr(mean)), "sage_kmean")
    return mean


def sage_quant(x_bits: np.ndarray, blk: int, mean_bits: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """(int8 codes HND, fp32 scales [B, H, ceil(L/blk)]) for HND x."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    b, h, l, d, sb, sh, sl = _hnd(x_bits)
    q = np.empty(x_bits.shape, dtype=np.int8)
    s = np.empty((b, h, (l + blk - 1) // blk), dtype=np.float32)
    mean = None if mean_bits is None else np.ascontiguousarray(mean_bits, dtype=np.uint16)
    _check(lib().or_sage_quant(_ptr(x_bits), None if mean is None else _ptr(mean), b, h, l, d, sb, sh, sl, blk,
                               _ptr(q), sb, sh, sl, _ptr(s)), "sage_quant")
    return q, s


def sage_attn_rows(q8: np.ndarray, qs: np.ndarray, blkq: int, k8: np.ndarray, ks: np.ndarray, blkk: int,
                   v_bits: np.ndarray, sm_scale: float, rows: np.ndarray, causal: bool = False,
                   p_bf16: bool = True) -> np.ndarray:
    """fp32 [len(rows), D] attention outputs for (b, h, i) rows; HND inputs."""
    q8 = np.ascontiguousarray(q8, dtype=np.int8)
    k8 = np.ascontiguousarray(k8, dtype=np.int8)
    v_bits = np.ascontiguousarray(v_bits, dtype=np.uint16)
    qs = np.ascontiguousarray(qs, dtype=np.float32)
    ks = np.ascontiguousarray(ks, dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int64).reshape(-1, 3)
    b, hq, lq, d, qsb, qsh, qsl = _hnd(q8)
    _, hkv, lk, _, ksb, ksh, ksl = _hnd(k8)
    _, _, _, _, vsb, vsh, vsl = _hnd(v_bits)
    out = np.empty((rows.shape[0], d), dtype=np.float32)
    _check(lib().or_sage_attn_rows(_ptr(q8), qsb, qsh, qsl, _ptr(qs), blkq,
                                   _ptr(k8), ksb, ksh, ksl, _ptr(ks), blkk,
                                   _ptr(v_bits), vsb, vsh, vsl,
                                   hq, hkv, lq, lk, d, sm_scale, int(causal), int(p_bf16),
                                   _ptr(rows), rows.shape[0], _ptr(out)), "sage_attn_rows")
    return out


# --- fused Q/K RMSNorm + RoPE + INT8 (qk_preprocess.cu) ---------------------

DTYPE_BF16, DTYPE_FP16, DTYPE_FP32 = 0, 1, 2


def f32_to_f16_bits(v: float) -> int:
    return int(lib().or_f32_to_f16_rne(v))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().or_f16_to_f32(h))


def qk_rms_rope_int8(x_bits: np.ndarray, dtype: int, norm_bits: np.ndarray, norm_scope: str, eps: float,
                     freqs: np.ndarray | None, rot_dim: int, split_half: bool,
                     tile: int, ntiles: int) -> tuple[np.ndarray, np.ndarray]:
    """One tensor (Q or K) of the fused preprocessor.  x_bits: [B, H, L, D]
    bf16/fp16 bit patterns; freqs: fp32 [fb, fs, rot_dim / 2, 2, 2] or None.
    Returns (int8 [B, H, L, D], fp32 scales [B, H, ntiles])."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    norm_bits = np.ascontiguousarray(norm_bits, dtype=np.uint16)
    b, h, l, d = x_bits.shape
    if freqs is not None:
        freqs = np.ascontiguousarray(freqs, dtype=np.float32)
        fb, fs = freqs.shape[0], freqs.shape[1]
        assert freqs.shape[2:] == (rot_dim // 2, 2, 2)
    else:
        fb = fs = 1
        assert rot_dim == 0
    q = np.empty(x_bits.shape, dtype=np.int8)
    s = np.empty((b, h, ntiles), dtype=np.float32)
    _check(lib().or_qk_rms_rope_int8(_ptr(x_bits), dtype, b, h, l, d, _ptr(norm_bits),
                                     1 if norm_scope == "row" else 0, eps,
                                     _ptr(freqs) if freqs is not None else None, fb, fs, rot_dim,
                                     int(split_half), tile, ntiles, _ptr(q), _ptr(s)),
           "qk_rms_rope_int8")
    return q, s


def _freq_args(freqs, rot_dim):
    if freqs is not None:
        freqs = np.ascontiguousarray(freqs, dtype=np.float32)
        assert freqs.shape[2:] == (rot_dim // 2, 2, 2)
        return freqs, freqs.shape[0], freqs.shape[1]
    assert rot_dim == 0
    return None, 1, 1


def qk_rms_rope_int8_ex(x_bits: np.ndarray, dtype: int, norm_bits: np.ndarray, norm_scope: str, eps: float,
                        freqs: np.ndarray | None, rot_dim: int, split_half: bool, tile: int, ntiles: int,
                        rotate: bool = False, anchors: np.ndarray | None = None,
                        anchor_values: np.ndarray | None = None) -> tuple[np.ndarray, np.ndarray]:
    """The fused preprocessor with the W8A8 transform: K minus its anchor
    row's processed values (when anchors[b, h] >= 0), then the shared
    Hadamard rotation, then per-tile INT8."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    norm_bits = np.ascontiguousarray(norm_bits, dtype=np.uint16)
    b, h, l, d = x_bits.shape
    freqs, fb, fs = _freq_args(freqs, rot_dim)
    anc = None if anchors is None else np.ascontiguousarray(anchors, dtype=np.int32)
    av = None if anchor_values is None else np.ascontiguousarray(anchor_values, dtype=np.float32)
    q = np.empty(x_bits.shape, dtype=np.int8)
    s = np.empty((b, h, ntiles), dtype=np.float32)
    _check(lib().or_qk_rms_rope_int8_ex(_ptr(x_bits), dtype, b, h, l, d, _ptr(norm_bits),
                                        1 if norm_scope == "row" else 0, eps,
                                        _ptr(freqs) if freqs is not None else None, fb, fs, rot_dim,
                                        int(split_half), tile, ntiles, int(rotate),
                                        None if anc is None else _ptr(anc), None if av is None else _ptr(av),
                                        _ptr(q), _ptr(s)), "qk_rms_rope_int8_ex")
    return q, s


def qk_fused_anchor(x_bits: np.ndarray, dtype: int, norm_bits: np.ndarray, norm_scope: str, eps: float,
                    freqs: np.ndarray | None, rot_dim: int, split_half: bool) -> tuple[np.ndarray, np.ndarray]:
    """(int32 anchors [B, H], fp32 anchor values [B, H, D]) of the fused
    preprocessor's K stabilisation."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    norm_bits = np.ascontiguousarray(norm_bits, dtype=np.uint16)
    b, h, l, d = x_bits.shape
    freqs, fb, fs = _freq_args(freqs, rot_dim)
    anchors = np.empty((b, h), dtype=np.int32)
    values = np.empty((b, h, d), dtype=np.float32)
    _check(lib().or_qk_fused_anchor(_ptr(x_bits), dtype, b, h, l, d, _ptr(norm_bits), 1 if norm_scope == "row" else 0,
                                    eps, _ptr(freqs) if freqs is not None else None, fb, fs, rot_dim,
                                    int(split_half), _ptr(anchors), _ptr(values)), "qk_fused_anchor")
    return anchors, values


def qk_processed(x_bits: np.ndarray, dtype: int, norm_bits: np.ndarray, norm_scope: str, eps: float,
                 freqs: np.ndarray | None, rot_dim: int, split_half: bool) -> np.ndarray:
    """fp32 [B, H, L, D] RMSNorm + RoPE values (each exactly representable in
    the input type) that the fused quantizer starts from."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    norm_bits = np.ascontiguousarray(norm_bits, dtype=np.uint16)
    b, h, l, d = x_bits.shape
    freqs, fb, fs = _freq_args(freqs, rot_dim)
    out = np.empty(x_bits.shape, dtype=np.float32)
    _check(lib().or_qk_processed(_ptr(x_bits), dtype, b, h, l, d, _ptr(norm_bits), 1 if norm_scope == "row" else 0,
                                 eps, _ptr(freqs) if freqs is not None else None, fb, fs, rot_dim, int(split_half),
                                 _ptr(out)), "qk_processed")
    return out


# --- W8A8 attention variant (fused.cu rotated/anchored Q/K, V per channel) --

def w8a8_sign_negative(channel: int) -> bool:
    return bool(lib().or_w8a8_sign_negative(channel))


def w8a8_hadamard(x: np.ndarray) -> np.ndarray:
    """The shared randomized Hadamard transform of one head row (fp32)."""
    y = np.array(x, dtype=np.float32, copy=True)
    assert y.ndim == 1 and y.size in (64, 128)
    lib().or_w8a8_hadamard(_ptr(y), y.size)
    return y


def w8a8_detect_anchor(k_bits: np.ndarray, dtype: int = DTYPE_BF16) -> np.ndarray:
    """int32 [B, H] anchor rows (-1 = no anchor) of HND K bit patterns."""
    k_bits = np.ascontiguousarray(k_bits, dtype=np.uint16)
    b, h, l, d = k_bits.shape
    out = np.empty((b, h), dtype=np.int32)
    for bi in range(b):
        for hi in range(h):
            out[bi, hi] = lib().or_w8a8_detect_anchor(_ptr(k_bits[bi, hi]), dtype, l, d, d)
    return out


def w8a8_quant_tiles(x_bits: np.ndarray, tile: int, ntiles: int, rotate: bool = True,
                     anchors: np.ndarray | None = None, dtype: int = DTYPE_BF16) -> tuple[np.ndarray, np.ndarray]:
    """(int8 [B, H, L, D], fp32 scales [B, H, ntiles]) of the rotated per-tile
    quantizer; x_bits HND bf16/fp16 bit patterns."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    b, h, l, d, sb, sh, sl = _hnd(x_bits)
    q = np.empty(x_bits.shape, dtype=np.int8)
    s = np.empty((b, h, ntiles), dtype=np.float32)
    anc = None if anchors is None else np.ascontiguousarray(anchors, dtype=np.int32)
    _check(lib().or_w8a8_quant_tiles(_ptr(x_bits), dtype, b, h, l, d, sb, sh, sl, tile, ntiles, int(rotate),
                                     None if anc is None else _ptr(anc), _ptr(q), _ptr(s)), "w8a8_quant_tiles")
    return q, s


def w8a8_quant_qk(q_bits: np.ndarray, k_bits: np.ndarray, dtype: int = DTYPE_BF16, rotate: bool = True,
                  stabilize_k: bool = True):
    """The reference's per_warp_int8_hadamard contract (quant.py:182-242):
    Q per 16 tokens with ceil(Lq/64)*4 scales, K per 64 tokens.  Returns
    (q8, q_scale, k8, k_scale, anchors or None)."""
    lq, lk = q_bits.shape[2], k_bits.shape[2]
    anchors = w8a8_detect_anchor(k_bits, dtype) if stabilize_k else None
    q8, qs = w8a8_quant_tiles(q_bits, 16, (lq + 63) // 64 * 4, rotate, None, dtype)
    k8, ks = w8a8_quant_tiles(k_bits, 64, (lk + 63) // 64, rotate, anchors, dtype)
    return q8, qs, k8, ks, anchors


def w8a8_quant_v(v_bits: np.ndarray, dtype: int = DTYPE_BF16) -> tuple[np.ndarray, np.ndarray]:
    """(int8 [B, H, D, Lpad], fp32 scales [B, H, D]) of the channel-wise V
    quantizer; v_bits HND."""
    v_bits = np.ascontiguousarray(v_bits, dtype=np.uint16)
    b, h, l, d, sb, sh, sl = _hnd(v_bits)
    lpad = (l + 63) // 64 * 64
    q = np.empty((b, h, d, lpad), dtype=np.int8)
    s = np.empty((b, h, d), dtype=np.float32)
    _check(lib().or_w8a8_quant_v(_ptr(v_bits), dtype, b, h, l, d, sb, sh, sl, lpad, _ptr(q), _ptr(s)),
           "w8a8_quant_v")
    return q, s


def w8a8_attn_rows(q8: np.ndarray, qs: np.ndarray, k8: np.ndarray, ks: np.ndarray, v8: np.ndarray,
                   vs: np.ndarray, lk: int, sm_scale: float, rows: np.ndarray, causal: bool = False) -> np.ndarray:
    """fp32 [len(rows), D] dense W8A8 attention outputs for (b, h, i) rows.
    q8/k8 HND int8, qs [B, Hq, nqs], ks [B, Hkv, nks], v8 [B, Hkv, D, Lpad],
    vs [B, Hkv, D]."""
    q8 = np.ascontiguousarray(q8, dtype=np.int8)
    k8 = np.ascontiguousarray(k8, dtype=np.int8)
    v8 = np.ascontiguousarray(v8, dtype=np.int8)
    qs = np.ascontiguousarray(qs, dtype=np.float32)
    ks = np.ascontiguousarray(ks, dtype=np.float32)
    vs = np.ascontiguousarray(vs, dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int64).reshape(-1, 3)
    b, hq, lq, d, qsb, qsh, qsl = _hnd(q8)
    _, hkv, lk8, _, ksb, ksh, ksl = _hnd(k8)
    assert lk8 == lk and v8.shape[:3] == (b, hkv, d)
    out = np.empty((rows.shape[0], d), dtype=np.float32)
    _check(lib().or_w8a8_attn_rows(_ptr(q8), qsb, qsh, qsl, _ptr(qs), qs.shape[2], _ptr(k8), ksb, ksh, ksl,
                                   _ptr(ks), ks.shape[2], _ptr(v8), v8.shape[3], _ptr(vs), hq, hkv, lq, lk, d,
                                   sm_scale, int(causal), _ptr(rows), rows.shape[0], _ptr(out)), "w8a8_attn_rows")
    return out


# --- Wan block: LayerNorm + AdaLN -------------------------------------------

def layer_norm_adaln(x, scale, shift, eps: float, dtype: int = DTYPE_BF16) -> np.ndarray:
    """LayerNorm(x) * (1 + scale) + shift with the reference's Welford order.
    x [B, L, H], scale/shift [B, steps, H]: uint16 bit patterns (dtype 0 bf16,
    1 fp16) or float32 arrays (dtype 2); the result has x's numpy dtype."""
    kind = np.float32 if dtype == DTYPE_FP32 else np.uint16
    x = np.ascontiguousarray(x, dtype=kind)
    scale = np.ascontiguousarray(scale, dtype=kind)
    shift = np.ascontiguousarray(shift, dtype=kind)
    b, l, h = x.shape
    assert scale.shape == shift.shape and scale.shape[0] == b and scale.shape[2] == h
    out = np.empty(x.shape, dtype=kind)
    _check(lib().or_layer_norm_adaln(_ptr(x), dtype, b, l, h, _ptr(scale), _ptr(shift), scale.shape[1], eps,
                                     _ptr(out)), "layer_norm_adaln")
    return out


def layer_norm_affine(x, weight, bias, eps: float, dtype: int = DTYPE_BF16) -> np.ndarray:
    """LayerNorm with an elementwise affine weight / bias: x [R, H] (uint16
    patterns for bf16 / fp16, float32 for fp32), weight / bias [H] in the same
    type.  Returns the output in the same representation."""
    x = np.ascontiguousarray(x)
    weight = np.ascontiguousarray(weight).reshape(-1)
    bias = np.ascontiguousarray(bias).reshape(-1)
    r, h = x.shape
    assert weight.shape == (h,) and bias.shape == (h,)
    out = np.empty_like(x)
    _check(lib().or_layer_norm_affine(_ptr(x), dtype, r, h, _ptr(weight), _ptr(bias), eps, _ptr(out)),
           "layer_norm_affine")
    return out
