/*
 * CPU oracle for the quantized DiT hot path (ConvRot W8A8 linear + Sage INT8
 * attention).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is a plain-C restatement of the
 * reference plugin's arithmetic, used as the checker for the HIP kernels.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product path (comfyui-turing-utils_amd/) never calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -fno-fast-math -ffp-contract=off).  IEEE
 * fp32 arithmetic without contraction is what makes the restatement bit-exact
 * for the integer outputs (codes, accumulators).
 *
 * Citations are to files under the reference tree
 * (brahianrosswill/comfyui-turing-utils).
 *
 * Parity status per function (how each is pinned is in tests/test_oracle_*.py):
 *   or_f32_to_bf16_rne        pinned: exhaustive-ish vs torch.bfloat16 cast
 *   or_convrot_rotate_group   pinned: dense Kronecker matrix (fp64), orthogonality,
 *                             involution, basis columns, regular-row property
 *   or_convrot_quant_i8       pinned: invariants + staged==row-buffer KAT
 *   or_convrot_quant_i8_t     fp16 elements pinned: numpy float16 restatement of
 *                             the rotation output, scale and quotient; zero /
 *                             tiny rows (division by fp16(scale) = 0); GELU
 *                             fp16 output vs torch float16 gelu(tanh)
 *   or_check_recip_quant      the GPU's reciprocal-multiply quotient gives the
 *                             IEEE-division code on every pair of the
 *                             quantizer's bf16 domain (exhaustive)
 *   or_int8_gemm_i32          pinned: numpy int64 matmul (brute force)
 *   or_int8_epilogue_bf16     pinned: fp64 closed form within bf16 rounding
 *   or_int8_epilogue_f32/_f16 pinned: numpy float32 step-by-step products and
 *                             sum (bit-exact), numpy float16 cast of that value
 *   or_residual_gate_bf16     pinned: numpy fp64 product-plus-sum rounded once
 *   or_sage_kmean             pinned: fp64 mean within one bf16 ulp
 *   or_sage_quant             pinned: invariants (max|q|==127, dequant error)
 *   or_sage_attn_rows         pinned: fp64 SDPA on dequantized inputs, torch SDPA
 *                             on raw inputs (reference gate rtol .08 / atol .06)
 *   or_f32_to_f16_rne         pinned: every fp32 class vs numpy float16 casts
 *   or_layer_norm_affine      pinned: torch layer_norm(weight, bias) in fp32 and
 *                             bf16 (equal apart from rounding ties), fp64 formula
 *   or_qk_rms_rope_int8       pinned: the reference's own KAT (torch restatement of
 *                             validate_compatible.py:241-286 + per-warp INT8,
 *                             codes within 2 LSB, scales rtol .015), fp64 RMSNorm,
 *                             identity / rotation-by-angle RoPE closed forms
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* bf16 helpers: convrot_quant.cu:293-309 (same in bf16_epilogue.cu:25-39).   */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

OR_API uint16_t or_f32_to_bf16_rne(float value) {
    const uint32_t bits = f2u(value);
    if ((bits & 0x7fffffffU) > 0x7f800000U) return 0x7fffU; /* canonical NaN */
    uint16_t upper = (uint16_t)(bits >> 16);
    const uint32_t rem = bits << 16;
    if (rem > 0x80000000U || (rem == 0x80000000U && (upper & 1U))) ++upper;
    return upper;
}

OR_API float or_bf16_to_f32(uint16_t v) { return u2f((uint32_t)v << 16); }

/* Threads the OpenMP loops below use (OMP_NUM_THREADS or the core count). */
OR_API int or_num_threads(void) { return omp_get_max_threads(); }

static inline float bf16_round_f32(float v) { return or_bf16_to_f32(or_f32_to_bf16_rne(v)); }

OR_API void or_f32_to_bf16_n(const float *x, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = or_f32_to_bf16_rne(x[i]);
}

/* ------------------------------------------------------------------------ */
/* ConvRot rotation.                                                         */
/*                                                                           */
/* G=256 (reference): R4 (x) R4 (x) R4 (x) R4 with                            */
/*   R4 = 1/2 [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]],                  */
/* applied digit by digit, stride 1 -> 4 -> 16 -> 64                          */
/* (convrot_quant.cu:104-116 fht_stage, :311-330 last stage, :384-391 first  */
/* stage inline).  Exact fp32 add order of each output:                      */
/*   y0 = 0.5*(((x0+x1)+x2)-x3)   y1 = 0.5*(((x0+x1)-x2)+x3)                  */
/*   y2 = 0.5*(((x0-x1)+x2)+x3)   y3 = 0.5*(((-x0+x1)+x2)+x3)                 */
/*                                                                           */
/* G=128 (build-defined; the reference supports only 256 and no regular      */
/* Hadamard matrix of order 128 exists): R4 (x) R4 (x) R4 on digits of stride */
/* 1, 4, 16, then the orthonormal H2 = (1/sqrt2)[[1,1],[1,-1]] on the stride- */
/* 64 digit: y0 = c*(x0+x1), y1 = c*(x0-x1), c = fp32(1/sqrt(2)).             */
/* ------------------------------------------------------------------------ */
static const float kInvSqrt2 = 0.70710678118654752440f;

static void r4_stage(const float *src, float *dst, int stride, int group) {
    for (int lane = 0; lane < group / 4; ++lane) {
        const int base = (lane % stride) + (lane / stride) * (4 * stride);
        const float x0 = src[base];
        const float x1 = src[base + stride];
        const float x2 = src[base + 2 * stride];
        const float x3 = src[base + 3 * stride];
        dst[base] = 0.5f * (((x0 + x1) + x2) - x3);
        dst[base + stride] = 0.5f * (((x0 + x1) - x2) + x3);
        dst[base + 2 * stride] = 0.5f * (((x0 - x1) + x2) + x3);
        dst[base + 3 * stride] = 0.5f * (((-x0 + x1) + x2) + x3);
    }
}

static void h2_stage(const float *src, float *dst, int stride, int group) {
    for (int lane = 0; lane < group / 2; ++lane) {
        const int base = (lane % stride) + (lane / stride) * (2 * stride);
        const float x0 = src[base];
        const float x1 = src[base + stride];
        dst[base] = kInvSqrt2 * (x0 + x1);
        dst[base + stride] = kInvSqrt2 * (x0 - x1);
    }
}

/* y = rotation(x) for one group, fp32 (before any bf16 rounding). */
OR_API int or_convrot_rotate_group(const float *x, float *y, int group) {
    float a[256], b[256];
    if (group != 128 && group != 256) return -1;
    r4_stage(x, a, 1, group);
    r4_stage(a, b, 4, group);
    r4_stage(b, a, 16, group);
    if (group == 256) r4_stage(a, y, 64, group);
    else h2_stage(a, y, 64, group);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Input activations folded into the quantizer (convrot_quant.cu:137-156,    */
/* :332-344):                                                                 */
/*   act 1, tanh-GELU:  bf16( (0.5 x) (1 + tanh(a (x + ((b x) x) x))) ),     */
/*                      a = 0.7978845608028654, b = 0.044715 (:145-156)       */
/*   act 2, SwiGLU:     (g / (1 + exp(-g))) u over the [g | u] halves of a   */
/*                      2K-wide row (:137-143), not rounded before the FHT    */
/* The reference calls CUDA's tanhf / expf, whose last-ulp behaviour is not   */
/* reproducible off-GPU.  This build defines exp and tanh by the fixed fp32   */
/* sequences below (the GPU kernel executes the same operations in the same   */
/* order, so activation outputs are bit-identical between the two):         */
/*   exp_det(v): Cody-Waite reduction n = rint(v log2 e),                     */
/*     r = (v - n ln2_hi) - n ln2_lo, degree-7 Taylor polynomial of e^r in    */
/*     Horner form, scaled by 2^n; 0 below -87, +inf above 88.72.             */
/*   tanh_det(u) = sign(u) (1 - 2 / (exp_det(2|u|) + 1)), |u| for            */
/*     |u| < 2^-12, 1 for |u| > 9.                                            */
/* Both are pinned against double-precision exp / tanh by error bounds.      */
/* ------------------------------------------------------------------------ */
OR_API float or_exp_det(float v) {
    if (v != v) return v;
    if (v > 88.72f) return INFINITY;
    if (v < -87.0f) return 0.0f;
    const float n = nearbyintf(v * 1.44269504f);
    const float r = (v - n * 0.693145752f) - n * 1.42860677e-6f;
    float p = 1.98412698e-4f;
    p = p * r + 1.38888889e-3f;
    p = p * r + 8.33333377e-3f;
    p = p * r + 4.16666679e-2f;
    p = p * r + 1.66666672e-1f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, (int)n);
}

OR_API float or_tanh_det(float u) {
    if (u != u) return u;
    const float a = fabsf(u);
    const float e = or_exp_det(2.0f * fminf(a, 9.0f));
    float t = 1.0f - 2.0f / (e + 1.0f);
    t = a < 0.000244140625f ? a : t;
    t = a > 9.0f ? 1.0f : t;
    return copysignf(t, u);
}

OR_API float or_gelu_tanh_bf16(float x) {
    const float inner = 0.7978845608028654f * (x + ((0.044715f * x) * x) * x);
    const float act = (0.5f * x) * (1.0f + or_tanh_det(inner));
    return bf16_round_f32(act);
}

OR_API float or_swiglu(float gate, float up) { return (gate / (1.0f + or_exp_det(-gate))) * up; }

static inline float load_act(const uint16_t *row, int64_t col, int64_t k, int act) {
    if (act == 2) return or_swiglu(or_bf16_to_f32(row[col]), or_bf16_to_f32(row[k + col]));
    if (act == 1) return or_gelu_tanh_bf16(or_bf16_to_f32(row[col]));
    return or_bf16_to_f32(row[col]);
}

OR_API uint16_t or_f32_to_f16_rne(float value);
OR_API float or_f16_to_f32(uint16_t h);
static inline float f16_round_f32(float v) { return or_f16_to_f32(or_f32_to_f16_rne(v)); }

/* fp16 elements (the reference's InputType = half, convrot_quant.cu:137-156):
 * GELU's output is rounded to fp16 (:153-155), SwiGLU's is not. */
OR_API float or_gelu_tanh_f16(float x) {
    const float inner = 0.7978845608028654f * (x + ((0.044715f * x) * x) * x);
    return f16_round_f32((0.5f * x) * (1.0f + or_tanh_det(inner)));
}

static inline float load_act_f16(const uint16_t *row, int64_t col, int64_t k, int act) {
    if (act == 2) return or_swiglu(or_f16_to_f32(row[col]), or_f16_to_f32(row[k + col]));
    if (act == 1) return or_gelu_tanh_f16(or_f16_to_f32(row[col]));
    return or_f16_to_f32(row[col]);
}

/* ------------------------------------------------------------------------ */
/* Row-buffer ConvRot INT8 quantizer: convrot_quant.cu:350-444 (Int4=false). */
/*   absmax over fp32 y of the whole row (:400-404)                           */
/*   scale  = max(min(absmax, 3.38953139e38) / 127, 1e-30)   (:408-412)       */
/*   rs     = bf16(scale)                                     (:417)          */
/*   q      = clamp(nearbyint(bf16(bf16(y) / rs)), -128, 127) (:431-441)      */
/* scales[row] keeps the unrounded fp32 scale (:413-415).                     */
/* staged != 0 selects the staged formulation's scale, absmax*(1/127)        */
/* (convrot_quant.cu:233-236), the reference's own cross-check partner.      */
/* ------------------------------------------------------------------------ */
/* dtype 1: fp16 elements, the two-pass kernels' InputType = half           */
/* (convrot_quant.cu:158-248): rotated values kept as fp16, clip 65504         */
/* (finite_max<half>, :58-62), q = clamp(nearbyint(fp16(fp16(y) / fp16(scale)))) */
/* (quant_div_to_float, :69-73).  fp16(scale) is 0 below 2^-25: the quotient */
/* is then +-inf or NaN, which the clamp maps to 127 / -128 (fmaxf(-128, NaN) */
/* is -128), as in the reference.                                             */
OR_API int or_convrot_quant_i8_t(const uint16_t *x, int64_t rows, int64_t k, int group, int act,
                                 int staged, int dtype, int8_t *q, float *scales) {
    if ((group != 128 && group != 256) || k <= 0 || k % group || (dtype != 0 && dtype != 1)) return -1;
    const int64_t in_width = act == 2 ? 2 * k : k;
    uint16_t *buf = (uint16_t *)malloc((size_t)k * sizeof(uint16_t));
    if (!buf) return -2;
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *row = x + r * in_width;
        float absmax = 0.0f;
        for (int64_t g = 0; g < k / group; ++g) {
            float xin[256], y[256];
            for (int i = 0; i < group; ++i)
                xin[i] = dtype ? load_act_f16(row, g * group + i, k, act) : load_act(row, g * group + i, k, act);
            or_convrot_rotate_group(xin, y, group);
            for (int i = 0; i < group; ++i) {
                absmax = fmaxf(absmax, fabsf(y[i]));
                buf[g * group + i] = dtype ? or_f32_to_f16_rne(y[i]) : or_f32_to_bf16_rne(y[i]);
            }
        }
        const float clipped = fminf(absmax, dtype ? 65504.0f : 3.38953139e38f);
        const float scale = staged ? fmaxf(clipped * (1.0f / 127.0f), 1.0e-30f)
                                   : fmaxf(clipped / 127.0f, 1.0e-30f);
        scales[r] = scale;
        const float rs = dtype ? f16_round_f32(scale) : bf16_round_f32(scale);
        for (int64_t c = 0; c < k; ++c) {
            const float v = dtype ? or_f16_to_f32(buf[c]) : or_bf16_to_f32(buf[c]);
            const float divided = dtype ? f16_round_f32(v / rs) : bf16_round_f32(v / rs);
            float qf = nearbyintf(divided);
            qf = fminf(127.0f, fmaxf(-128.0f, qf));
            q[r * k + c] = (int8_t)qf;
        }
    }
    free(buf);
    return 0;
}

OR_API int or_convrot_quant_i8(const uint16_t *x, int64_t rows, int64_t k, int group, int act,
                               int staged, int8_t *q, float *scales) {
    return or_convrot_quant_i8_t(x, rows, k, group, act, staged, 0, q, scales);
}

/* The GPU quantizer forms the quotient bf16(y) / bf16(scale) as one multiply
 * by the correctly rounded reciprocal of the (per-row) bf16 scale.
 * or_check_recip_quant below proves, over every pair the quantizer can
 * produce -- every divisor b that bf16(scale) can take (positive normal bf16,
 * 1e-30 <= b <= 2^128/127) and every finite bf16 dividend a with |a| <= 130 b
 * (the row-buffer invariant |bf16(y)| <= bf16(absmax) <= 128.5 bf16(scale))
 * -- that the INT8 code clamp(nearbyint(bf16(q))) is the same as with IEEE
 * division. */
static inline int quant_code(float d) {
    float qf = nearbyintf(bf16_round_f32(d));
    qf = fminf(127.0f, fmaxf(-128.0f, qf));
    return (int)qf;
}

/* The same domain with the quotient formed as a * RN(1 / b): one multiply
 * by the correctly rounded reciprocal (what the GPU quantizer uses).  Its
 * fp32 result can differ from a / b in the last place, but a and b both
 * carry 8 significant bits, so a / b is never within 2^-17 (relative) of a
 * bf16 rounding midpoint unless it is bf16-exact, and the two roundings of
 * the reciprocal product stay within 2^-23: the bf16 quotient, and hence the
 * code, is the same.  Returns the number of differing codes. */
OR_API int64_t or_check_recip_quant(int64_t *pairs, int64_t *fp32_mismatch) {
    int64_t bad_code = 0, bad_fp32 = 0, n = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : bad_code, bad_fp32, n)
    for (uint32_t bb = 0x0080; bb < 0x7f80; ++bb) {
        const float b = u2f(bb << 16);
        if (b < 1.0e-30f || b > 3.38953139e38f / 127.0f * 1.01f) continue;
        const float r = 1.0f / b;
        for (uint32_t ab = 0; ab < 0x10000; ++ab) {
            if ((ab & 0x7f80) == 0x7f80) continue; /* inf / nan */
            const float a = u2f(ab << 16);
            if (fabsf(a) > 130.0f * b) continue;
            ++n;
            const float ieee = a / b;
            const float rq = a * r;
            if (f2u(ieee) != f2u(rq)) ++bad_fp32;
            if (quant_code(ieee) != quant_code(rq)) ++bad_code;
        }
    }
    if (pairs) *pairs = n;
    if (fp32_mismatch) *fp32_mismatch = bad_fp32;
    return bad_code;
}


/* ------------------------------------------------------------------------ */
/* INT8 x INT8 -> INT32: acc[m][n] = sum_k A[m][k] * W[n][k].                */
/* The reference's turing_int8_linear contracts A [M,K] row-major with W     */
/* [N,K] row-major (w4a8.cu:1185-1219, bindings.cpp:371-421).  Exact integer  */
/* math: |acc| <= K * 128 * 128 < 2^31 for K < 131072.                        */
/* ------------------------------------------------------------------------ */
OR_API int or_int8_gemm_i32(const int8_t *a, const int8_t *w, int64_t m, int64_t n, int64_t k,
                            int32_t *acc) {
    if (k >= 131072) return -1;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        const int8_t *ar = a + i * k;
        for (int64_t j = 0; j < n; ++j) {
            const int8_t *wr = w + j * k;
            int32_t s = 0;
            for (int64_t t = 0; t < k; ++t) s += (int32_t)ar[t] * (int32_t)wr[t];
            acc[i * n + j] = s;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Epilogue: out = bf16_rn(((float(acc) * as[m]) * ws[n]) + bias[n]).        */
/* Operation order of the CUTLASS EVT tree Mult(Mult(Acc, as), ws) then      */
/* Plus(., bias) (w4a8.cu:480-525); bias arrives as fp32 (bindings.cpp:379-  */
/* 383); the no-bias op dequantize_int8_bf16 is the same without the add     */
/* (bf16_epilogue.cu:105-119).  ws_scalar != 0 broadcasts ws[0].             */
/* ------------------------------------------------------------------------ */
OR_API int or_int8_epilogue_bf16(const int32_t *acc, int64_t acc_ld, const float *as,
                                 const float *ws, int ws_scalar, const float *bias, int64_t m,
                                 int64_t n, uint16_t *out) {
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t j = 0; j < n; ++j) {
            float v = (float)acc[i * acc_ld + j];
            v = v * as[i];
            v = v * ws[ws_scalar ? 0 : j];
            if (bias) v = v + bias[j];
            out[i * n + j] = or_f32_to_bf16_rne(v);
        }
    }
    return 0;
}

/* The same epilogue value unrounded (fp32 output_dtype) and rounded once to  */
/* fp16 (fp16 output_dtype; dispatch.py:538-615, :660-668): RNE, overflow to  */
/* +-inf, subnormals kept, every NaN written as 0x7e00.                      */
static inline float epilogue_value(const int32_t *acc, int64_t acc_ld, const float *as, const float *ws,
                                   int ws_scalar, const float *bias, int64_t i, int64_t j) {
    float v = (float)acc[i * acc_ld + j];
    v = v * as[i];
    v = v * ws[ws_scalar ? 0 : j];
    if (bias) v = v + bias[j];
    return v;
}

OR_API int or_int8_epilogue_f32(const int32_t *acc, int64_t acc_ld, const float *as, const float *ws,
                                int ws_scalar, const float *bias, int64_t m, int64_t n, float *out) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) out[i * n + j] = epilogue_value(acc, acc_ld, as, ws, ws_scalar, bias, i, j);
    return 0;
}

OR_API uint16_t or_f32_to_f16_rne(float value);

OR_API int or_int8_epilogue_f16(const int32_t *acc, int64_t acc_ld, const float *as, const float *ws,
                                int ws_scalar, const float *bias, int64_t m, int64_t n, uint16_t *out) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            const float v = epilogue_value(acc, acc_ld, as, ws, ws_scalar, bias, i, j);
            out[i * n + j] = v != v ? (uint16_t)0x7e00U : or_f32_to_f16_rne(v);
        }
    return 0;
}

/* Gated residual of tu_int8_gemm_bf16_residual (no reference counterpart:   */
/* the torch add / addcmul after a Wan block's o and FFN-down projections):  */
/*   out = bf16_rn(fmaf(y, g, r)), g = gate[i / gate_rows][j] or 1.          */
OR_API int or_residual_gate_bf16(const uint16_t *y, const uint16_t *residual, const uint16_t *gate,
                                 int64_t gate_rows, int64_t m, int64_t n, uint16_t *out) {
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t j = 0; j < n; ++j) {
            const float g = gate ? or_bf16_to_f32(gate[(i / gate_rows) * n + j]) : 1.0f;
            out[i * n + j] = or_f32_to_bf16_rne(fmaf(or_bf16_to_f32(y[i * n + j]), g,
                                                     or_bf16_to_f32(residual[i * n + j])));
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Sage K mean (smoothing).  The reference defines smoothing as subtracting  */
/* a per-(batch, head) channel mean stored in the input type before the       */
/* block absmax (fused.cu:93-128, sub_mean); it does not define how the mean */
/* is computed.  This build fixes the fp32 summation order so that the GPU   */
/* and this restatement agree bit for bit:                                   */
/*   chunk c covers tokens [128c, 128c+128);                                 */
/*   rows = 256 / (D/8) lanes-rows, per = 128 / rows tokens per row;          */
/*   p[r][d]   = sum_{j=0..per-1} x[128c + r + rows*j][d]   (ascending j)    */
/*   chunk[d]  = sum_{r=0..rows-1} p[r][d]                   (ascending r)    */
/*   total[d]  = sum_{c ascending} chunk[c][d]                                */
/*   mean[d]   = bf16_rn(total[d] / (float)L)                                 */
/* Tokens at or beyond L are skipped.                                         */
/* x is addressed with element strides (batch, head, seq); channels are       */
/* contiguous.                                                                */
/* ------------------------------------------------------------------------ */
OR_API int or_sage_kmean(const uint16_t *x, int64_t batch, int64_t heads, int64_t len, int64_t dim,
                         int64_t s_b, int64_t s_h, int64_t s_l, uint16_t *mean /* [B,H,D] */) {
    if (dim != 64 && dim != 128) return -1;
    const int rows = 256 / (int)(dim / 8);
    const int per = 128 / rows;
    const int64_t chunks = (len + 127) / 128;
    float *tot = (float *)malloc((size_t)dim * sizeof(float));
    float *p = (float *)malloc((size_t)rows * dim * sizeof(float));
    if (!tot || !p) { free(tot); free(p); return -2; }
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t h = 0; h < heads; ++h) {
            const uint16_t *base = x + b * s_b + h * s_h;
            for (int64_t d = 0; d < dim; ++d) tot[d] = 0.0f;
            for (int64_t c = 0; c < chunks; ++c) {
                for (int r = 0; r < rows; ++r) {
                    for (int64_t d = 0; d < dim; ++d) {
                        float s = 0.0f;
                        for (int j = 0; j < per; ++j) {
                            const int64_t t = 128 * c + r + (int64_t)rows * j;
                            if (t < len) s = s + or_bf16_to_f32(base[t * s_l + d]);
                        }
                        p[r * dim + d] = s;
                    }
                }
                for (int64_t d = 0; d < dim; ++d) {
                    float s = 0.0f;
                    for (int r = 0; r < rows; ++r) s = s + p[r * dim + d];
                    tot[d] = tot[d] + s;
                }
            }
            for (int64_t d = 0; d < dim; ++d)
                mean[(b * heads + h) * dim + d] = or_f32_to_bf16_rne(tot[d] / (float)len);
        }
    }
    free(tot);
    free(p);
    return 0;
}

/* cvt.rni.sat.s8.f32 (numeric_conversion.cuh:144-149): round half to even,
 * saturate to [-128, 127], NaN -> 0. */
static inline int8_t sat_rne_s8(float v) {
    if (v != v) return 0;
    float r = nearbyintf(v);
    if (r > 127.0f) r = 127.0f;
    if (r < -128.0f) r = -128.0f;
    return (int8_t)r;
}

/* ------------------------------------------------------------------------ */
/* Sage per-block INT8 quantizer: QuantInt8Kernel (fused.cu:66-200).          */
/*   v      = float(x) - float(mean[d])  (sub_mean, :97-128)                  */
/*   amax   = max(1e-7, max |v| over the block's tokens x channels) (:149-159)*/
/*   scale  = amax / 127            (:166)                                    */
/*   q      = cvt.rni.sat.s8(v * (127 / amax))   (:171-187)                   */
/* Tokens past L count as 0 and are not written.  Scale layout [B,H,nblk].    */
/* The reference builds this extension with --use_fast_math; the restatement */
/* uses IEEE division (the approximate forms are not reproduced).             */
/* ------------------------------------------------------------------------ */
OR_API int or_sage_quant(const uint16_t *x, const uint16_t *mean /* [B,H,D] or NULL */,
                         int64_t batch, int64_t heads, int64_t len, int64_t dim, int64_t s_b,
                         int64_t s_h, int64_t s_l, int64_t blk, int8_t *q, int64_t qs_b,
                         int64_t qs_h, int64_t qs_l, float *scale /* [B,H,nblk] */) {
    const int64_t nblk = (len + blk - 1) / blk;
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t h = 0; h < heads; ++h) {
            const uint16_t *xb = x + b * s_b + h * s_h;
            int8_t *qb = q + b * qs_b + h * qs_h;
            const uint16_t *mu = mean ? mean + (b * heads + h) * dim : NULL;
            for (int64_t blkid = 0; blkid < nblk; ++blkid) {
                float amax = 0.0000001f;
                for (int64_t t = blkid * blk; t < (blkid + 1) * blk && t < len; ++t)
                    for (int64_t d = 0; d < dim; ++d) {
                        float v = or_bf16_to_f32(xb[t * s_l + d]);
                        if (mu) v = v - or_bf16_to_f32(mu[d]);
                        amax = fmaxf(amax, fabsf(v));
                    }
                scale[(b * heads + h) * nblk + blkid] = amax / 127.0f;
                const float mult = 127.0f / amax;
                for (int64_t t = blkid * blk; t < (blkid + 1) * blk && t < len; ++t)
                    for (int64_t d = 0; d < dim; ++d) {
                        float v = or_bf16_to_f32(xb[t * s_l + d]);
                        if (mu) v = v - or_bf16_to_f32(mu[d]);
                        qb[t * qs_l + d] = sat_rne_s8(v * mult);
                    }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Sage attention on quantized Q/K and bf16 V, for a subset of query rows.   */
/* Reference math (qk_int_sv_f16_cuda_sm75.cu:117-118, :375-381, :411-466;   */
/* attn_utils.cuh:464-568, :676-703, :920-973):                               */
/*   s[j]  = float(sum_d q8[i][d] k8[j][d]) * (sm_scale*log2e) * qs * ks      */
/*   p[j]  = 2^(s[j] - max_j s)   (masked keys excluded)                      */
/*   P[j]  = round(p[j]) to the PV operand type (bf16 here; the reference's   */
/*           Turing kernel used fp16)                                         */
/*   o[d]  = (sum_j P[j] v[j][d]) / (sum_j P[j])                              */
/* Computed in double from the rounded P; the GPU's online softmax differs   */
/* from this only by fp32 rounding, which the attention tolerance covers.    */
/* Causal masking is top-left aligned (kv_idx > q_idx masked,                */
/* attn_utils.cuh:407-431).  GQA: q head h reads kv head h / (Hq/Hkv).        */
/* Rows are given as a list of (b, h, i) triples; out is [nrows, D] fp32.     */
/* ------------------------------------------------------------------------ */
OR_API int or_sage_attn_rows(const int8_t *q8, int64_t q_sb, int64_t q_sh, int64_t q_sl,
                             const float *qs, int64_t blkq,
                             const int8_t *k8, int64_t k_sb, int64_t k_sh, int64_t k_sl,
                             const float *ks, int64_t blkk,
                             const uint16_t *v, int64_t v_sb, int64_t v_sh, int64_t v_sl,
                             int64_t hq, int64_t hkv, int64_t lq, int64_t lk, int64_t dim,
                             float sm_scale, int causal, int p_bf16,
                             const int64_t *rows /* [nrows,3] */, int64_t nrows, float *out) {
    const double log2e = 1.4426950408889634;
    const int64_t nbq = (lq + blkq - 1) / blkq;
    const int64_t nbk = (lk + blkk - 1) / blkk;
    const int64_t groups = hq / hkv;
#pragma omp parallel
    {
        double *s = (double *)malloc((size_t)lk * sizeof(double));
        double *o = (double *)malloc((size_t)dim * sizeof(double));
#pragma omp for schedule(dynamic)
        for (int64_t r = 0; r < nrows; ++r) {
            const int64_t b = rows[3 * r], h = rows[3 * r + 1], i = rows[3 * r + 2];
            const int64_t hk = h / groups;
            const int8_t *qi = q8 + b * q_sb + h * q_sh + i * q_sl;
            const float qscale = qs[(b * hq + h) * nbq + i / blkq];
            const int64_t jmax = causal ? (i + 1 < lk ? i + 1 : lk) : lk;
            double m = -INFINITY;
            for (int64_t j = 0; j < jmax; ++j) {
                const int8_t *kj = k8 + b * k_sb + hk * k_sh + j * k_sl;
                int32_t acc = 0;
                for (int64_t d = 0; d < dim; ++d) acc += (int32_t)qi[d] * (int32_t)kj[d];
                const double kscale = ks[(b * hkv + hk) * nbk + j / blkk];
                s[j] = (double)acc * ((double)sm_scale * log2e) * (double)qscale * kscale;
                if (s[j] > m) m = s[j];
            }
            double l = 0.0;
            for (int64_t d = 0; d < dim; ++d) o[d] = 0.0;
            for (int64_t j = 0; j < jmax; ++j) {
                double p = exp2(s[j] - m);
                if (p_bf16) p = (double)bf16_round_f32((float)p);
                l += p;
                const uint16_t *vj = v + b * v_sb + hk * v_sh + j * v_sl;
                for (int64_t d = 0; d < dim; ++d) o[d] += p * (double)or_bf16_to_f32(vj[d]);
            }
            for (int64_t d = 0; d < dim; ++d) out[r * dim + d] = (float)(o[d] / l);
        }
        free(s);
        free(o);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* IEEE binary16 conversions (round to nearest even, subnormals kept).        */
/* ------------------------------------------------------------------------ */
OR_API uint16_t or_f32_to_f16_rne(float value) {
    const uint32_t bits = f2u(value);
    const uint32_t sign = (bits >> 16) & 0x8000U;
    const uint32_t absb = bits & 0x7fffffffU;
    if (absb > 0x7f800000U) return (uint16_t)(sign | 0x7e00U); /* NaN */
    if (absb >= 0x477ff000U) return (uint16_t)(sign | 0x7c00U); /* rounds to inf */
    if (absb < 0x38800000U) {                                   /* half subnormal or 0 */
        /* value = absb-float; subnormal unit 2^-24: round(v * 2^24) half-even */
        const float v = u2f(absb) * 16777216.0f; /* exact scaling by 2^24 */
        const float r = nearbyintf(v);
        return (uint16_t)(sign | (uint32_t)r);
    }
    /* normal: rebias exponent, round the 13 dropped mantissa bits */
    uint32_t m = absb - 0x38000000U; /* exponent 127 -> 15 */
    const uint32_t rem = m & 0x1fffU;
    m >>= 13;
    if (rem > 0x1000U || (rem == 0x1000U && (m & 1U))) ++m;
    return (uint16_t)(sign | m);
}

OR_API float or_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000U) << 16;
    const uint32_t e = (h >> 10) & 0x1fU, m = h & 0x3ffU;
    if (e == 0) {
        const float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000U | (m << 13));
    return u2f(sign | ((e + 112U) << 23) | (m << 13));
}

static inline float t_to_f32(uint16_t v, int dtype) { return dtype ? or_f16_to_f32(v) : or_bf16_to_f32(v); }
static inline float t_round(float v, int dtype) {
    return dtype ? or_f16_to_f32(or_f32_to_f16_rne(v)) : bf16_round_f32(v);
}

/* Sum of squares of one head row (D channels) in the order the GPU uses:    */
/* packs of 8 channels each accumulate x*x by FMA from 0, then the D/8 pack  */
/* sums are combined by a butterfly: s[p] += s[p ^ off] for off = D/16 .. 1  */
/* (qk_preprocess.cu:530-537 uses the same order).                           */
static float head_sumsq(const uint16_t *row, int64_t dim, int dtype) {
    float s[16];
    const int packs = (int)(dim / 8);
    for (int p = 0; p < packs; ++p) {
        float acc = 0.0f;
        for (int c = 0; c < 8; ++c) {
            const float v = t_to_f32(row[p * 8 + c], dtype);
            acc = fmaf(v, v, acc);
        }
        s[p] = acc;
    }
    for (int off = packs / 2; off > 0; off >>= 1) {
        float t[16];
        for (int p = 0; p < packs; ++p) t[p] = s[p] + s[p ^ off];
        memcpy(s, t, sizeof(float) * (size_t)packs);
    }
    return s[0];
}

/* ------------------------------------------------------------------------ */
/* Fused Q/K RMSNorm + RoPE + per-tile INT8, one tensor (Q or K):            */
/* quantize_tile / processed_tile_value (qk_preprocess.cu:99-197, :417-552). */
/*   rrms  = 1 / sqrt(sumsq / n + eps)   head scope: n = D, sum of the head  */
/*           row (head_sumsq); row scope: n = H*D, the heads' head_sumsq      */
/*           added in head order (the reference uses rsqrtf; here IEEE)      */
/*   a_c   = T((x_c * rrms) * w)   w = norm[c] or norm[h*D + c]               */
/*   c < rot_dim: pair = split ? c mod pairs : c / 2, first/second = the     */
/*           pair's channels (split: pair, pair + pairs; else 2 pair, +1),   */
/*           comp = split ? c >= pairs : c & 1,                              */
/*           y_c = T(fma(f[pair][comp][1], a_second, f[pair][comp][0] * a_first)) */
/*   else  y_c = a_c                                                          */
/*   per tile of `tile` tokens: amax = max(1e-7, max |y|), scale = amax / 127 */
/*           q = clamp(rint(y * (127 / amax)), -127, 127)                     */
/* x: [B][H][L][D] contiguous (dtype 0 bf16, 1 fp16 bit patterns); freqs:    */
/* f32 [fb][fs][rot_dim/2][2][2] (fb, fs in {1, B}, {1, L}); q: [B][H][L][D];*/
/* scales: [B][H][ntiles] (tiles past L get 1e-7 / 127).                     */
/* ------------------------------------------------------------------------ */
OR_API void or_w8a8_hadamard(float *x, int dim);

/* Row-scope (norm_scope 1) or head-scope rrms of every (b, h, t), the      */
/* quantize path's order (head_sumsq; heads added in order).                 */
static void qk_rrms_all(const uint16_t *x, int dtype, int64_t batch, int64_t heads, int64_t len, int64_t dim,
                        int norm_scope, float eps, float *rrms) {
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t t = 0; t < len; ++t) {
            if (norm_scope) {
                float total = 0.0f;
                for (int64_t h = 0; h < heads; ++h)
                    total += head_sumsq(x + ((b * heads + h) * len + t) * dim, dim, dtype);
                const float r = 1.0f / sqrtf(total / (float)(heads * dim) + eps);
                for (int64_t h = 0; h < heads; ++h) rrms[(b * heads + h) * len + t] = r;
            } else {
                for (int64_t h = 0; h < heads; ++h) {
                    const float sq = head_sumsq(x + ((b * heads + h) * len + t) * dim, dim, dtype);
                    rrms[(b * heads + h) * len + t] = 1.0f / sqrtf(sq / (float)dim + eps);
                }
            }
        }
}

/* processed_value (qk_preprocess.cu:97-145): channel c of token row `row`   */
/* after RMSNorm (a = T((x rrms) w)) and RoPE (T(fma(f1, a2, f0 a1))).       */
static float qk_processed(const uint16_t *row, int dtype, int64_t c, float r, const uint16_t *norm,
                          int norm_scope, int64_t h, int64_t dim, const float *fr, int64_t rot_dim,
                          int split_half) {
    const int64_t pairs = rot_dim / 2;
    const int64_t wi = norm_scope ? h * dim + c : c;
    const float a = t_round((t_to_f32(row[c], dtype) * r) * t_to_f32(norm[wi], dtype), dtype);
    if (c >= rot_dim) return a;
    const int64_t pair = split_half ? (c < pairs ? c : c - pairs) : c / 2;
    const int64_t first = split_half ? pair : 2 * pair;
    const int64_t second = split_half ? pair + pairs : first + 1;
    const int comp = split_half ? (c >= pairs) : (int)(c & 1);
    const int64_t w0 = norm_scope ? h * dim + first : first;
    const int64_t w1 = norm_scope ? h * dim + second : second;
    const float x0 = t_round((t_to_f32(row[first], dtype) * r) * t_to_f32(norm[w0], dtype), dtype);
    const float x1 = t_round((t_to_f32(row[second], dtype) * r) * t_to_f32(norm[w1], dtype), dtype);
    const float f0 = fr[pair * 4 + comp * 2 + 0];
    const float f1 = fr[pair * 4 + comp * 2 + 1];
    return t_round(fmaf(f1, x1, f0 * x0), dtype);
}

/* Fused variant with the W8A8 transform (qk_preprocess.cu:417-563 with      */
/* Rotate / AllowAnchor): y = processed value; for K with anchor >= 0,       */
/* y -= anchor_values[c]; rotate: y = hadamard(y) per token; then the tile   */
/* amax / codes as above.  anchors / anchor_values: [B][H] / [B][H][D] or   */
/* NULL.                                                                     */
OR_API int or_qk_rms_rope_int8_ex(const uint16_t *x, int dtype, int64_t batch, int64_t heads, int64_t len,
                                  int64_t dim, const uint16_t *norm, int norm_scope, float eps,
                                  const float *freqs, int64_t fb, int64_t fs, int64_t rot_dim,
                                  int split_half, int64_t tile, int64_t ntiles, int rotate,
                                  const int32_t *anchors, const float *anchor_values, int8_t *q, float *scales) {
    if ((dim != 64 && dim != 128) || rot_dim < 0 || rot_dim > dim || (rot_dim & 1)) return -1;
    if (ntiles * tile < len) return -1;
    const int64_t pairs = rot_dim / 2;
    float *rrms = (float *)malloc(sizeof(float) * (size_t)(batch * heads * len));
    float *y = (float *)malloc(sizeof(float) * (size_t)(tile * dim));
    if (!rrms || !y) { free(rrms); free(y); return -2; }
    qk_rrms_all(x, dtype, batch, heads, len, dim, norm_scope, eps, rrms);
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < heads; ++h) {
            const int anchored = anchors && anchor_values && anchors[b * heads + h] >= 0;
            const float *av = anchored ? anchor_values + (b * heads + h) * dim : NULL;
            for (int64_t ti = 0; ti < ntiles; ++ti) {
                float amax = 0.0000001f;
                const int64_t t0 = ti * tile;
                for (int64_t to = 0; to < tile && t0 + to < len; ++to) {
                    const int64_t t = t0 + to;
                    const uint16_t *row = x + ((b * heads + h) * len + t) * dim;
                    const float r = rrms[(b * heads + h) * len + t];
                    const float *fr = freqs ? freqs + ((fb == 1 ? 0 : b) * fs + (fs == 1 ? 0 : t)) * pairs * 4 : NULL;
                    float *v = y + to * dim;
                    for (int64_t c = 0; c < dim; ++c) {
                        v[c] = qk_processed(row, dtype, c, r, norm, norm_scope, h, dim, fr, rot_dim, split_half);
                        if (av) v[c] -= av[c];
                    }
                    if (rotate) or_w8a8_hadamard(v, (int)dim);
                    for (int64_t c = 0; c < dim; ++c) amax = fmaxf(amax, fabsf(v[c]));
                }
                scales[(b * heads + h) * ntiles + ti] = amax / 127.0f;
                const float inv = 127.0f / amax;
                for (int64_t to = 0; to < tile && t0 + to < len; ++to)
                    for (int64_t c = 0; c < dim; ++c) {
                        float r = nearbyintf(y[to * dim + c] * inv);
                        r = fminf(127.0f, fmaxf(-127.0f, r));
                        q[((b * heads + h) * len + t0 + to) * dim + c] = (int8_t)r;
                    }
            }
        }
    free(rrms);
    free(y);
    return 0;
}

/* The processed values (RMSNorm + RoPE, rounded to T) of every token, fp32 */
/* [B][H][L][D]: the quantizer's input before the W8A8 transform.            */
OR_API int or_qk_processed(const uint16_t *x, int dtype, int64_t batch, int64_t heads, int64_t len, int64_t dim,
                           const uint16_t *norm, int norm_scope, float eps, const float *freqs, int64_t fb,
                           int64_t fs, int64_t rot_dim, int split_half, float *out) {
    const int64_t pairs = rot_dim / 2;
    float *rrms = (float *)malloc(sizeof(float) * (size_t)(batch * heads * len));
    if (!rrms) return -2;
    qk_rrms_all(x, dtype, batch, heads, len, dim, norm_scope, eps, rrms);
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t t = 0; t < len; ++t) {
                const uint16_t *row = x + ((b * heads + h) * len + t) * dim;
                const float *fr = freqs ? freqs + ((fb == 1 ? 0 : b) * fs + (fs == 1 ? 0 : t)) * pairs * 4 : NULL;
                for (int64_t c = 0; c < dim; ++c)
                    out[((b * heads + h) * len + t) * dim + c] =
                        qk_processed(row, dtype, c, rrms[(b * heads + h) * len + t], norm, norm_scope, h, dim, fr,
                                     rot_dim, split_half);
            }
    free(rrms);
    return 0;
}

OR_API int or_qk_rms_rope_int8(const uint16_t *x, int dtype, int64_t batch, int64_t heads, int64_t len,
                               int64_t dim, const uint16_t *norm, int norm_scope, float eps,
                               const float *freqs, int64_t fb, int64_t fs, int64_t rot_dim,
                               int split_half, int64_t tile, int64_t ntiles, int8_t *q, float *scales) {
    return or_qk_rms_rope_int8_ex(x, dtype, batch, heads, len, dim, norm, norm_scope, eps, freqs, fb, fs, rot_dim,
                                  split_half, tile, ntiles, 0, NULL, NULL, q, scales);
}


/* ======================================================================== */
/* W8A8 attention variant (loader default `w8a8` backend).                   */
/* ======================================================================== */

/* Sign diagonal of the shared Q/K Hadamard transform: channel c is negated  */
/* when bit (c & 31) of word c >> 5 is 0 (fused.cu:206-212).                 */
static const uint32_t kW8a8Signs[4] = {0x1035997bu, 0x8087f5eeu, 0xee2e4e1au, 0x71132418u};

OR_API int or_w8a8_sign_negative(int channel) {
    return ((kW8a8Signs[channel >> 5] >> (channel & 31)) & 1u) == 0u;
}

/* Randomized normalised Walsh-Hadamard transform of one head row in place   */
/* (attention_hadamard8, fused.cu:214-260), exact fp32 operation order:      */
/*   x_c = -x_c for negative-sign channels;                                  */
/*   within each pack of 8 channels, spans 1, 2, 4: (l, r) -> (l + r, l - r);*/
/*   across packs (pack index bits 1, 2, 4 [, 8]): the pack without the bit  */
/*   takes mine + other, the pack with it other - mine, from the old values; */
/*   finally x_c *= 1/8 (D = 64) or 0.08838834764831845f (D = 128).           */
OR_API void or_w8a8_hadamard(float *x, int dim) {
    const int packs = dim / 8;
    for (int c = 0; c < dim; ++c)
        if (or_w8a8_sign_negative(c)) x[c] = -x[c];
    for (int p = 0; p < packs; ++p) {
        float *v = x + 8 * p;
        for (int span = 1; span < 8; span <<= 1)
            for (int base = 0; base < 8; base += 2 * span)
                for (int o = 0; o < span; ++o) {
                    const float l = v[base + o], r = v[base + o + span];
                    v[base + o] = l + r;
                    v[base + o + span] = l - r;
                }
    }
    for (int bit = 1; bit < packs; bit <<= 1) {
        float old[128];
        memcpy(old, x, sizeof(float) * (size_t)dim);
        for (int p = 0; p < packs; ++p)
            for (int j = 0; j < 8; ++j) {
                const float mine = old[8 * p + j], other = old[8 * (p ^ bit) + j];
                x[8 * p + j] = (p & bit) ? other - mine : mine + other;
            }
    }
    const float norm = dim == 64 ? 0.125f : 0.08838834764831845f;
    for (int c = 0; c < dim; ++c) x[c] *= norm;
}

/* Lane-0 result of a 32-lane shfl_down tree (offsets 16, 8, 4, 2, 1): the   */
/* order the reference's warp reductions produce.                            */
static float tree32_sum(const float *v) {
    float t[32];
    memcpy(t, v, sizeof(t));
    for (int off = 16; off > 0; off >>= 1)
        for (int i = 0; i < off; ++i) t[i] = t[i] + t[i + off];
    return t[0];
}
static float tree32_max(const float *v) {
    float t[32];
    memcpy(t, v, sizeof(t));
    for (int off = 16; off > 0; off >>= 1)
        for (int i = 0; i < off; ++i) t[i] = fmaxf(t[i], t[i + off]);
    return t[0];
}

/* K stabilisation anchor of one (batch, kv head): DetectKAnchorKernel       */
/* (fused.cu:409-575).  Nine keys at rows s (L - 1) / 8 (integer division)   */
/* are sampled; per channel c (one of 128 threads, 4 warps of 32):           */
/*   E_c   = fma chain of x^2 over the samples, M_c = max |x|,               */
/*   S_c   = sequential sum of the samples,                                  */
/*   dist_c[j] = fma(9 x_j - S_c, 9 x_j - S_c, 0);                            */
/* the totals are warp trees (tree32_*) added warp 0..3 from 0.              */
/* The candidate with the smallest total distance (first on ties) is the    */
/* anchor; with r = x - anchor, E' and M' are formed the same way, and the  */
/* anchor row is kept iff E' < E and M' <= M * 1.125f, else -1.             */
/* x: dtype 0 bf16 / 1 fp16 bit patterns, channel stride 1; dim <= 128.      */
/* The detector's decision on nine sample rows (channels >= dim are 0):     */
/* the selected sample (0..8) when centring on it helps, else -1.            */
static int anchor_decide(float samples[9][128], int64_t dim) {
    float e_lane[128], m_lane[128], d_lane[9][128], be_lane[128], bm_lane[128];
    for (int c = 0; c < 128; ++c) {
        float e = 0.0f, m = 0.0f, sum = 0.0f;
        for (int j = 0; j < 9; ++j) d_lane[j][c] = 0.0f;
        if (c < dim) {
            for (int s = 0; s < 9; ++s) {
                const float v = samples[s][c];
                e = fmaf(v, v, e);
                m = fmaxf(m, fabsf(v));
                sum += v;
            }
            for (int j = 0; j < 9; ++j) {
                const float d = 9.0f * samples[j][c] - sum;
                d_lane[j][c] = fmaf(d, d, 0.0f);
            }
        }
        e_lane[c] = e;
        m_lane[c] = m;
    }
    float tot_e = 0.0f, tot_m = 0.0f, dist[9];
    for (int w = 0; w < 4; ++w) {
        tot_e += tree32_sum(e_lane + 32 * w);
        tot_m = fmaxf(tot_m, tree32_max(m_lane + 32 * w));
    }
    int best = 0;
    float best_d = 3.402823466e+38F;
    for (int j = 0; j < 9; ++j) {
        dist[j] = 0.0f;
        for (int w = 0; w < 4; ++w) dist[j] += tree32_sum(d_lane[j] + 32 * w);
        if (dist[j] < best_d) {
            best = j;
            best_d = dist[j];
        }
    }
    for (int c = 0; c < 128; ++c) {
        float e = 0.0f, m = 0.0f;
        if (c < dim) {
            const float a = samples[best][c];
            for (int s = 0; s < 9; ++s) {
                const float r = samples[s][c] - a;
                e = fmaf(r, r, e);
                m = fmaxf(m, fabsf(r));
            }
        }
        be_lane[c] = e;
        bm_lane[c] = m;
    }
    float tot_be = 0.0f, tot_bm = 0.0f;
    for (int w = 0; w < 4; ++w) {
        tot_be += tree32_sum(be_lane + 32 * w);
        tot_bm = fmaxf(tot_bm, tree32_max(bm_lane + 32 * w));
    }
    const int improves = tot_be < tot_e && tot_bm <= tot_m * 1.125f;
    return improves ? best : -1;
}

OR_API int32_t or_w8a8_detect_anchor(const uint16_t *x, int dtype, int64_t len, int64_t dim, int64_t s_l) {
    float samples[9][128];
    if (dim > 128 || dim <= 0 || len <= 0) return -2;
    for (int s = 0; s < 9; ++s) {
        const int64_t row = (int64_t)s * (len - 1) / 8;
        for (int c = 0; c < 128; ++c) samples[s][c] = c < dim ? t_to_f32(x[row * s_l + c], dtype) : 0.0f;
    }
    const int sel = anchor_decide(samples, dim);
    return sel >= 0 ? (int32_t)((int64_t)sel * (len - 1) / 8) : -1;
}

/* K anchor of the fused preprocessor: detect_anchor_kernel                  */
/* (qk_preprocess.cu:250-416).  The nine samples are the processed values    */
/* (RMSNorm + RoPE, rounded to T) of rows s (L - 1) / 8; their rrms is the   */
/* row-scope rrms, or for head scope 1 / sqrt(S / D + eps) with S a          */
/* sequential fma chain over the head's D channels (the reference uses      */
/* rsqrtf; here IEEE).  The decision is anchor_decide; anchor_values        */
/* [B][H][D] = the selected sample's values, or 0 when none is kept.         */
OR_API int or_qk_fused_anchor(const uint16_t *x, int dtype, int64_t batch, int64_t heads, int64_t len,
                              int64_t dim, const uint16_t *norm, int norm_scope, float eps, const float *freqs,
                              int64_t fb, int64_t fs, int64_t rot_dim, int split_half, int32_t *anchors,
                              float *anchor_values) {
    if ((dim != 64 && dim != 128) || len <= 0) return -1;
    const int64_t pairs = rot_dim / 2;
    float *rrms = (float *)malloc(sizeof(float) * (size_t)(batch * heads * len));
    if (!rrms) return -2;
    if (norm_scope) qk_rrms_all(x, dtype, batch, heads, len, dim, 1, eps, rrms);
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < heads; ++h) {
            float samples[9][128];
            for (int sm = 0; sm < 9; ++sm) {
                const int64_t t = (int64_t)sm * (len - 1) / 8;
                const uint16_t *row = x + ((b * heads + h) * len + t) * dim;
                float r;
                if (norm_scope) {
                    r = rrms[(b * heads + h) * len + t];
                } else {
                    float sq = 0.0f;
                    for (int64_t c = 0; c < dim; ++c) {
                        const float v = t_to_f32(row[c], dtype);
                        sq = fmaf(v, v, sq);
                    }
                    r = 1.0f / sqrtf(sq / (float)dim + eps);
                }
                const float *fr = freqs ? freqs + ((fb == 1 ? 0 : b) * fs + (fs == 1 ? 0 : t)) * pairs * 4 : NULL;
                for (int c = 0; c < 128; ++c)
                    samples[sm][c] = c < dim ? qk_processed(row, dtype, c, r, norm, norm_scope, h, dim, fr, rot_dim,
                                                            split_half)
                                             : 0.0f;
            }
            const int sel = anchor_decide(samples, dim);
            anchors[b * heads + h] = sel >= 0 ? (int32_t)((int64_t)sel * (len - 1) / 8) : -1;
            for (int64_t c = 0; c < dim; ++c) anchor_values[(b * heads + h) * dim + c] = sel >= 0 ? samples[sel][c] : 0.0f;
        }
    free(rrms);
    return 0;
}

/* Rotated per-tile INT8 of one tensor (Q or K): quant_int8_tile             */
/* (fused.cu:262-407) as launched by QuantQKInt8Kernel (:577-636).           */
/*   v     = float(x) - float(x[anchor row]) (K only, when anchor >= 0)      */
/*   v     = hadamard(v) when rotate                                         */
/*   amax  = max(1e-7, max |v| over the tile's tokens x channels)            */
/*   scale = amax / 127,  q = cvt.rni.sat.s8(v * (127 / amax))               */
/* Tiles of `tile` tokens (Q: 16, K: 64); tiles past L get 1e-7 / 127.       */
/* x: [B][H][L][D] with strides (channel stride 1); anchors: [B][H] or NULL; */
/* q: [B][H][L][D] contiguous; scales: [B][H][ntiles].                       */
OR_API int or_w8a8_quant_tiles(const uint16_t *x, int dtype, int64_t batch, int64_t heads, int64_t len,
                               int64_t dim, int64_t s_b, int64_t s_h, int64_t s_l, int64_t tile, int64_t ntiles,
                               int rotate, const int32_t *anchors, int8_t *q, float *scales) {
    if ((dim != 64 && dim != 128) || ntiles * tile < len) return -1;
    float *y = (float *)malloc(sizeof(float) * (size_t)(tile * dim));
    if (!y) return -2;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < heads; ++h) {
            const uint16_t *xb = x + b * s_b + h * s_h;
            const int32_t anchor = anchors ? anchors[b * heads + h] : -1;
            for (int64_t ti = 0; ti < ntiles; ++ti) {
                float amax = 0.0000001f;
                const int64_t t0 = ti * tile;
                for (int64_t to = 0; to < tile && t0 + to < len; ++to) {
                    float *v = y + to * dim;
                    for (int64_t c = 0; c < dim; ++c) {
                        v[c] = t_to_f32(xb[(t0 + to) * s_l + c], dtype);
                        if (anchor >= 0) v[c] -= t_to_f32(xb[(int64_t)anchor * s_l + c], dtype);
                    }
                    if (rotate) or_w8a8_hadamard(v, (int)dim);
                    for (int64_t c = 0; c < dim; ++c) amax = fmaxf(amax, fabsf(v[c]));
                }
                scales[(b * heads + h) * ntiles + ti] = amax / 127.0f;
                const float mult = 127.0f / amax;
                for (int64_t to = 0; to < tile && t0 + to < len; ++to)
                    for (int64_t c = 0; c < dim; ++c)
                        q[((b * heads + h) * len + t0 + to) * dim + c] = sat_rne_s8(y[to * dim + c] * mult);
            }
        }
    free(y);
    return 0;
}

/* Channel-wise signed INT8 V: quantize_value_kernel                         */
/* (quant_v_int8_cuda_sm75.cu:58-164).                                       */
/*   scale[c] = max(amax_c / 127, 1e-12)  (amax over all L tokens)           */
/*   q[c][t]  = cvt.rni.sat.s8(float(v[t][c]) * (1 / scale[c]))              */
/* Output layout (this build's, channel-major with keys in natural order):   */
/* q [B][H][D][lpad] with zeros for t >= L.  The reference permutes keys     */
/* within groups of 16 for its Turing MMA fragment; the codes are the same.  */
OR_API int or_w8a8_quant_v(const uint16_t *v, int dtype, int64_t batch, int64_t heads, int64_t len, int64_t dim,
                           int64_t s_b, int64_t s_h, int64_t s_l, int64_t lpad, int8_t *q, float *scale) {
    if (lpad < len || lpad % 64) return -1;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t h = 0; h < heads; ++h) {
            const uint16_t *vb = v + b * s_b + h * s_h;
            for (int64_t c = 0; c < dim; ++c) {
                float amax = 0.0f;
                for (int64_t t = 0; t < len; ++t) amax = fmaxf(amax, fabsf(t_to_f32(vb[t * s_l + c], dtype)));
                const float sc = fmaxf(amax / 127.0f, 1.0e-12f);
                const float inv = 1.0f / sc;
                scale[(b * heads + h) * dim + c] = sc;
                int8_t *qc = q + ((b * heads + h) * dim + c) * lpad;
                for (int64_t t = 0; t < lpad; ++t)
                    qc[t] = t < len ? sat_rne_s8(t_to_f32(vb[t * s_l + c], dtype) * inv) : 0;
            }
        }
    return 0;
}

/* cvt.rni.sat.u8.f32 (attn_utils.cuh:588-597): round half to even, clamp to */
/* [0, 255], NaN -> 0.                                                       */
static inline int sat_rne_u8(float v) {
    if (v != v) return 0;
    float r = nearbyintf(v);
    if (r > 255.0f) r = 255.0f;
    if (r < 0.0f) r = 0.0f;
    return (int)r;
}

/* Dense W8A8 attention rows: the ForceDense/UseW8A8 specialisation of       */
/* sparse_attention_kernel (sol_sparse_cuda_sm75.cu:1182-1322) with          */
/* update_mdo(exp_offset) / RS_to_u8 / accumulate_d / compute_int8_sv /      */
/* normalize_d (attn_utils.cuh:31-34, :436-568, :588-623, :676-703,          */
/* :791-841, :920-973).  Per query row, key blocks of 64 in order:           */
/*   s_j   = float(q8 . k8_j); masked (j >= Lk, causal j > i) -> -5e6        */
/*   f     = (sm_scale * log2 e) * q_scale * k_scale[block]                  */
/*   m'    = max(m, fma(max_j s_j, f, -log2 255))    (m starts at -5e6)      */
/*   a     = 2^(m - m'); d = d * a; O = O * a                                */
/*   p_j   = 2^(fma(s_j, f, -m')),  P_j = cvt.rni.sat.u8(p_j)                */
/*   d    += sum p_j (the unquantised p),  O_c += float(sum_j P_j v8_j[c])   */
/* out_c = O_c * (1 / d) * v_scale[c], fp32 (the caller rounds to the output */
/* dtype).  exp2 / reciprocal are the exact libm forms (the reference uses   */
/* ex2.approx / rcp.approx).  d starts at 1 like the reference; the first    */
/* block's a = 2^(-5e6 - m') is 0.  q_scale: [B][Hq][nqs] with one scale per */
/* 16 query rows; k_scale: [B][Hkv][nks] per 64 keys; v8: [B][Hkv][D][lpad]; */
/* v_scale: [B][Hkv][D].  Rows are (b, h, i) triples; out is [nrows][D].     */
OR_API int or_w8a8_attn_rows(const int8_t *q8, int64_t q_sb, int64_t q_sh, int64_t q_sl, const float *qs,
                             int64_t nqs, const int8_t *k8, int64_t k_sb, int64_t k_sh, int64_t k_sl,
                             const float *ks, int64_t nks, const int8_t *v8, int64_t lpad, const float *vs,
                             int64_t hq, int64_t hkv, int64_t lq, int64_t lk, int64_t dim, float sm_scale,
                             int causal, const int64_t *rows, int64_t nrows, float *out) {
    (void)lq;
    const float scale_log2 = sm_scale * 1.44269504088896340736f;
    const float offset = 7.9943534f;
    const int64_t groups = hq / hkv;
    const int64_t nblk = (lk + 63) / 64;
    if (lpad < nblk * 64 || nks < nblk) return -1;
#pragma omp parallel
    {
        float *o = (float *)malloc(sizeof(float) * (size_t)dim);
        float s[64];
        int pq[64];
#pragma omp for schedule(dynamic)
        for (int64_t r = 0; r < nrows; ++r) {
            const int64_t b = rows[3 * r], h = rows[3 * r + 1], i = rows[3 * r + 2];
            const int64_t hk = h / groups;
            const int8_t *qi = q8 + b * q_sb + h * q_sh + i * q_sl;
            const float qscale = qs[(b * hq + h) * nqs + i / 16];
            const float *ksr = ks + (b * hkv + hk) * nks;
            const int8_t *vh = v8 + (b * hkv + hk) * dim * lpad;
            const int64_t blocks = causal ? (i / 64 + 1 < nblk ? i / 64 + 1 : nblk) : nblk;
            float m = -5000000.0f, d = 1.0f;
            for (int64_t c = 0; c < dim; ++c) o[c] = 0.0f;
            for (int64_t blk = 0; blk < blocks; ++blk) {
                float mx = -5000000.0f;
                for (int j = 0; j < 64; ++j) {
                    const int64_t key = 64 * blk + j;
                    float sv = -5000000.0f;
                    if (key < lk && !(causal && key > i)) {
                        const int8_t *kj = k8 + b * k_sb + hk * k_sh + key * k_sl;
                        int32_t acc = 0;
                        for (int64_t c = 0; c < dim; ++c) acc += (int32_t)qi[c] * (int32_t)kj[c];
                        sv = (float)acc;
                    }
                    s[j] = sv;
                    mx = fmaxf(mx, sv);
                }
                const float f = (scale_log2 * qscale) * ksr[blk];
                const float m_new = fmaxf(m, fmaf(mx, f, -offset));
                const float a = exp2f(m - m_new);
                d *= a;
                for (int64_t c = 0; c < dim; ++c) o[c] *= a;
                for (int j = 0; j < 64; ++j) {
                    const float p = exp2f(fmaf(s[j], f, -m_new));
                    pq[j] = sat_rne_u8(p);
                    d += p;
                }
                for (int64_t c = 0; c < dim; ++c) {
                    int32_t acc = 0;
                    for (int j = 0; j < 64; ++j) acc += pq[j] * (int32_t)vh[c * lpad + 64 * blk + j];
                    o[c] += (float)acc;
                }
                m = m_new;
            }
            const float rd = 1.0f / d;
            for (int64_t c = 0; c < dim; ++c) out[r * dim + c] = (o[c] * rd) * vs[(b * hkv + hk) * dim + c];
        }
        free(o);
    }
    return 0;
}

/* ======================================================================== */
/* Wan block: LayerNorm + AdaLN modulation.                                  */
/* ======================================================================== */

typedef struct { float mean, m2; int count; } or_welford;

/* welford_combine (segmented_rms_adaln.cu:87-101). */
static or_welford welford_combine(or_welford l, or_welford r) {
    if (r.count == 0) return l;
    if (l.count == 0) return r;
    const int count = l.count + r.count;
    const float delta = r.mean - l.mean;
    l.mean = l.mean + (delta * (float)r.count) / (float)count;
    l.m2 = l.m2 + (r.m2 + (((delta * delta) * (float)l.count) * (float)r.count) / (float)count);
    l.count = count;
    return l;
}

/* layer_norm_adaln_kernel (segmented_rms_adaln.cu:236-307), one row:       */
/*   256 threads, thread t takes columns t, t + 256, ... in order:           */
/*     count++, delta = v - mean, mean += delta / count,                     */
/*     m2 = fma(delta, v - mean, m2)   (nvcc contracts the reference's      */
/*                                      m2 += delta * (v - mean))           */
/*   32-lane shfl_down trees of welford_combine, the 8 tree results combined */
/*   in order from {0, 0, 0};  var = m2 / count, inv = 1 / sqrt(var + eps)   */
/*   (the reference uses rsqrtf; here IEEE)                                  */
/*   out = T(fma(T((x - mean) inv), T(1 + scale), shift))                    */
/*   (the reference's float a * b + c, contracted).                          */
/* Modulation row of token t: steps == 1 -> 0; else group = ceil-ish        */
/* repeats (L / steps, + 1 when it does not divide), row = min(t / group,   */
/* steps - 1).  x/out: [B][L][H]; scale/shift: [B][steps][H]; dtype 0 bf16,  */
/* 1 fp16 (2-byte patterns), 2 fp32 (T rounding is then the identity).       */
static inline float ln_load(const void *p, int64_t i, int dtype) {
    return dtype == 2 ? ((const float *)p)[i] : t_to_f32(((const uint16_t *)p)[i], dtype);
}
static inline float ln_round(float v, int dtype) { return dtype == 2 ? v : t_round(v, dtype); }

/* affine != 0: LayerNorm with an elementwise affine weight w and bias b    */
/* (scale / shift carry w / b, one row for every token): out = T(fma(       */
/* (x - mean) inv, w, b)), the normalized value not rounded -- the          */
/* single-rounding form of torch's layer_norm, which ComfyUI runs for the   */
/* Wan block's norm3 (the reference leaves that norm to ComfyUI).            */
static int layer_norm_rows(const void *x, int dtype, int64_t batch, int64_t len, int64_t hidden,
                           const void *scale, const void *shift, int64_t steps, float eps, int affine, void *out) {
    if (hidden <= 0 || steps <= 0) return -1;
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < batch * len; ++row) {
        const int64_t b = row / len, t = row % len;
        int64_t mt = 0;
        if (steps > 1) {
            const int64_t repeats = len / steps;
            const int64_t group = repeats * steps == len ? repeats : repeats + 1;
            mt = t / (group > 1 ? group : 1);
            if (mt > steps - 1) mt = steps - 1;
        }
        const int64_t xr = row * hidden;
        or_welford lane[256];
        for (int th = 0; th < 256; ++th) {
            or_welford w = {0.0f, 0.0f, 0};
            for (int64_t c = th; c < hidden; c += 256) {
                const float v = ln_load(x, xr + c, dtype);
                ++w.count;
                const float delta = v - w.mean;
                w.mean = w.mean + delta / (float)w.count;
                w.m2 = fmaf(delta, v - w.mean, w.m2);
            }
            lane[th] = w;
        }
        or_welford total = {0.0f, 0.0f, 0};
        for (int wp = 0; wp < 8; ++wp) {
            or_welford *v = lane + 32 * wp;
            or_welford tmp[32];
            memcpy(tmp, v, sizeof(tmp));
            for (int off = 16; off > 0; off >>= 1)
                for (int i = 0; i < off; ++i) tmp[i] = welford_combine(tmp[i], tmp[i + off]);
            total = welford_combine(total, tmp[0]);
        }
        const float mean = total.mean;
        const float var = total.m2 / (float)total.count;
        const float inv = 1.0f / sqrtf(var + eps);
        const int64_t mrow = (b * steps + mt) * hidden;
        for (int64_t c = 0; c < hidden; ++c) {
            float r;
            if (affine) {
                r = fmaf((ln_load(x, xr + c, dtype) - mean) * inv, ln_load(scale, mrow + c, dtype),
                         ln_load(shift, mrow + c, dtype));
            } else {
                const float n = ln_round((ln_load(x, xr + c, dtype) - mean) * inv, dtype);
                const float m = ln_round(1.0f + ln_load(scale, mrow + c, dtype), dtype);
                r = fmaf(n, m, ln_load(shift, mrow + c, dtype));
            }
            if (dtype == 2) ((float *)out)[xr + c] = r;
            else ((uint16_t *)out)[xr + c] = dtype ? or_f32_to_f16_rne(r) : or_f32_to_bf16_rne(r);
        }
    }
    return 0;
}

OR_API int or_layer_norm_adaln(const void *x, int dtype, int64_t batch, int64_t len, int64_t hidden,
                               const void *scale, const void *shift, int64_t steps, float eps, void *out) {
    return layer_norm_rows(x, dtype, batch, len, hidden, scale, shift, steps, eps, 0, out);
}

/* rows x hidden, one weight / bias row of hidden values for all rows. */
OR_API int or_layer_norm_affine(const void *x, int dtype, int64_t rows, int64_t hidden, const void *weight,
                                const void *bias, float eps, void *out) {
    return layer_norm_rows(x, dtype, 1, rows, hidden, weight, bias, 1, eps, 1, out);
}
