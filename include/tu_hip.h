/*
 * tu_hip.h -- C ABI of the MI355X (gfx950) kernels for the quantized DiT hot
 * path of comfyui-turing-utils: ConvRot W8A8 linear and Sage INT8 attention.
 *
 * Library: libtu_hip.so (comfyui-turing-utils_amd/comfyui_turing_utils_kernel/).
 *
 * Conventions
 *   - Every pointer is a device pointer on the current HIP device, except
 *     where noted.  bf16 tensors are passed as `const void *` holding IEEE
 *     bfloat16 bit patterns.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Work is
 *     enqueued asynchronously; nothing synchronises.
 *   - The return value is 0 on success.  A non-zero value means nothing was
 *     launched (argument or device check failed) or the launch failed; the
 *     message is available from tu_last_error() on the same host thread.
 *   - Strides are in elements.  The innermost (channel) dimension must be
 *     contiguous.
 *   - No entry point allocates device memory: outputs and scratch are
 *     provided by the caller.
 *
 * Each entry point names the reference interface it replaces.  Paths are
 * relative to the reference tree.
 */
#ifndef TU_HIP_H_
#define TU_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status / introspection ------------------------------------------------- */

/* Message of the last failed call on this host thread ("" if none). */
const char *tu_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int32_t tu_abi_version(void);

/* 1 if `device` is a gfx950 (MI355X-class) GPU this library was built for,
 * 0 otherwise; negative on a HIP error.  Replaces the sm75 predicate
 * comfyui_turing_utils/hardware.py:24-32. */
int32_t tu_device_supported(int32_t device);

/* ConvRot INT8 activation quantizer -------------------------------------- */

/* Input activation applied on load (low byte of `act`). */
#define TU_ACT_NONE 0      /* a = x */
#define TU_ACT_GELU_TANH 1 /* a = bf16(0.5x(1 + tanh(0.7978845608028654(x + 0.044715x^3)))) */
#define TU_ACT_SWIGLU 2    /* a = silu(gate) * up; x rows are [gate | up], 2*cols wide */
/* OR-ed into `act`: scale = absmax * (1/127) (the two-pass kernels' formula,
 * convrot_quant.cu:233-236) instead of absmax / 127. */
#define TU_CONVROT_STAGED_SCALE 0x100
/* OR-ed into `act`: x holds IEEE fp16 instead of bf16, as the reference's
 * two-pass kernels with InputType = half (convrot_quant.cu:158-248): the GELU
 * output and the rotated values are rounded to fp16, the absmax clip is 65504
 * and q = clamp(rne(fp16(fp16(y) / fp16(scale))), -128, 127) with IEEE
 * division (quant_div_to_float, convrot_quant.cu:69-73). */
#define TU_CONVROT_FP16_INPUT 0x200

/* Rotates each row of the activated input a = act(x) by the block-Hadamard
 * ConvRot transform (group 128 or 256), then quantizes per row to symmetric
 * INT8:
 *   y        = rotate(a) in fp32, absmax_r = max |y[r][:]|
 *   scale[r] = max(min(absmax_r, 3.38953139e38) / 127, 1e-30)
 *   q[r][c]  = clamp(rne(bf16(bf16(y[r][c]) / bf16(scale[r]))), -128, 127)
 * x: bf16 [rows, cols] (TU_ACT_SWIGLU: [rows, 2*cols]), row-major contiguous.
 * q: int8 [rows, cols]; scale: fp32 [rows].  cols % group == 0, cols <= 65536;
 * x and q 16-byte aligned.  tanh and exp inside the activations are fixed
 * fp32 sequences (range reduction by ln2 and a degree-7 Taylor polynomial;
 * tanh(u) = 1 - 2/(e^2u + 1)), bit-identical to the CPU oracle.
 * Replaces turing_utils::bf16_int8_convrot_quantize (act 0 and 2;
 * kernel/comfyui_turing_utils_kernel/ops.py:257-282 ->
 * kernel/csrc/bindings.cpp:603-646 -> kernel/csrc/turing/convrot_quant.cu:566-589),
 * turing_utils::bf16_gelu_int8_convrot_quantize (act 1; ops.py:313-331 ->
 * convrot_quant.cu:145-156, :332-344, :616-630) and, with
 * TU_CONVROT_STAGED_SCALE, turing_utils::gelu_int8_convrot_quantize /
 * swiglu_int8_convrot_quantize (ops.py:163-186, :215-233 ->
 * bindings.cpp:474-510, :550-600 -> convrot_quant.cu:158-248, :470-563). */
int32_t tu_convrot_quant_i8(const void *x_bf16, int8_t *q, float *scale, int64_t rows,
                            int64_t cols, int32_t group, int32_t act, void *stream);

/* INT8 GEMM ---------------------------------------------------------------- */

/* out[m][n] = bf16_rn(((float(acc) * a_scale[m]) * w_scale[n]) + bias[n]),
 * acc[m][n] = sum_k a[m][k] * w[n][k] (exact int32).
 * a: int8 [m, k] row-major; w: int8 [n, k] row-major; a_scale: fp32 [m];
 * w_scale: fp32 [n]; bias: fp32 [n] or NULL; out: bf16 [m, n] row-major.
 * Requires k % 16 == 0 and n % 8 == 0 (the reference's constraint).
 * Replaces turing_utils::int8_linear (ops.py:96-126 -> bindings.cpp:371-421
 * -> kernel/csrc/turing/w4a8.cu:1185-1219). */
int32_t tu_int8_gemm_bf16(const int8_t *a, const int8_t *w, const float *a_scale,
                          const float *w_scale, const float *bias, void *out_bf16, int64_t m,
                          int64_t n, int64_t k, void *stream);

/* The same GEMM and epilogue value, written as fp16 rounded once from fp32
 * (round-to-nearest-even, overflow to +-inf, fp16 subnormals kept, every NaN
 * as 0x7e00): out: fp16 [m, n] row-major.  Replaces the fp16 output_dtype of
 * the plugin's W8A8 GEMM call (comfyui_turing_utils/quantization/
 * dispatch.py:538-615, output_dtype = out_dtype or x.dtype at :660-668),
 * which the reference serves through comfy-kitchen's fused INT8 linear. */
int32_t tu_int8_gemm_f16(const int8_t *a, const int8_t *w, const float *a_scale,
                         const float *w_scale, const float *bias, void *out_f16, int64_t m,
                         int64_t n, int64_t k, void *stream);

/* The same epilogue value unrounded: out: fp32 [m, n] row-major, the fp32
 * output_dtype of the same call (dispatch.py:538-615, :660-668). */
int32_t tu_int8_gemm_f32(const int8_t *a, const int8_t *w, const float *a_scale,
                         const float *w_scale, const float *bias, float *out, int64_t m,
                         int64_t n, int64_t k, void *stream);

/* Output types and tile policies of tu_int8_gemm_ex. */
#define TU_OUT_BF16 0
#define TU_OUT_F16 1
#define TU_OUT_F32 2
#define TU_OUT_I32 3
#define TU_GEMM_TILE_AUTO 0 /* chosen from the grid: tu_int8_gemm_tile_policy */
#define TU_GEMM_TILE_256 1  /* 256 x 256 output tiles */
#define TU_GEMM_TILE_128 2  /* 128 (rows of a) x 256 output tiles */
#define TU_GEMM_TILE_192 3  /* 256 (rows of a) x 192 output tiles */

/* The GEMM above with its output type and tile policy as arguments: out_type
 * TU_OUT_BF16 / _F16 / _F32 as tu_int8_gemm_bf16 / _f16 / _f32, TU_OUT_I32 as
 * tu_int8_gemm_i32 (scales and bias ignored, may be NULL).  Every tile policy
 * gives the same bits.  Replaces the low-level binding's tile_policy argument
 * (kernel/csrc/bindings.cpp:872-879 -> kernel/csrc/turing/w4a8.cu:799-858,
 * where policy 0 is the heuristic and 1-5 force a CUTLASS tile). */
int32_t tu_int8_gemm_ex(const int8_t *a, const int8_t *w, const float *a_scale, const float *w_scale,
                        const float *bias, void *out, int32_t out_type, int64_t m, int64_t n, int64_t k,
                        int32_t tile_policy, void *stream);

/* The tile policy TU_GEMM_TILE_AUTO picks for an m x n output on a device
 * with `cus` compute units: TU_GEMM_TILE_128 or TU_GEMM_TILE_192 when that
 * tile's rounds of `cus` workgroups cost less than the 256 x 256 tiles'
 * (host only, no HIP call).  Counterpart of the heuristic of
 * w4a8.cu:837-851. */
int32_t tu_int8_gemm_tile_policy(int64_t m, int64_t n, int32_t cus);

/* The same GEMM with a gated residual add fused into the epilogue, for a DiT
 * block's x + y * gate: out[m][n] = bf16_rn(fma(y, g, residual[m][n])) with
 * y the tu_int8_gemm_bf16 value above, g = gate[m / gate_rows][n] (bf16 [G, n],
 * one row per gate_rows consecutive output rows, e.g. per batch entry) or 1
 * when gate is NULL (then exactly bf16_rn(y + residual)).  residual: bf16
 * [m, n], may be out (in place); residual, gate 16-byte aligned.
 * No counterpart in the reference's ops: it fuses the torch add / addcmul
 * that a ComfyUI Wan block (the caller of comfyui_turing_utils/adapters/
 * wan.py:55-137) runs after the o and FFN-down projections. */
int32_t tu_int8_gemm_bf16_residual(const int8_t *a, const int8_t *w, const float *a_scale,
                                   const float *w_scale, const float *bias, const void *residual_bf16,
                                   const void *gate_bf16, int64_t gate_rows, void *out_bf16, int64_t m,
                                   int64_t n, int64_t k, void *stream);

/* acc[m][n] = sum_k a[m][k] * w[n][k] as int32, row-major [m, n].  Same
 * kernel as tu_int8_gemm_bf16 with the epilogue replaced by an int32 store;
 * the accumulator half of the reference's cuBLAS INT8 + epilogue split
 * (comfyui_turing_utils/quantization/dispatch.py:481-535). */
int32_t tu_int8_gemm_i32(const int8_t *a, const int8_t *w, int32_t *acc, int64_t m, int64_t n,
                         int64_t k, void *stream);

/* out[m][n] = bf16_rn((float(acc[m*acc_ld + n]) * a_scale[m]) * w_scale[ws_scalar ? 0 : n])
 * for n < cols.  Replaces turing_utils::dequantize_int8_bf16 (ops.py:129-160
 * -> bindings.cpp:423-472 -> kernel/csrc/turing/bf16_epilogue.cu:147-218). */
int32_t tu_dequant_i32_bf16(const int32_t *acc, int64_t acc_ld, const float *a_scale,
                            const float *w_scale, int32_t ws_scalar, void *out_bf16, int64_t m,
                            int64_t cols, void *stream);

/* Sage attention: Q/K quantization ---------------------------------------- */

/* Per-(batch, head) channel mean of K over the sequence, rounded to bf16,
 * with a fixed fp32 summation order (128-token chunks; see the oracle
 * or_sage_kmean).  k: bf16, element strides (s_b, s_h, s_l), channels
 * contiguous; dim in {64, 128}.  chunk_sums: fp32 scratch of
 * batch*heads*ceil(len/128)*dim elements.  mean: bf16 [batch, heads, dim].
 * Smoothing is the `sub_mean` path of QuantInt8Kernel
 * (kernel/csrc/turing/sage/fused.cu:93-128); the reference does not ship a
 * mean kernel (its production path disables smoothing, turing_sage/core.py:421). */
int32_t tu_sage_kmean(const void *k_bf16, int64_t batch, int64_t heads, int64_t len,
                      int64_t dim, int64_t s_b, int64_t s_h, int64_t s_l, float *chunk_sums,
                      void *mean_bf16, void *stream);

/* tu_sage_kmean without caller scratch and without any allocation: the
 * chunk sums live in a file-scope device array of 2^22 floats (16 MiB) that
 * each GPU running the library holds until the process ends; its device
 * address is looked up once per device on the first call there.  Same
 * arguments and result as tu_sage_kmean minus `chunk_sums`; rejects
 * batch*heads*ceil(len/128)*dim > 2^22 (e.g. Wan-14B's B1 H40 L32760 D128
 * needs 1310720).  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other host threads) race; calls in one
 * stream are ordered.  No counterpart in the reference: it is for callers
 * that cannot allocate (HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). */
int32_t tu_sage_kmean_noalloc(const void *k_bf16, int64_t batch, int64_t heads, int64_t len,
                              int64_t dim, int64_t s_b, int64_t s_h, int64_t s_l, void *mean_bf16,
                              void *stream);

/* Per-block symmetric INT8 quantization of Q or K, optionally after
 * subtracting a per-(batch, head) channel mean (K smoothing):
 *   amax = max(1e-7, max |x - mean| over blk tokens x dim channels)
 *   scale[b][h][t / blk] = amax / 127;  q = sat_rne_s8((x - mean) * (127 / amax))
 * x: bf16 strides (s_b, s_h, s_l); q: int8 strides (q_b, q_h, q_l);
 * scale: fp32 [batch, heads, ceil(len / blk)]; mean: bf16 [batch, heads, dim]
 * or NULL.  blk in {16, 32, 64, 128}; dim in {64, 128}.
 * Replaces quant_per_block_int8_cuda / quant_per_warp_int8_cuda
 * (kernel/csrc/turing/sage/fused.cu:899-1068, QuantInt8Kernel :66-200). */
int32_t tu_sage_quant(const void *x_bf16, const void *mean_bf16, int64_t batch, int64_t heads,
                      int64_t len, int64_t dim, int64_t s_b, int64_t s_h, int64_t s_l,
                      int64_t blk, int8_t *q, int64_t q_b, int64_t q_h, int64_t q_l,
                      float *scale, void *stream);

/* Sage attention: V layout prologue ----------------------------------------- */

/* Writes V^T: vt[b][h][d][lpad] = v[b][h][key][d] for key < len and 0 for
 * len <= key < lpad (lpad % 64 == 0, lpad >= len).  v: bf16 with element
 * strides (s_b, s_h, s_l), channels contiguous; dim 64 or 128.  This is the PV
 * operand layout of tu_sage_attn_fwd (keys contiguous per channel).  It plays
 * the role of the reference's V staging in shared memory
 * (kernel/csrc/turing/sage/attn_utils.cuh:125-136, load_v_global_to_share). */
int32_t tu_sage_v_prep(const void *v_bf16, int64_t batch, int64_t heads, int64_t len, int64_t dim,
                       int64_t s_b, int64_t s_h, int64_t s_l, void *vt_bf16, int64_t lpad, void *stream);

/* Sage attention: forward --------------------------------------------------- */

/* O = softmax(Q K^T * sm_scale) V on INT8 Q/K and bf16 V:
 *   s = float(q8 . k8) * q_scale[row / blkq] * k_scale[key / blkk] * sm_scale
 *   online softmax in base 2, P rounded to bf16, O accumulated in fp32 by
 *   bf16 MFMA, O / rowsum(P) stored as bf16.
 * q8: int8 [batch, hq, lq, dim] addressed by strides (q_sb, q_sh, q_sl);
 * k8: int8 likewise with hkv heads (hq % hkv == 0, GQA); vt: bf16
 * [batch, hkv, dim, lpad] from tu_sage_v_prep; o: bf16 by strides.
 * q_scale: fp32 [batch, hq, ceil(lq/blkq)]; k_scale: fp32 [batch, hkv, ceil(lk/blkk)].
 * dim 64 or 128 (the reference's two kernel widths, turing_sage/core.py
 * :436-448; narrower heads are zero-padded by the caller); blkq >= 1;
 * blkk % 64 == 0.  causal: top-left aligned.
 * Replaces qk_int8_sv_f16_accum_f32_attn
 * (kernel/csrc/turing/sage/qk_int_sv_f16_cuda_sm75.cu:984-1123), the kernel
 * behind turing_utils::sage_attention (turing_sage/custom_ops.py:137-168). */
int32_t tu_sage_attn_fwd(const int8_t *q8, const float *q_scale, int64_t blkq, const int8_t *k8,
                         const float *k_scale, int64_t blkk, const void *vt_bf16, int64_t lpad,
                         void *o_bf16, int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk,
                         int64_t dim, int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb,
                         int64_t k_sh, int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                         float sm_scale, int32_t causal, void *stream);

/* The same attention with the keys split into kv_splits ranges, for grids
 * that fill the GPU badly (few heads x query blocks): each workgroup covers
 * one query block and one key range and writes its unnormalized O, exponent
 * base and row sum to `partial`; a second kernel merges the ranges,
 * O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s, and stores bf16.
 * Non-causal only; 1 <= kv_splits <= min(ceil(lk / 64), 256) (kv_splits = 1
 * is tu_sage_attn_fwd).  partial: fp32 workspace of at least
 * splits * batch * hq * lq * (dim + 2) * 4 bytes, 16-byte aligned, where
 * splits = ceil(T / ceil(T / kv_splits)) for T = ceil(lk / 64).  Results
 * agree with tu_sage_attn_fwd to fp32 rounding of the merge and to the bf16
 * rounding of P against each range's own exponent base.  The reference has
 * no split form; its single kernel is qk_int_sv_f16_cuda_sm75.cu:984-1123. */
int32_t tu_sage_attn_fwd_split(const int8_t *q8, const float *q_scale, int64_t blkq, const int8_t *k8,
                               const float *k_scale, int64_t blkk, const void *vt_bf16, int64_t lpad,
                               void *o_bf16, int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk,
                               int64_t dim, int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb,
                               int64_t k_sh, int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                               float sm_scale, int32_t kv_splits, void *partial, int64_t partial_bytes,
                               void *stream);

/* Number of key ranges tu_sage_attn_fwd_split should use on a GPU with `cus`
 * compute units (1: do not split): workgroups run in rounds of `cus`, and
 * each costs its key tiles plus a fixed part.  Host-only arithmetic, no HIP
 * call; no counterpart in the reference. */
int32_t tu_sage_attn_kv_splits(int64_t batch, int64_t hq, int64_t lq, int64_t lk, int32_t causal, int32_t cus);

/* Sage attention: fused Q/K preprocessing -------------------------------- */

/* RMSNorm + RoPE + per-tile INT8 of Q and K in one pass, the producer of the
 * attention's Q/K (Q per 16-token tile, K per 64-token tile):
 *   rrms  = 1 / sqrt(sumsq / n + eps)    norm_scope 0: the token's head row
 *           (n = dim); 1: all heads of the token (n = heads * dim); q_rrms /
 *           k_rrms are fp32 [batch, len] scratch for it (their contents
 *           afterwards are not part of the result)
 *   a_c   = T((x_c * rrms) * w_c)        T = bf16 (dtype 0) or fp16 (dtype 1);
 *           w = norm[c] (scope 0) or norm[head * dim + c] (scope 1)
 *   c < rot_dim: y_c = T(fma(f[pair][comp][1], a_second, f[pair][comp][0] * a_first))
 *           with pairs (2p, 2p + 1) or, split_half, (p, p + rot_dim / 2), and
 *           comp the channel's position in its pair; else y_c = a_c
 *   tile: amax = max(1e-7, max |y|); scale = amax / 127;
 *           q = clamp(rint(y * 127 / amax), -127, 127)
 * q, k: T with element strides (s_b, s_h, s_l), channels contiguous,
 * 16-byte aligned rows; dim in {64, 128}.  freqs: T [f_batches, f_len, 1,
 * rot_dim / 2, 2, 2] by element strides (f_sb, f_sl, pair f_sp, row f_sr,
 * column f_sc); f_batches in {1, batch}, f_len in {1, lq == lk}.  q8, k8:
 * int8 by strides.  q_scale: fp32 [batch, hq, ceil(lq / 64) * 4] (tiles past
 * lq get 1e-7 / 127); k_scale: fp32 [batch, hk, ceil(lk / 64)].
 * rotate != 0 (the W8A8 variant): after RoPE each token row is rotated by
 * the shared sign-diagonal Walsh-Hadamard transform of tu_w8a8_quant_qk
 * before the tile amax; with anchors / anchor_values (int32 [batch, hk] /
 * fp32 [batch, hk, dim], both or neither, rotate required) K is first
 * centred on its stabilisation anchor, detected on the processed values of
 * nine sampled rows (head scope: their rrms from a sequential fma chain).
 * Replaces turing_utils::qk_rms_rope_int8 (kernel/comfyui_turing_utils_kernel/
 * turing_sage/custom_ops.py:63-134 -> quant.py:6-87 -> kernel/csrc/turing/
 * sage/qk_preprocess.cu:250-416 (anchor), :417-629, :632-753). */
int32_t tu_qk_rms_rope_int8(const void *q, const void *k, int32_t dtype, int64_t batch, int64_t hq,
                            int64_t hk, int64_t lq, int64_t lk, int64_t dim, int64_t q_sb, int64_t q_sh,
                            int64_t q_sl, int64_t k_sb, int64_t k_sh, int64_t k_sl, const void *q_norm,
                            const void *k_norm, int32_t norm_scope, float eps, const void *freqs,
                            int64_t rot_dim, int32_t split_half, int64_t f_batches, int64_t f_len,
                            int64_t f_sb, int64_t f_sl, int64_t f_sp, int64_t f_sr, int64_t f_sc,
                            float *q_rrms, float *k_rrms, int8_t *q8, int64_t qo_sb, int64_t qo_sh,
                            int64_t qo_sl, int8_t *k8, int64_t ko_sb, int64_t ko_sh, int64_t ko_sl,
                            float *q_scale, float *k_scale, int32_t rotate, int32_t *anchors,
                            float *anchor_values, void *stream);

/* Dense W8A8 attention (the loader-default `w8a8` backend) ----------------- */

/* Hadamard-rotated per-tile INT8 of Q and K with the optional K anchor:
 *   anchors != NULL: anchor[b][h] = the K stabilisation row (-1 = none),
 *     computed first; v = x - x[anchor] for K
 *   rotate: v = H v, H = the sign-diagonal normalised Walsh-Hadamard
 *     transform shared by Q and K (Q.K is unchanged)
 *   tile (Q: 16 tokens, K: 64 tokens): amax = max(1e-7, max |v|);
 *     scale = amax / 127; q = cvt.rni.sat.s8(v * (127 / amax))
 * q, k: bf16 (dtype 0) or fp16 (dtype 1) by element strides, channels
 * contiguous, 16-byte aligned rows; dim in {64, 128}.  q8, k8: int8 by
 * strides (8-byte aligned rows).  q_scale: fp32 [batch, hq, ceil(lq/64)*4];
 * k_scale: fp32 [batch, hk, ceil(lk/64)]; anchors: int32 [batch, hk] or NULL.
 * Replaces per_warp_int8_hadamard (turing_sage/quant.py:182-242 ->
 * kernel/csrc/turing/sage/fused.cu:1252-1290: DetectKAnchorKernel :409-575,
 * QuantQKInt8Kernel with ROTATE :577-636, attention_hadamard8 :202-260). */
int32_t tu_w8a8_quant_qk(const void *q, const void *k, int32_t dtype, int64_t batch, int64_t hq,
                         int64_t hk, int64_t lq, int64_t lk, int64_t dim, int64_t q_sb, int64_t q_sh,
                         int64_t q_sl, int64_t k_sb, int64_t k_sh, int64_t k_sl, int8_t *q8,
                         int64_t q8_sb, int64_t q8_sh, int64_t q8_sl, int8_t *k8, int64_t k8_sb,
                         int64_t k8_sh, int64_t k8_sl, float *q_scale, float *k_scale,
                         int32_t *anchors, int32_t rotate, void *stream);

/* Bytes of device scratch tu_w8a8_quant_v needs (-1 on bad sizes). */
int64_t tu_w8a8_quant_v_workspace(int64_t batch, int64_t heads, int64_t len, int64_t dim);

/* Channel-wise signed INT8 V:
 *   scale[c] = max(amax_c / 127, 1e-12) over all len tokens;
 *   vq[c][t] = cvt.rni.sat.s8(v[t][c] * (1 / scale[c])), 0 for t >= len.
 * v: bf16/fp16 by element strides, 16-byte aligned rows; dim in {64, 128}.
 * vq: int8 [batch, heads, dim, lpad] with lpad = ceil(len/64)*64 (keys in
 * natural order); scale: fp32 [batch, heads, dim]; workspace:
 * tu_w8a8_quant_v_workspace bytes.  Replaces quantize_v_int8_sm75 (turing_sage/core.py:772-784 ->
 * kernel/csrc/turing/sage/quant_v_int8_cuda_sm75.cu:58-164, :177-246); the
 * reference's 16-token key permutation (its Turing MMA fragment order) is
 * not used, the codes are the same. */
int32_t tu_w8a8_quant_v(const void *v, int32_t dtype, int64_t batch, int64_t heads, int64_t len,
                        int64_t dim, int64_t s_b, int64_t s_h, int64_t s_l, int8_t *vq, int64_t lpad,
                        float *scale, void *workspace, int64_t workspace_bytes, void *stream);

/* Dense W8A8 attention forward on INT8 Q/K/V:
 *   s = float(q8 . k8); masked keys (>= lk; causal: key > query, top-left)
 *       get the raw score -5e6
 *   f = (sm_scale * log2 e) * q_scale[row / 16] * k_scale[key / 64]
 *   online over 64-key tiles: m = max(m, fma(max s, f, -log2 255)),
 *       p = 2^(fma(s, f, -m)), P = cvt.rni.sat.u8(p), l += p,
 *       O += P . vq (exact), O and l rescaled by 2^(m_old - m)
 *   out = O / l * v_scale[channel], bf16 (out_fp16 0) or fp16 (1)
 * q8, k8: int8 by element strides (16-byte aligned rows), dim == 128, GQA
 * hq % hkv == 0; q_scale: fp32 [batch, hq, nqs >= ceil(lq/16)]; k_scale:
 * fp32 [batch, hkv, nks >= ceil(lk/64)]; vq, v_scale from tu_w8a8_quant_v
 * (lpad = ceil(lk/64)*64); out by strides.
 * Replaces sol_sparse_online_w8a8_prequantized_attn with force_dense
 * (turing_sage/core.py:916-982 -> kernel/csrc/turing/sage/
 * sol_sparse_cuda_sm75.cu:2767-2932 -> sparse_attention_kernel
 * <D, T, UseW8A8, ForceDense> :709-1394), the kernel behind
 * turing_utils::w8a8_attention (turing_sage/custom_ops.py:171-210). */
int32_t tu_w8a8_attn_fwd(const int8_t *q8, const float *q_scale, int64_t nqs, const int8_t *k8,
                         const float *k_scale, int64_t nks, const int8_t *vt, const float *v_scale,
                         int64_t lpad, void *out, int32_t out_fp16,
                         int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk, int64_t dim,
                         int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb, int64_t k_sh,
                         int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl, float sm_scale,
                         int32_t causal, void *stream);

/* Wan block: LayerNorm + AdaLN --------------------------------------------- */

/* out = T(fma(T((x - mean) / sqrt(var + eps)), T(1 + scale), shift)) per row
 * of `hidden` channels, mean / var from fp32 Welford statistics in the
 * reference's order (256 threads striding the row, 32-lane trees, eight tree
 * results combined in order).  x, out: [batch, len, hidden] contiguous;
 * scale, shift: [batch, steps, hidden] contiguous, token t of a row uses
 * modulation row min(t / g, steps - 1) with g = len / steps, + 1 when steps
 * does not divide len (steps == 1: row 0).  dtype 0 bf16, 1 fp16, 2 fp32 (T
 * = the element type).  eps finite and positive.  Rows up to hidden 8192
 * stay in registers (x read once); wider rows read x twice.
 * Replaces turing_utils::layer_norm_adaln (kernel/comfyui_turing_utils_kernel/
 * ops.py:399-418 -> kernel/csrc/turing/segmented_rms_adaln.cu:236-307,
 * :372-409). */
int32_t tu_layer_norm_adaln(const void *x, const void *scale, const void *shift, void *out, int32_t dtype,
                            int64_t batch, int64_t len, int64_t hidden, int64_t steps, float eps,
                            void *stream);

/* LayerNorm with an elementwise affine weight and bias shared by all rows:
 *   out[r][c] = T(fma((x[r][c] - mean_r) / sqrt(var_r + eps), weight[c], bias[c]))
 * with the statistics of tu_layer_norm_adaln (same order) and one rounding to
 * the element type T.  x/out: [rows, hidden] contiguous; weight/bias:
 * [hidden]; dtype 0 bf16, 1 fp16, 2 fp32.  No counterpart in the reference's
 * kernel package: ComfyUI's torch LayerNorm(elementwise_affine=True) runs the
 * Wan block's norm3, which the reference's Wan adapter leaves in place
 * (comfyui_turing_utils/adapters/wan.py:55-137 patches only the attention). */
int32_t tu_layer_norm_affine(const void *x, const void *weight, const void *bias, void *out,
                             int32_t dtype, int64_t rows, int64_t hidden, float eps, void *stream);

/* LayerNorm fused with the ConvRot INT8 quantizer (G = 128, bf16 only): the
 * codes q [rows, hidden] and row scales row_scale [rows] that
 * tu_convrot_quant_i8(out, q, row_scale, rows, hidden, 128, 0) writes for the
 * bf16 out of tu_layer_norm_adaln (dtype 0, same arguments) resp.
 * tu_layer_norm_affine, bit for bit; the normalized rows are not written.
 * hidden a multiple of 256 in [256, 5120]; x, scale / weight, shift / bias
 * and q 16-byte aligned.  No counterpart in the reference, which runs the
 * norm (ops.py:399-418) and the linear's activation quantizer
 * (quantization/dispatch.py:538-615) as two ops; for the Wan block's norm1 /
 * norm2 -> qkv / FFN-up and norm3 -> cross-attention q projections. */
int32_t tu_layer_norm_adaln_convrot_quant_i8(const void *x, const void *scale, const void *shift, int8_t *q,
                                             float *row_scale, int64_t batch, int64_t len, int64_t hidden,
                                             int64_t steps, float eps, void *stream);
int32_t tu_layer_norm_affine_convrot_quant_i8(const void *x, const void *weight, const void *bias, int8_t *q,
                                              float *row_scale, int64_t rows, int64_t hidden, float eps,
                                              void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TU_HIP_H_ */
