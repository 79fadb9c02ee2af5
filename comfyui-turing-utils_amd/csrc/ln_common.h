// LayerNorm helpers shared by the LayerNorm kernels (adaln.hip) and the
// LayerNorm-fused ConvRot quantizer (convrot_quant.hip): element types, the
// Welford combine with known counts, and the half-wave statistics and output
// of the 16-bit row kernels.
//
// Reference semantics: layer_norm_adaln_kernel
// (kernel/csrc/turing/segmented_rms_adaln.cu:236-307): fp32 Welford
// statistics in a fixed order -- 256 threads, thread t takes columns t,
// t + 256, ... (count++, delta = v - mean, mean += delta / count,
// m2 += delta * (v - mean), the last contracted to an fma as nvcc does), then
// 32-lane shfl_down trees of welford_combine and the eight tree results
// combined in order.  1 / sqrt is IEEE (the reference uses rsqrtf).
#pragma once

#include "tu_common.h"

namespace tu {
namespace {

constexpr int kLnThreads = 256;  // the reference's threads per row

// Element types: 0 bf16, 1 fp16 (2-byte patterns), 2 fp32.
template <int kT> struct Elem { typedef uint16_t type; };
template <> struct Elem<2> { typedef float type; };

template <int kT>
__device__ __forceinline__ float to_f32(typename Elem<kT>::type v) {
    if constexpr (kT == 2) return v;
    else if constexpr (kT == 1) return static_cast<float>(__builtin_bit_cast(_Float16, v));
    else return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round to the element type (RNE) and back; the asm keeps the fp32 value
// from being fused into a single-rounding mixed-precision FMA.
template <int kT>
__device__ __forceinline__ float t_round(float v) {
    if constexpr (kT == 2) return v;
    asm("" : "+v"(v));
    if constexpr (kT == 1) return static_cast<float>(static_cast<_Float16>(v));
    else return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(v))) << 16);
}

// The fp32 result is pinned before the fp16 conversion: otherwise the
// compiler folds "fp32 fma, then round to fp16" into one single-rounding
// v_fma_mix instruction, which differs on fp32 values near fp16 ties.
template <int kT>
__device__ __forceinline__ typename Elem<kT>::type from_f32(float v) {
    if constexpr (kT == 2) return v;
    else if constexpr (kT == 1) {
        asm("" : "+v"(v));
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    }
    else return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}

// Correctly rounded a / b from y = RN(1 / b), b a positive integer <= 2^13:
// Markstein's correction -- q = RN(a y) is within an ulp of a / b, the
// remainder a - b q is exact under fma, and RN(q + (a - b q) y) = RN(a / b).
// Verified on every fp32 mantissa in [1, 2) for each denominator the LayerNorm
// kernels pass; exact power-of-two scaling carries that to |a| in
// [2^-96, 2^100] (no subnormal step), and anything else -- zero, tiny, huge,
// inf, NaN -- takes the IEEE division.
// The range test is one wave-wide vote, so the common case costs no
// exec-mask juggling; lanes out of range then take the division.
__device__ __forceinline__ float div_rn(float a, float b, float y) {
    const uint32_t e = (__float_as_uint(a) >> 23) & 0xffu;
    const bool out = e - 31u >= 197u;
    const float q = a * y;
    float r = __builtin_fmaf(__builtin_fmaf(-q, b, a), y, q);
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(out) != 0, 0)) r = out ? a / b : r;
    return r;
}

// welford_combine with both counts known and y = RN(1 / (lc + rc)).
__device__ __forceinline__ void combine_known(float &mean, float &m2, float r_mean, float r_m2, float lc, float rc,
                                              float y) {
    const float count = lc + rc;
    const float delta = r_mean - mean;
    mean = mean + div_rn(delta * rc, count, y);
    m2 = m2 + (r_m2 + div_rn(((delta * delta) * lc) * rc, count, y));
}

// RN(1 / n) of the combine counts of a row whose 256 threads each hold P
// values (hidden = 256 P): the 32-lane tree levels (2P .. 32P) and the
// in-order combine of the eight tree results (64P .. 256P).
struct Recips {
    float level[5];
    float total[8];
};

// Host: the Recips of rows of 256 per columns (host IEEE division: RN(1 / n)).
inline Recips uniform_recips(int per) {
    Recips rc{};
    for (int lvl = 0; lvl < 5; ++lvl) rc.level[lvl] = 1.0f / static_cast<float>(per << (lvl + 1));
    for (int i = 1; i < kLnThreads / 32; ++i) rc.total[i] = 1.0f / static_cast<float>((i + 1) * 32 * per);
    return rc;
}

// ---------------------------------------------------------------------------
// 16-bit rows with hidden = 256 per: the statistics above in the same order,
// computed by a 32-lane half-wave.  Virtual thread t of the reference's 256
// (columns t, t + 256, ...) is chain e = t & 7 of lane p = t >> 3 of the
// half-wave, so column block i of a lane's 8 chains is the 16 contiguous
// bytes at 256 i + 8 p: every load and store is 16 bytes wide.  The
// 32-thread tree levels of offset 16 and 8 are lane swaps (p ^ 2, p ^ 1,
// DPP within a quad of lanes); offsets 4, 2, 1 combine chains of one lane.
// ---------------------------------------------------------------------------
template <int kT>
__device__ __forceinline__ float lo16(uint32_t w) {
    if constexpr (kT == 1) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
    else return __uint_as_float(w << 16);
}
template <int kT>
__device__ __forceinline__ float hi16(uint32_t w) {
    if constexpr (kT == 1) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
    else return __uint_as_float(w & 0xffff0000u);
}
template <int kT>
__device__ __forceinline__ float unpack16(const u32x4 &v, int e) {
    return (e & 1) ? hi16<kT>(v[e >> 1]) : lo16<kT>(v[e >> 1]);
}

// Value from lane (lane & ~3) | (lane & 3 ^ kXor) of the same quad (DPP).
template <int kXor>
__device__ __forceinline__ float quad_xor(float v) {
    constexpr int kSel = kXor == 2 ? 0x4e : 0xb1;  // quad_perm [2,3,0,1] / [1,0,3,2]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kSel, 0xf, 0xf, false));
}

// Modulation row of token row `row`: b * steps + mt.
__device__ __forceinline__ int64_t modulation_row(int64_t row, int64_t len, int64_t steps) {
    const int64_t b = row / len, t = row - b * len;
    int64_t mt = 0;
    if (steps > 1) {
        const int64_t repeats = len / steps;
        const int64_t group = repeats * steps == len ? repeats : repeats + 1;
        mt = min(t / max<int64_t>(group, 1), steps - 1);
    }
    return b * steps + mt;
}

// True when the Markstein quotient of div_rn does not cover a: the biased
// exponent of a is outside [31, 227], i.e. |a| < 2^-96 (zero and subnormals
// included), |a| >= 2^101, inf or NaN.
__device__ __forceinline__ bool div_out(float a) {
    const float m = fabsf(a);
    return !(m >= 0x1p-96f) || !(m < 0x1p101f);
}

// Row statistics of one half-wave's row from its lane's column blocks xs[i]
// (i < per; hidden = 256 per): the mean mu and inv = 1 / sqrt(var + eps),
// the same in every lane of the half-wave.  `half_base` is the byte address
// of lane 0 of this half-wave for ds_bpermute (0 or 128).
template <int kT, int kPer>
__device__ __forceinline__ void ln16_row_stats(const u32x4 (&xs)[kPer], int per, int hidden, float eps,
                                               const Recips &rc, int half_base, float &mu, float &inv) {
    // Welford over each chain's columns in order; the count at step i is
    // i + 1 for every chain.  One wave-wide vote per step for the 8 ranges.
    float mean[8], m2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) mean[e] = m2[e] = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        if (i < per) {
            const float n = static_cast<float>(i + 1), y = 1.0f / static_cast<float>(i + 1);
            float v[8], delta[8], r[8];
            bool out_any = false;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[e] = unpack16<kT>(xs[i], e);
                delta[e] = v[e] - mean[e];
                out_any = out_any || div_out(delta[e]);
                const float q = delta[e] * y;
                r[e] = __builtin_fmaf(__builtin_fmaf(-q, n, delta[e]), y, q);
            }
            if (__builtin_expect(__builtin_amdgcn_ballot_w64(out_any) != 0, 0)) {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (div_out(delta[e])) r[e] = delta[e] / n;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                mean[e] = mean[e] + r[e];
                m2[e] = __builtin_fmaf(delta[e], v[e] - mean[e], m2[e]);
            }
        }
    }

    // 32-thread trees: offset 16 = lane p ^ 2, offset 8 = lane p ^ 1, then
    // offsets 4, 2, 1 between the chains of lane p = 0 (mod 4).
    float cnt = static_cast<float>(per);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float r_mean = quad_xor<2>(mean[e]), r_m2 = quad_xor<2>(m2[e]);
        combine_known(mean[e], m2[e], r_mean, r_m2, cnt, cnt, rc.level[0]);
    }
    cnt += cnt;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float r_mean = quad_xor<1>(mean[e]), r_m2 = quad_xor<1>(m2[e]);
        combine_known(mean[e], m2[e], r_mean, r_m2, cnt, cnt, rc.level[1]);
    }
    cnt += cnt;
#pragma unroll
    for (int lvl = 2, half = 4; lvl < 5; ++lvl, half >>= 1) {
#pragma unroll
        for (int e = 0; e < half; ++e) combine_known(mean[e], m2[e], mean[e + half], m2[e + half], cnt, cnt, rc.level[lvl]);
        cnt += cnt;
    }
    // the eight tree results (lanes 0, 4, .., 28 of the half-wave, chain 0),
    // combined in order by every lane
    float tm = __int_as_float(__builtin_amdgcn_ds_bpermute(half_base, __float_as_int(mean[0])));
    float tv = __int_as_float(__builtin_amdgcn_ds_bpermute(half_base, __float_as_int(m2[0])));
#pragma unroll
    for (int j = 1; j < kLnThreads / 32; ++j) {
        const float om = __int_as_float(__builtin_amdgcn_ds_bpermute(half_base + 16 * j, __float_as_int(mean[0])));
        const float ov = __int_as_float(__builtin_amdgcn_ds_bpermute(half_base + 16 * j, __float_as_int(m2[0])));
        combine_known(tm, tv, om, ov, static_cast<float>(j) * cnt, cnt, rc.total[j]);
    }
    const float var = div_rn(tv, static_cast<float>(hidden), rc.total[kLnThreads / 32 - 1]);
    mu = tm;
    inv = 1.0f / __builtin_sqrtf(var + eps);
}

// The output's per-column factors, the same for every row of one modulation
// row: m = T(1 + scale) (AdaLN) or weight (affine), and shift / bias, as fp32.
// Staged in LDS once per workgroup: [0, hidden) m, [hidden, 2 hidden) shift.
template <int kT, bool kAffine>
__device__ __forceinline__ void stage_modulation(float *mod, const uint16_t *__restrict__ sc,
                                                 const uint16_t *__restrict__ sh, int hidden) {
    for (int c = 8 * static_cast<int>(threadIdx.x); c < hidden; c += 8 * kLnThreads) {
        const u32x4 sv = *reinterpret_cast<const u32x4 *>(sc + c);
        const u32x4 hv = *reinterpret_cast<const u32x4 *>(sh + c);
        f32x4 m0, m1, h0, h1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float s = unpack16<kT>(sv, e);
            const float m = kAffine ? s : t_round<kT>(1.0f + s);
            const float h = unpack16<kT>(hv, e);
            if (e < 4) { m0[e] = m; h0[e] = h; } else { m1[e - 4] = m; h1[e - 4] = h; }
        }
        *reinterpret_cast<f32x4 *>(mod + c) = m0;
        *reinterpret_cast<f32x4 *>(mod + c + 4) = m1;
        *reinterpret_cast<f32x4 *>(mod + hidden + c) = h0;
        *reinterpret_cast<f32x4 *>(mod + hidden + c + 4) = h1;
    }
}

// The outputs of one column block (8 values of xv) from their per-column
// factors mv (T(1 + scale), or the affine weight) and hv (shift / bias):
//   AdaLN:  T(fma(T((x - mu) inv), mv, hv))
//   affine: T(fma((x - mu) inv, mv, hv))
template <int kT, bool kAffine>
__device__ __forceinline__ u32x4 ln16_emit8(const u32x4 &xv, const float (&mv)[8], const float (&hv)[8], float mu,
                                            float inv) {
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint16_t half[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int e = 2 * j + k;
            const float value = unpack16<kT>(xv, e);
            if constexpr (kAffine) {
                half[k] = from_f32<kT>(__builtin_fmaf((value - mu) * inv, mv[e], hv[e]));
            } else {
                const float nv = t_round<kT>((value - mu) * inv);
                half[k] = from_f32<kT>(__builtin_fmaf(nv, mv[e], hv[e]));
            }
        }
        o[j] = static_cast<uint32_t>(half[0]) | (static_cast<uint32_t>(half[1]) << 16);
    }
    return o;
}

}  // namespace
}  // namespace tu
