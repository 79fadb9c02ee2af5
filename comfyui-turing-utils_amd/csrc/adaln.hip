// LayerNorm + AdaLN modulation for gfx950, the Wan block's norm1 / norm2
// (bf16, fp16 or fp32 rows):
//   out = T(fma(T((x - mean) / sqrt(var + eps)), T(1 + scale), shift))
// per token row of hidden channels, with the token's modulation row of
// scale / shift.
//
// Reference semantics: layer_norm_adaln_kernel
// (kernel/csrc/turing/segmented_rms_adaln.cu:236-307): fp32 Welford
// statistics in a fixed order -- 256 threads, thread t takes columns t,
// t + 256, ... (count++, delta = v - mean, mean += delta / count,
// m2 += delta * (v - mean), the last contracted to an fma as nvcc does), then
// 32-lane shfl_down trees of welford_combine and the eight tree results
// combined in order.  Kept exactly so that the CPU oracle restates it bit for
// bit; 1 / sqrt is IEEE (the reference uses rsqrtf).
//
// The affine variant (kAffine) is LayerNorm with an elementwise weight w and
// bias b shared by every row, as ComfyUI's LayerNorm(elementwise_affine=True)
// runs the Wan block's norm3 (torch layer_norm computes in fp32 and rounds
// once): out = T(fma((x - mean) / sqrt(var + eps), w, b)), same statistics.
//
// MI355X mapping: one workgroup of 256 threads (4 wave64) per row; a wave64
// holds two 32-lane trees (xor partners below 32 stay in the half).  Up to
// hidden 8192 a thread keeps its columns in registers between the statistics
// and output passes, so x is read once: 2 B in + 2 B out per element; wider
// rows (kPer == 0) read x again in the output pass, same column order.
#include "tu_common.h"

namespace tu {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxPerThread = 32;  // register-resident rows: hidden <= 8192

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
// Verified on every fp32 mantissa in [1, 2) for each denominator this file
// passes; exact power-of-two scaling carries that to |a| in [2^-96, 2^100]
// (no subnormal step), and anything else -- zero, tiny, huge, inf, NaN --
// takes the IEEE division.
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

struct Welford {
    float mean, m2;
    int count;
};

__device__ __forceinline__ Welford combine(Welford l, Welford r) {
    if (r.count == 0) return l;
    if (l.count == 0) return r;
    const int count = l.count + r.count;
    const float delta = r.mean - l.mean;
    l.mean = l.mean + (delta * static_cast<float>(r.count)) / static_cast<float>(count);
    l.m2 = l.m2 + (r.m2 + (((delta * delta) * static_cast<float>(l.count)) * static_cast<float>(r.count)) /
                              static_cast<float>(count));
    l.count = count;
    return l;
}

// The same combine with both counts known and y = RN(1 / (lc + rc)).
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

// One workgroup per token row.  kPer > 0: the thread's columns t + 256 i
// (i < kPer) and their modulation values stay in registers; kUniform: every
// thread holds exactly hidden / 256 of them and all counts are known (and
// kExact: that number is kPer itself, so no column needs a bounds test).
template <int kT, int kPer, bool kUniform, bool kAffine, bool kExact = false>
__global__ __launch_bounds__(kThreads) void layer_norm_adaln_kernel(const typename Elem<kT>::type *__restrict__ x,
                                                                   const typename Elem<kT>::type *__restrict__ scale,
                                                                   const typename Elem<kT>::type *__restrict__ shift,
                                                                   typename Elem<kT>::type *__restrict__ out,
                                                                   int64_t len, int hidden, int64_t steps, float eps,
                                                                   Recips rc) {
    typedef typename Elem<kT>::type E;
    __shared__ Welford trees[kThreads / 32];
    __shared__ float row_stats[2];
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const int64_t b = row / len, t = row - b * len;
    int64_t mt = 0;
    if (steps > 1) {
        const int64_t repeats = len / steps;
        const int64_t group = repeats * steps == len ? repeats : repeats + 1;
        mt = min(t / max<int64_t>(group, 1), steps - 1);
    }
    const E *xr = x + row * hidden;
    const E *sc = scale + (b * steps + mt) * hidden;
    const E *sh = shift + (b * steps + mt) * hidden;
    E *orow = out + row * hidden;
    const int per = kExact ? kPer : hidden / kThreads;  // kUniform: values per thread

    constexpr int kKeep = kPer > 0 ? kPer : 1;
    float v[kKeep], mod[kKeep], add[kKeep];
    Welford w{0.0f, 0.0f, 0};
    if constexpr (kPer > 0) {
        // all loads first, unconditional from an in-bounds column (column 0
        // past the row end), so the modulation row's latency hides behind the
        // statistics
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = tid + i * kThreads;
            const bool in = kUniform ? i < per : c < hidden;
            const int cs = in ? c : 0;
            const float xv = to_f32<kT>(xr[cs]), sv = to_f32<kT>(sc[cs]), hv = to_f32<kT>(sh[cs]);
            v[i] = in ? xv : 0.0f;
            mod[i] = sv;
            add[i] = hv;
        }
        // the count at step i is i + 1 (columns are taken in order and stop
        // at the row end), so 1 / count is a constant
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = tid + i * kThreads;
            if (kUniform ? i < per : c < hidden) {
                ++w.count;
                const float delta = v[i] - w.mean;
                w.mean = w.mean + div_rn(delta, static_cast<float>(i + 1), 1.0f / static_cast<float>(i + 1));
                w.m2 = __builtin_fmaf(delta, v[i] - w.mean, w.m2);
            }
        }
    } else {
        for (int c = tid; c < hidden; c += kThreads) {
            const float value = to_f32<kT>(xr[c]);
            ++w.count;
            const float delta = value - w.mean;
            w.mean = w.mean + delta / static_cast<float>(w.count);
            w.m2 = __builtin_fmaf(delta, value - w.mean, w.m2);
        }
    }

    float mean, var;
    if constexpr (kUniform) {
        float cnt = static_cast<float>(per);
#pragma unroll
        for (int lvl = 0, off = 16; off > 0; off >>= 1, ++lvl) {
            const float r_mean = __shfl_xor(w.mean, off), r_m2 = __shfl_xor(w.m2, off);
            combine_known(w.mean, w.m2, r_mean, r_m2, cnt, cnt, rc.level[lvl]);
            cnt += cnt;
        }
        if ((tid & 31) == 0) trees[tid >> 5] = w;
        __syncthreads();
        // the in-order combine of the eight tree results, by the first wave
        // only; the others take mean and variance from LDS
        if (tid < 64) {
            mean = trees[0].mean;
            float m2 = trees[0].m2;
#pragma unroll
            for (int i = 1; i < kThreads / 32; ++i)
                combine_known(mean, m2, trees[i].mean, trees[i].m2, static_cast<float>(i) * cnt, cnt, rc.total[i]);
            var = div_rn(m2, static_cast<float>(hidden), rc.total[kThreads / 32 - 1]);
            if (tid == 0) {
                row_stats[0] = mean;
                row_stats[1] = var;
            }
        }
        __syncthreads();
        mean = row_stats[0];
        var = row_stats[1];
    } else {
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) {
            const Welford other{__shfl_xor(w.mean, off), __shfl_xor(w.m2, off), __shfl_xor(w.count, off)};
            w = combine(w, other);
        }
        if ((tid & 31) == 0) trees[tid >> 5] = w;
        __syncthreads();
        Welford total{0.0f, 0.0f, 0};
#pragma unroll
        for (int i = 0; i < kThreads / 32; ++i) total = combine(total, trees[i]);
        mean = total.mean;
        var = total.m2 / static_cast<float>(total.count);
    }
    const float inv = 1.0f / __builtin_sqrtf(var + eps);

    auto emit = [&](int c, float value, float s, float h) {
        if constexpr (kAffine) {
            orow[c] = from_f32<kT>(__builtin_fmaf((value - mean) * inv, s, h));
        } else {
            const float n = t_round<kT>((value - mean) * inv);
            const float m = t_round<kT>(1.0f + s);
            orow[c] = from_f32<kT>(__builtin_fmaf(n, m, h));
        }
    };
    if constexpr (kPer > 0) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int c = tid + i * kThreads;
            if (kUniform ? i < per : c < hidden) emit(c, v[i], mod[i], add[i]);
        }
    } else {
        for (int c = tid; c < hidden; c += kThreads) emit(c, to_f32<kT>(xr[c]), to_f32<kT>(sc[c]), to_f32<kT>(sh[c]));
    }
}

// ---------------------------------------------------------------------------
// 16-bit rows with hidden = 256 per (per <= kPer): the same statistics in the
// same order, computed by half-waves.  Virtual thread t of the reference's
// 256 (columns t, t + 256, ...) is chain e = t & 7 of lane p = t >> 3 of a
// 32-lane half-wave, so column block i of a lane's 8 chains is the 16
// contiguous bytes at 256 i + 8 p: every load and store is 16 bytes wide.
// The 32-thread tree levels of offset 16 and 8 are lane swaps (p ^ 2, p ^ 1,
// DPP within a quad of lanes); offsets 4, 2, 1 combine chains of one lane.
// One row per half-wave, eight rows per workgroup.
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

// The output's per-column factors, the same for every row of one modulation
// row: m = T(1 + scale) (AdaLN) or weight (affine), and shift / bias, as fp32.
// Staged in LDS once per workgroup: [0, hidden) m, [hidden, 2 hidden) shift.
template <int kT, bool kAffine>
__device__ __forceinline__ void stage_modulation(float *mod, const uint16_t *__restrict__ sc,
                                                 const uint16_t *__restrict__ sh, int hidden) {
    for (int c = 8 * static_cast<int>(threadIdx.x); c < hidden; c += 8 * kThreads) {
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

template <int kT, int kPer, bool kAffine>
__global__ __launch_bounds__(kThreads) void layer_norm_rows16_kernel(const uint16_t *__restrict__ x,
                                                                    const uint16_t *__restrict__ scale,
                                                                    const uint16_t *__restrict__ shift,
                                                                    uint16_t *__restrict__ out, int64_t rows,
                                                                    int64_t len, int hidden, int per, int64_t steps,
                                                                    float eps, Recips rc) {
    extern __shared__ __align__(16) float mod[];
    const int tid = threadIdx.x;
    const int p = tid & 31;  // lane of the half-wave: virtual threads 8 p .. 8 p + 7
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * (kThreads / 32);
    const int64_t row_raw = row0 + (tid >> 5);
    // a half-wave past the last row computes the last row again and stores nothing
    const int64_t row = min(row_raw, rows - 1);
    const int64_t mrow = modulation_row(row, len, steps);
    // the workgroup's first row's modulation row goes to LDS; a half-wave
    // whose row has another one (batch or step boundary) reads its own
    const int64_t mrow0 = modulation_row(row0, len, steps);
    const bool staged = mrow == mrow0;
    const uint16_t *xr = x + row * hidden + 8 * p;
    const uint16_t *sc = scale + mrow * hidden + 8 * p;
    const uint16_t *sh = shift + mrow * hidden + 8 * p;

    u32x4 xs[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (i < per) xs[i] = *reinterpret_cast<const u32x4 *>(xr + 256 * i);

    stage_modulation<kT, kAffine>(mod, scale + mrow0 * hidden, shift + mrow0 * hidden, hidden);
    __syncthreads();

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
    const int base = (tid & 32) << 2;  // byte address of lane 0 of this half
    float tm = __int_as_float(__builtin_amdgcn_ds_bpermute(base, __float_as_int(mean[0])));
    float tv = __int_as_float(__builtin_amdgcn_ds_bpermute(base, __float_as_int(m2[0])));
#pragma unroll
    for (int j = 1; j < kThreads / 32; ++j) {
        const float om = __int_as_float(__builtin_amdgcn_ds_bpermute(base + 16 * j, __float_as_int(mean[0])));
        const float ov = __int_as_float(__builtin_amdgcn_ds_bpermute(base + 16 * j, __float_as_int(m2[0])));
        combine_known(tm, tv, om, ov, static_cast<float>(j) * cnt, cnt, rc.total[j]);
    }
    const float var = div_rn(tv, static_cast<float>(hidden), rc.total[kThreads / 32 - 1]);
    const float mu = tm;
    const float inv = 1.0f / __builtin_sqrtf(var + eps);
    if (row_raw >= rows) return;

    uint16_t *orow = out + row * hidden + 8 * p;
    const float *mod_m = mod + 8 * p, *mod_h = mod + hidden + 8 * p;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        if (i < per) {
            float mv[8], hv[8];
            if (staged) {
                const f32x4 m0 = *reinterpret_cast<const f32x4 *>(mod_m + 256 * i);
                const f32x4 m1 = *reinterpret_cast<const f32x4 *>(mod_m + 256 * i + 4);
                const f32x4 h0 = *reinterpret_cast<const f32x4 *>(mod_h + 256 * i);
                const f32x4 h1 = *reinterpret_cast<const f32x4 *>(mod_h + 256 * i + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    mv[e] = m0[e]; mv[e + 4] = m1[e];
                    hv[e] = h0[e]; hv[e + 4] = h1[e];
                }
            } else {
                const u32x4 sv = *reinterpret_cast<const u32x4 *>(sc + 256 * i);
                const u32x4 shv = *reinterpret_cast<const u32x4 *>(sh + 256 * i);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float s = unpack16<kT>(sv, e);
                    mv[e] = kAffine ? s : t_round<kT>(1.0f + s);
                    hv[e] = unpack16<kT>(shv, e);
                }
            }
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint16_t half[2];
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int e = 2 * j + k;
                    const float value = unpack16<kT>(xs[i], e);
                    if constexpr (kAffine) {
                        half[k] = from_f32<kT>(__builtin_fmaf((value - mu) * inv, mv[e], hv[e]));
                    } else {
                        const float nv = t_round<kT>((value - mu) * inv);
                        half[k] = from_f32<kT>(__builtin_fmaf(nv, mv[e], hv[e]));
                    }
                }
                o[j] = static_cast<uint32_t>(half[0]) | (static_cast<uint32_t>(half[1]) << 16);
            }
            *reinterpret_cast<u32x4 *>(orow + 256 * i) = o;
        }
    }
}

template <int kT, bool kAffine>
void launch(const void *xv, const void *scv, const void *shv, void *outv, int64_t rows, int64_t len, int hidden,
            int64_t steps, float eps, hipStream_t s) {
    typedef typename Elem<kT>::type E;
    const E *x = static_cast<const E *>(xv), *sc = static_cast<const E *>(scv), *sh = static_cast<const E *>(shv);
    E *out = static_cast<E *>(outv);
    const int per = (hidden + kThreads - 1) / kThreads;
    const dim3 grid(static_cast<unsigned>(rows));
    Recips rc{};
    const bool uniform = hidden % kThreads == 0 && per <= kMaxPerThread;
    if (uniform) {
        // host IEEE division: RN(1 / n)
        for (int lvl = 0; lvl < 5; ++lvl) rc.level[lvl] = 1.0f / static_cast<float>(per << (lvl + 1));
        for (int i = 1; i < kThreads / 32; ++i) rc.total[i] = 1.0f / static_cast<float>((i + 1) * 32 * per);
    }
    if constexpr (kT != 2) {
        const bool aligned = ((reinterpret_cast<uintptr_t>(xv) | reinterpret_cast<uintptr_t>(scv) |
                               reinterpret_cast<uintptr_t>(shv) | reinterpret_cast<uintptr_t>(outv)) & 15) == 0;
        if (uniform && aligned) {
            const dim3 g16(static_cast<unsigned>((rows + kThreads / 32 - 1) / (kThreads / 32)));
            const uint16_t *x16 = static_cast<const uint16_t *>(xv), *sc16 = static_cast<const uint16_t *>(scv),
                           *sh16 = static_cast<const uint16_t *>(shv);
            uint16_t *o16 = static_cast<uint16_t *>(outv);
#define TU_LN16(P) \
    layer_norm_rows16_kernel<kT, P, kAffine><<<g16, kThreads, 2 * hidden * sizeof(float), s>>>(x16, sc16, sh16, o16, rows, len, \
                                                                                           hidden, per, steps, eps, rc)
            if (per <= 4) TU_LN16(4);
            else if (per <= 8) TU_LN16(8);
            else if (per <= 16) TU_LN16(16);
            else if (per <= 20) TU_LN16(20);
            else TU_LN16(32);
#undef TU_LN16
            return;
        }
    }
#define TU_LN(P, U, X)                                                                       \
    layer_norm_adaln_kernel<kT, P, U, kAffine, X><<<grid, kThreads, 0, s>>>(x, sc, sh, out, len, hidden, \
                                                                            steps, eps, rc)
#define TU_LN2(P)                                  \
    if (uniform && per == P) TU_LN(P, true, true); \
    else if (uniform) TU_LN(P, true, false);       \
    else TU_LN(P, false, false)
    if (per <= 4) { TU_LN2(4); }
    else if (per <= 8) { TU_LN2(8); }
    else if (per <= 16) { TU_LN2(16); }
    else if (per <= 20) { TU_LN2(20); }
    else if (per <= kMaxPerThread) { TU_LN2(32); }
    else TU_LN(0, false, false);
#undef TU_LN2
#undef TU_LN
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_layer_norm_adaln(const void *x, const void *scale, const void *shift, void *out, int32_t dtype,
                                       int64_t batch, int64_t len, int64_t hidden, int64_t steps, float eps,
                                       void *stream) {
    using namespace tu;
    TU_REQUIRE(dtype >= 0 && dtype <= 2, "LayerNorm+AdaLN dtype must be 0 (bf16), 1 (fp16) or 2 (fp32), got %d",
               dtype);
    TU_REQUIRE(batch > 0 && len > 0 && hidden > 0 && steps > 0, "LayerNorm+AdaLN dimensions must be positive");
    TU_REQUIRE(batch * len <= 0x7fffffff && hidden <= 0x7fffffff && steps <= 0x7fffffff,
               "LayerNorm+AdaLN dimensions exceed the kernel range");
    TU_REQUIRE(eps > 0.0f && eps <= 3.4e38f, "LayerNorm epsilon must be finite and positive");
    TU_REQUIRE(x && scale && shift && out, "LayerNorm+AdaLN pointers must be non-null");
    if (require_gfx950()) return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int h = static_cast<int>(hidden);
    if (dtype == 2) launch<2, false>(x, scale, shift, out, batch * len, len, h, steps, eps, s);
    else if (dtype == 1) launch<1, false>(x, scale, shift, out, batch * len, len, h, steps, eps, s);
    else launch<0, false>(x, scale, shift, out, batch * len, len, h, steps, eps, s);
    return check_launch("tu_layer_norm_adaln");
}

extern "C" int32_t tu_layer_norm_affine(const void *x, const void *weight, const void *bias, void *out,
                                        int32_t dtype, int64_t rows, int64_t hidden, float eps, void *stream) {
    using namespace tu;
    TU_REQUIRE(dtype >= 0 && dtype <= 2, "LayerNorm dtype must be 0 (bf16), 1 (fp16) or 2 (fp32), got %d", dtype);
    TU_REQUIRE(rows >= 0 && hidden > 0, "LayerNorm rows must be >= 0 and hidden positive");
    TU_REQUIRE(rows <= 0x7fffffff && hidden <= 0x7fffffff, "LayerNorm dimensions exceed the kernel range");
    TU_REQUIRE(eps > 0.0f && eps <= 3.4e38f, "LayerNorm epsilon must be finite and positive");
    TU_REQUIRE(x && weight && bias && out, "LayerNorm pointers must be non-null");
    if (require_gfx950()) return -1;
    if (rows == 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int h = static_cast<int>(hidden);
    // one batch of `rows` tokens and a single "modulation" row: weight / bias
    if (dtype == 2) launch<2, true>(x, weight, bias, out, rows, rows, h, 1, eps, s);
    else if (dtype == 1) launch<1, true>(x, weight, bias, out, rows, rows, h, 1, eps, s);
    else launch<0, true>(x, weight, bias, out, rows, rows, h, 1, eps, s);
    return check_launch("tu_layer_norm_affine");
}
