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
