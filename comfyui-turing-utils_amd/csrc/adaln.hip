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
#include "ln_common.h"

namespace tu {
namespace {

constexpr int kThreads = kLnThreads;
constexpr int kMaxPerThread = 32;  // register-resident rows: hidden <= 8192

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
// 16-bit rows with hidden = 256 per (per <= kPer): the statistics of
// ln16_row_stats, one row per half-wave, eight rows per workgroup.
// ---------------------------------------------------------------------------
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

    float mu, inv;
    ln16_row_stats<kT, kPer>(xs, per, hidden, eps, rc, (tid & 32) << 2, mu, inv);
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
            const u32x4 o = ln16_emit8<kT, kAffine>(xs[i], mv, hv, mu, inv);
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
    const bool uniform = hidden % kThreads == 0 && per <= kMaxPerThread;
    const Recips rc = uniform ? uniform_recips(per) : Recips{};
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
