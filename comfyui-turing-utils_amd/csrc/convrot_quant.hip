// ConvRot INT8 activation quantizer for gfx950.
//
// Semantics follow the reference's whole-row ("row-buffer") kernel
// bf16_rowbuffer_convrot_quantize_kernel<T, SwiGLU=false, Int4=false>
// (kernel/csrc/turing/convrot_quant.cu:350-444):
//   1. each group of G columns is rotated by the block-Hadamard transform in
//      fp32, one radix-4 digit at a time (stride 1 -> 4 -> 16 -> 64) with the
//      exact add order of convrot_quant.cu:104-116;
//   2. the row absmax is taken over the fp32 outputs, the outputs are kept as
//      bf16 (round-to-nearest-even);
//   3. scale = max(min(absmax, bf16 max) / 127, 1e-30);
//      q = clamp(rne(bf16(bf16(y) / bf16(scale))), -128, 127).
// With the staged-scale flag the scale is absmax * (1/127) instead, as in the
// reference's two-pass kernels (convrot_quant.cu:233-236) behind the
// gelu_/swiglu_int8_convrot_quantize ops; everything else is identical.
// G = 128 is this build's extension: three radix-4 digits then the
// orthonormal radix-2 digit (1/sqrt2)[[1,1],[1,-1]] on stride 64.
//
// MI355X mapping: one workgroup (4 wave64) per row.  Each wave rotates whole
// groups in its own 1 KiB LDS scratch (no workgroup barrier between stages),
// writes the bf16 row into an LDS row buffer and reduces the absmax with
// cross-lane max; one workgroup barrier, then every thread quantizes 8
// contiguous columns (16 B LDS read, 8 B global store).  The division by
// bf16(scale) is a reciprocal multiply plus one FMA correction (Markstein),
// which the CPU tests prove yields the same INT8 code as IEEE division for
// every (value, scale) pair the quantizer can produce.
#include "tu_common.h"

namespace tu {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr float kInvSqrt2 = 0.70710678118654752440f;

__device__ __forceinline__ void lds_wave_sync() {
    // LDS operations of one wave complete in order; this stops the compiler
    // from moving LDS accesses across the point and drains outstanding ones.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// One radix-4 digit in place on buf (G floats): lane gl owns the 4 elements
// base + {0, 1, 2, 3} * S, base = (gl % S) + (gl / S) * 4S.
template <int S>
__device__ __forceinline__ void r4_stage_lds(float *buf, int gl) {
    const int base = (gl % S) + (gl / S) * (4 * S);
    const float x0 = buf[base];
    const float x1 = buf[base + S];
    const float x2 = buf[base + 2 * S];
    const float x3 = buf[base + 3 * S];
    buf[base] = 0.5f * (((x0 + x1) + x2) - x3);
    buf[base + S] = 0.5f * (((x0 + x1) - x2) + x3);
    buf[base + 2 * S] = 0.5f * (((x0 - x1) + x2) + x3);
    buf[base + 3 * S] = 0.5f * (((-x0 + x1) + x2) + x3);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Correctly rounded quotient a / b for the quantizer's domain, given
// y = RN(1 / b): q0 = RN(a y), r = a - b q0 (exact by FMA), RN(q0 + r y).
__device__ __forceinline__ float div_markstein(float a, float b, float y) {
    const float q0 = a * y;
    const float r = __builtin_fmaf(-q0, b, a);
    const float q = __builtin_fmaf(r, y, q0);
    return __builtin_isinf(a) ? a : q;
}

// Input activations, operation for operation the fixed fp32 sequences of the
// CPU oracle (exp by Cody-Waite reduction and a degree-7 Taylor polynomial,
// tanh from exp), so activation outputs are bit-identical to it:
//   tanh-GELU: bf16((0.5 x) (1 + tanh(a (x + ((b x) x) x))))  (convrot_quant.cu:145-156)
//   SwiGLU:    (g / (1 + exp(-g))) u                           (convrot_quant.cu:137-143)
__device__ __forceinline__ float exp_det(float v) {
    if (v != v) return v;
    if (v > 88.72f) return __builtin_inff();
    if (v < -87.0f) return 0.0f;
    const float n = __builtin_rintf(v * 1.44269504f);
    const float r = (v - n * 0.693145752f) - n * 1.42860677e-6f;
    float p = 1.98412698e-4f;
    p = p * r + 1.38888889e-3f;
    p = p * r + 8.33333377e-3f;
    p = p * r + 4.16666679e-2f;
    p = p * r + 1.66666672e-1f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return __builtin_ldexpf(p, static_cast<int>(n));
}

__device__ __forceinline__ float tanh_det(float u) {
    if (u != u) return u;
    const float a = fabsf(u);
    const float e = exp_det(2.0f * fminf(a, 9.0f));
    float t = 1.0f - 2.0f / (e + 1.0f);
    t = a < 0.000244140625f ? a : t;
    t = a > 9.0f ? 1.0f : t;
    return __builtin_copysignf(t, u);
}

__device__ __forceinline__ float gelu_tanh_bf16(float x) {
    const float inner = 0.7978845608028654f * (x + ((0.044715f * x) * x) * x);
    const float act = (0.5f * x) * (1.0f + tanh_det(inner));
    return bf16_round(act);
}

__device__ __forceinline__ float swiglu(float gate, float up) { return (gate / (1.0f + exp_det(-gate))) * up; }

__device__ __forceinline__ int32_t quant_code(float v, float rs, float ry) {
    const float divided = bf16_round(div_markstein(v, rs, ry));
    float qf = __builtin_rintf(divided);
    qf = fminf(127.0f, fmaxf(-128.0f, qf));
    return static_cast<int32_t>(qf);
}

// kAct: 0 none, 1 tanh-GELU, 2 SwiGLU (x rows are [gate | up], 2k wide).
template <int G, int kAct>
__global__ __launch_bounds__(kThreads) void convrot_quant_i8_kernel(
    const uint16_t *__restrict__ x, int8_t *__restrict__ q, float *__restrict__ scales, int k,
    int row_buffer_bytes, int staged_scale) {
    extern __shared__ __align__(16) unsigned char smem[];
    uint16_t *row_buf = reinterpret_cast<uint16_t *>(smem);
    __shared__ float wave_amax[kWaves];

    constexpr int kLanesPerGroup = G / 4;           // each lane holds 4 elements
    constexpr int kGroupsPerWave = 64 / kLanesPerGroup;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int gsub = lane / kLanesPerGroup;
    const int gl = lane % kLanesPerGroup;
    float *buf = reinterpret_cast<float *>(smem + row_buffer_bytes) + wave * 256 + gsub * G;

    const int64_t row = blockIdx.x;
    const uint16_t *xrow = x + row * static_cast<int64_t>(kAct == 2 ? 2 * k : k);
    const int groups = k / G;
    float absmax = 0.0f;

    for (int g0 = wave * kGroupsPerWave; g0 < groups; g0 += kWaves * kGroupsPerWave) {
        const int g = g0 + gsub;
        const bool active = g < groups;
        const int col = g * G + 4 * gl;
        float x0 = 0.0f, x1 = 0.0f, x2 = 0.0f, x3 = 0.0f;
        if (active) {
            const u32x2 v = *reinterpret_cast<const u32x2 *>(xrow + col);
            x0 = bf16_bits_to_f32(v.x & 0xffffu);
            x1 = bf16_bits_to_f32(v.x >> 16);
            x2 = bf16_bits_to_f32(v.y & 0xffffu);
            x3 = bf16_bits_to_f32(v.y >> 16);
            if constexpr (kAct == 1) {
                x0 = gelu_tanh_bf16(x0);
                x1 = gelu_tanh_bf16(x1);
                x2 = gelu_tanh_bf16(x2);
                x3 = gelu_tanh_bf16(x3);
            } else if constexpr (kAct == 2) {
                const u32x2 u = *reinterpret_cast<const u32x2 *>(xrow + k + col);
                x0 = swiglu(x0, bf16_bits_to_f32(u.x & 0xffffu));
                x1 = swiglu(x1, bf16_bits_to_f32(u.x >> 16));
                x2 = swiglu(x2, bf16_bits_to_f32(u.y & 0xffffu));
                x3 = swiglu(x3, bf16_bits_to_f32(u.y >> 16));
            }
        }
        // Stride-1 digit in registers (convrot_quant.cu:384-391).
        f32x4 y;
        y.x = 0.5f * (((x0 + x1) + x2) - x3);
        y.y = 0.5f * (((x0 + x1) - x2) + x3);
        y.z = 0.5f * (((x0 - x1) + x2) + x3);
        y.w = 0.5f * (((-x0 + x1) + x2) + x3);
        *reinterpret_cast<f32x4 *>(buf + 4 * gl) = y;
        lds_wave_sync();
        r4_stage_lds<4>(buf, gl);
        lds_wave_sync();
        r4_stage_lds<16>(buf, gl);
        lds_wave_sync();
        if constexpr (G == 256) {
            // Stride-64 digit, stored as bf16 (convrot_quant.cu:311-330).
            const int base = gl;
            const float a0 = buf[base], a1 = buf[base + 64], a2 = buf[base + 128],
                        a3 = buf[base + 192];
            const float o0 = 0.5f * (((a0 + a1) + a2) - a3);
            const float o1 = 0.5f * (((a0 + a1) - a2) + a3);
            const float o2 = 0.5f * (((a0 - a1) + a2) + a3);
            const float o3 = 0.5f * (((-a0 + a1) + a2) + a3);
            if (active) {
                absmax = fmaxf(absmax, fmaxf(fmaxf(fabsf(o0), fabsf(o1)), fmaxf(fabsf(o2), fabsf(o3))));
                uint16_t *dst = row_buf + g * G + base;
                dst[0] = static_cast<uint16_t>(bf16_rne_bits(o0));
                dst[64] = static_cast<uint16_t>(bf16_rne_bits(o1));
                dst[128] = static_cast<uint16_t>(bf16_rne_bits(o2));
                dst[192] = static_cast<uint16_t>(bf16_rne_bits(o3));
            }
        } else {
            // Radix-2 digit on stride 64: lane gl owns pairs (b, b + 64) for
            // b = gl and b = gl + 32.
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int base = gl + 32 * h;
                const float a0 = buf[base], a1 = buf[base + 64];
                const float o0 = kInvSqrt2 * (a0 + a1);
                const float o1 = kInvSqrt2 * (a0 - a1);
                if (active) {
                    absmax = fmaxf(absmax, fmaxf(fabsf(o0), fabsf(o1)));
                    uint16_t *dst = row_buf + g * G + base;
                    dst[0] = static_cast<uint16_t>(bf16_rne_bits(o0));
                    dst[64] = static_cast<uint16_t>(bf16_rne_bits(o1));
                }
            }
        }
        lds_wave_sync();
    }

    absmax = wave_max(absmax);
    if (lane == 0) wave_amax[wave] = absmax;
    __syncthreads();
    float amax = wave_amax[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) amax = fmaxf(amax, wave_amax[w]);
    const float clipped = fminf(amax, 3.38953139e38f);
    const float scale = fmaxf(staged_scale ? clipped * (1.0f / 127.0f) : clipped / 127.0f, 1.0e-30f);
    if (tid == 0) scales[row] = scale;
    const float rs = bf16_round(scale);
    const float ry = 1.0f / rs;

    int8_t *qrow = q + row * static_cast<int64_t>(k);
    for (int c = tid * 8; c < k; c += kThreads * 8) {
        const u32x4 v = *reinterpret_cast<const u32x4 *>(row_buf + c);
        uint32_t packed[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t w0 = h ? v.z : v.x;
            const uint32_t w1 = h ? v.w : v.y;
            const int32_t c0 = quant_code(bf16_bits_to_f32(w0 & 0xffffu), rs, ry);
            const int32_t c1 = quant_code(bf16_bits_to_f32(w0 >> 16), rs, ry);
            const int32_t c2 = quant_code(bf16_bits_to_f32(w1 & 0xffffu), rs, ry);
            const int32_t c3 = quant_code(bf16_bits_to_f32(w1 >> 16), rs, ry);
            packed[h] = (static_cast<uint32_t>(c0) & 0xffu) | ((static_cast<uint32_t>(c1) & 0xffu) << 8) |
                        ((static_cast<uint32_t>(c2) & 0xffu) << 16) | (static_cast<uint32_t>(c3) << 24);
        }
        u32x2 out;
        out.x = packed[0];
        out.y = packed[1];
        *reinterpret_cast<u32x2 *>(qrow + c) = out;
    }
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_convrot_quant_i8(const void *x_bf16, int8_t *q, float *scale, int64_t rows,
                                       int64_t cols, int32_t group, int32_t act, void *stream) {
    using namespace tu;
    TU_REQUIRE(group == 128 || group == 256, "ConvRot group_size must be 128 or 256, got %d", group);
    const int staged_scale = (act & TU_CONVROT_STAGED_SCALE) != 0;
    act &= ~TU_CONVROT_STAGED_SCALE;
    TU_REQUIRE(act >= TU_ACT_NONE && act <= TU_ACT_SWIGLU,
               "ConvRot input activation must be 0 (none), 1 (tanh-GELU) or 2 (SwiGLU), got %d", act);
    TU_REQUIRE(rows >= 0 && cols > 0 && cols % group == 0,
               "ConvRot width must be positive and divisible by %d, got %lld", group,
               static_cast<long long>(cols));
    TU_REQUIRE(rows <= 0x7fffffff && cols <= (1 << 20), "ConvRot dimensions out of range");
    TU_REQUIRE(x_bf16 && q && scale, "ConvRot pointers must be non-null");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(x_bf16) & 7) == 0 && (reinterpret_cast<uintptr_t>(q) & 7) == 0,
               "ConvRot input must be 8-byte aligned");
    if (require_gfx950()) return -1;
    if (rows == 0) return 0;
    const int k = static_cast<int>(cols);
    const int row_buffer_bytes = (k * 2 + 15) / 16 * 16;
    const size_t lds = static_cast<size_t>(row_buffer_bytes) + kWaves * 256 * sizeof(float);
    TU_REQUIRE(lds <= 160 * 1024 - 64, "ConvRot row of %d columns exceeds LDS", k);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(rows));
    const auto *xp = static_cast<const uint16_t *>(x_bf16);
#define TU_CONVROT_LAUNCH(G, A) convrot_quant_i8_kernel<G, A><<<grid, kThreads, lds, s>>>(xp, q, scale, k, row_buffer_bytes, staged_scale)
    if (group == 256) {
        if (act == 0) TU_CONVROT_LAUNCH(256, 0);
        else if (act == 1) TU_CONVROT_LAUNCH(256, 1);
        else TU_CONVROT_LAUNCH(256, 2);
    } else {
        if (act == 0) TU_CONVROT_LAUNCH(128, 0);
        else if (act == 1) TU_CONVROT_LAUNCH(128, 1);
        else TU_CONVROT_LAUNCH(128, 2);
    }
#undef TU_CONVROT_LAUNCH
    return check_launch("tu_convrot_quant_i8");
}
