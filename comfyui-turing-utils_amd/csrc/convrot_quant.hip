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
// With the fp16-input flag the elements are IEEE binary16, as the two-pass
// kernels' InputType = half instantiation (convrot_quant.cu:158-248): GELU
// output, rotated values and the quotient are rounded to fp16 where the bf16
// path rounds to bf16, the absmax clip is 65504 (finite_max<half>, :58-62),
// and the quotient is an IEEE division by fp16(scale) (quant_div_to_float,
// :69-73).  fp16(scale) is 0 when scale < 2^-25 (all-zero or tiny rows): the
// reference then divides by zero and its clamp maps the resulting +-inf to
// 127 / -128 and NaN (0 / 0) to -128; the same happens here.
// G = 128 is this build's extension: three radix-4 digits then the
// orthonormal radix-2 digit (1/sqrt2)[[1,1],[1,-1]] on stride 64.
//
// MI355X mapping: one workgroup per row; the row is cut into 1024-column
// chunks and each wave takes up to four of them (ceil(chunks / 4) waves),
// loading all of its input with 16-byte loads before any arithmetic.  Few
// waves per row keep the per-row barrier short and let more rows share a CU
// (measured faster than one chunk per wave).  A lane holds 16 consecutive
// columns of one group, so the stride-1 and
// stride-4 digits are register arithmetic.  One wave-local LDS transpose
// (fp32, padded so reads are conflict-free) then gives each lane the 16
// elements that share their two low digits, and the stride-16 and stride-64
// digits are register arithmetic again.  The rotated values stay in
// registers as packed bf16 while the row absmax is reduced (cross-lane max,
// one workgroup barrier); each lane then quantizes its own values and a
// second, byte-sized wave-local transpose puts the codes back in column order
// for 16-byte stores.  The division by bf16(scale) is one multiply by its
// correctly rounded reciprocal: its fp32 result can differ from the IEEE
// quotient in the last place, but value and scale both carry 8 significant
// bits, so the quotient is never that close to a bf16 rounding midpoint, and
// the CPU tests check, over every (value, scale) pair the quantizer can
// produce, that the INT8 code is the IEEE division's.
#include <type_traits>

#include "ln_common.h"
#include "tu_common.h"

namespace tu {
namespace {

constexpr int kChunk = 1024;      // columns per wave pass: 64 lanes x 16
constexpr int kMaxWaves = 16;
constexpr int kTableThreads = 512;  // waves of a GELU-by-table workgroup, at most 8
constexpr int kMaxPasses = 4;     // so a row holds at most 65536 columns
constexpr int kMaxCols = kChunk * kMaxWaves * kMaxPasses;
constexpr int kScratchBytes = 8 * 144 * 4;  // per wave: the larger of the two padded layouts
constexpr float kInvSqrt2 = 0.70710678118654752440f;
// Per-group slots of a wave's scratch: the fp32 transpose (dwords, padded so
// the groups of a wave fall on different banks) and the code transpose (bytes).
template <int G> constexpr int group_dwords() { return G == 128 ? 144 : 272; }
template <int G> constexpr int code_group_bytes() { return G + 16; }

__device__ __forceinline__ void lds_wave_sync() {
    // LDS operations of one wave complete in order; this stops the compiler
    // from moving LDS accesses across the point and drains outstanding ones.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// One radix-4 butterfly in the reference's add order (convrot_quant.cu:104-116).
__device__ __forceinline__ void r4(float &x0, float &x1, float &x2, float &x3) {
    const float y0 = 0.5f * (((x0 + x1) + x2) - x3);
    const float y1 = 0.5f * (((x0 + x1) - x2) + x3);
    const float y2 = 0.5f * (((x0 - x1) + x2) + x3);
    const float y3 = 0.5f * (((-x0 + x1) + x2) + x3);
    x0 = y0;
    x1 = y1;
    x2 = y2;
    x3 = y3;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
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

// exp_det on [0, 18], where none of its guards applies: the same operations.
__device__ __forceinline__ float exp_det_0_18(float v) {
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

template <bool kF16>
__device__ __forceinline__ float tanh_det(float u) {
    if (u != u) return u;
    const float a = fabsf(u);
    const float e = exp_det_0_18(2.0f * fminf(a, 9.0f));
    // 2 / b for b = e + 1 in [2, 7e7].  bf16 inputs: q0 = 2 rcp(b), one FMA
    // residual and one FMA correction, equal to the IEEE quotient for every b
    // that a bf16 input reaches (the GELU quantizer's GPU test runs all of
    // them).  fp16 inputs reach other values of b: IEEE division.
    const float b = e + 1.0f;
    float q;
    if constexpr (kF16) {
        q = 2.0f / b;
    } else {
        const float y = __builtin_amdgcn_rcpf(b);
        const float q0 = 2.0f * y;
        q = __builtin_fmaf(__builtin_fmaf(-q0, b, 2.0f), y, q0);
    }
    float t = 1.0f - q;
    t = a < 0.000244140625f ? a : t;
    t = a > 9.0f ? 1.0f : t;
    return __builtin_copysignf(t, u);
}

template <bool kF16>
__device__ __forceinline__ float gelu_tanh_f32(float x) {
    const float inner = 0.7978845608028654f * (x + ((0.044715f * x) * x) * x);
    return (0.5f * x) * (1.0f + tanh_det<kF16>(inner));
}

__device__ __forceinline__ float swiglu(float gate, float up) { return (gate / (1.0f + exp_det(-gate))) * up; }

// Round-to-nearest-even to bf16 by the gfx950 conversion instruction
// (v_cvt_pk_bf16_f32).  Identical to bf16_rne_bits for every non-NaN input;
// a NaN keeps an unspecified NaN payload, which is harmless where this is
// used: the rotated row buffer and the quotient only feed the division,
// rint and clamp, where any NaN yields the same code.
__device__ __forceinline__ uint16_t hw_bf16_bits(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
}

// fp16 (RNE by the hardware conversion) and back.  The empty asm pins the
// fp32 value first, so the compiler cannot fold "fp32 multiply, then round to
// fp16" into one single-rounding mixed-precision FMA.
__device__ __forceinline__ uint16_t hw_f16_bits(float v) {
    asm("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}
__device__ __forceinline__ float hw_f16_round(float v) { return f16_bits_to_f32(hw_f16_bits(v)); }

// Element type of the input and of the rotated row buffer.
template <bool kF16>
__device__ __forceinline__ float elem_to_f32(uint32_t b) {
    if constexpr (kF16) return f16_bits_to_f32(b & 0xffffu);
    else return bf16_bits_to_f32(b & 0xffffu);
}
template <bool kF16>
__device__ __forceinline__ uint32_t elem_bits(float v) {
    if constexpr (kF16) return hw_f16_bits(v);
    else return hw_bf16_bits(v);
}

__device__ __forceinline__ int32_t code_of(float divided) {
    float qf = __builtin_rintf(divided);
    qf = fminf(127.0f, fmaxf(-128.0f, qf));
    return static_cast<int32_t>(qf);
}

// Codes of two values: both quotients rounded to bf16 by one conversion.
__device__ __forceinline__ void quant_code2(float v0, float v1, float ry, int32_t &c0, int32_t &c1) {
    const uint32_t d = hw_bf16x2_bits(v0 * ry, v1 * ry);
    c0 = code_of(__uint_as_float(d << 16));
    c1 = code_of(__uint_as_float(d & 0xffff0000u));
}

// fp16 elements: fp16(v / rs) with IEEE division (rs may be 0, see the top).
__device__ __forceinline__ int32_t quant_code_f16(float v, float rs) {
    const float divided = hw_f16_round(v / rs);
    float qf = __builtin_rintf(divided);
    qf = fminf(127.0f, fmaxf(-128.0f, qf));
    return static_cast<int32_t>(qf);
}

// The GELU output is rounded to the element type before the rotation
// (convrot_quant.cu:153-155); SwiGLU's is not (:137-143).
template <bool kF16>
__device__ __forceinline__ float activate(float v, float up, std::integral_constant<int, 0>) { return v; }
template <bool kF16>
__device__ __forceinline__ float activate(float v, float up, std::integral_constant<int, 1>) {
    if constexpr (kF16) return hw_f16_round(gelu_tanh_f32<true>(v));
    else return bf16_round(gelu_tanh_f32<false>(v));
}
template <bool kF16>
__device__ __forceinline__ float activate(float v, float up, std::integral_constant<int, 2>) { return swiglu(v, up); }

// bf16 tanh-GELU by table.  The output is a function of the input's 16 bits:
//   |x| in [2^-12, 8): a table of the 2 x 15 x 128 bf16 values there, built
//     in LDS by each workgroup with activate<false> itself, so equal to it
//     by construction;
//   |x| < 2^-12: |inner| < 2^-12, so tanh_det returns inner unchanged and
//     gelu = bf16((0.5 x) (1 + inner)) = bf16(0.5 x): 0.5 x is exact, and
//     either 1 + inner rounds to 1 (|x| < 2^-24) or 0.5 x is a normal bf16
//     value that a relative change below 2^-12 cannot round away from;
//   8 <= |x| < inf: inner > 9, tanh_det returns +-1, gelu = x (x > 0) or -0;
//   inf / NaN: activate<false> itself (the caller's rare branch).
// The table interleaves the signs: entry 2 (mag - kGeluLutLo) + sign.
constexpr uint32_t kGeluLutLo = 115u << 7;  // magnitude bits of 2^-12
constexpr int kGeluLutHalf = 15 * 128;      // exponents 2^-12 .. 2^2, 128 mantissas each
// Both signs, each padded to 2048 entries so that any 11-bit rel indexes
// inside the table (the padding is never selected).
constexpr int kGeluLut = 2 * 2048;

__device__ __forceinline__ uint32_t gelu_lut_entry(int idx) {
    if ((idx >> 1) >= kGeluLutHalf) return 0u;  // padding
    const uint32_t bits = (static_cast<uint32_t>(idx & 1) << 15) | (kGeluLutLo + static_cast<uint32_t>(idx >> 1));
    const float g = activate<false>(bf16_bits_to_f32(bits), 0.0f, std::integral_constant<int, 1>{});
    return __float_as_uint(g) >> 16;  // exact: g is a bf16 value (or the canonical NaN)
}

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// 0xffff in each 16-bit half of x whose bit 15 is set, else 0 (one
// v_pk_ashrrev_i16; written out because the compiler otherwise splits the
// halves into compares and selects).  op_sel_hi:[0,1]: the high half also
// takes its shift count from the low 16 bits of the constant 15.
__device__ __forceinline__ uint32_t half_sign_masks(uint32_t x) {
    uint32_t r;
    asm("v_pk_ashrrev_i16 %0, 15, %1 op_sel_hi:[0,1]" : "=v"(r) : "v"(x));
    return r;
}

// GELU of the two bf16 values packed in w (low half first) as two packed
// bf16 results, on packed 16-bit integer arithmetic: per half,
//   rel = mag - kGeluLutLo (wrapping: >= 0x8000 exactly for |x| < 2^-12,
//         since mag - kGeluLutLo <= 0x7fff - kGeluLutLo < 0x8000 otherwise),
//   rel < kGeluLutHalf: the table; rel >= 0x8000: bf16(0.5 x); else x or -0.
// Split in steps so that a lane's table reads can all be in flight before
// the first is used: gelu_pair_lookup reads the two entries, then
// gelu_pair_fast (a wave whose pass has no unusual input) or
// gelu_pair_select (any input) picks the results.
__device__ __forceinline__ uint32_t gelu_pair_rel(uint32_t w) {
    const u16x2 rel = __builtin_bit_cast(u16x2, w & 0x7fff7fffu) - static_cast<uint16_t>(kGeluLutLo);
    return __builtin_bit_cast(uint32_t, rel);
}

// The table entries of both halves of w, at byte offset 4 (rel mod 2048) +
// 2 sign: one packed shift of rel, one of w and one bit-select make both
// offsets (entries of halves outside the table range are read, in bounds,
// and never selected).
__device__ __forceinline__ uint32_t gelu_pair_lookup(uint32_t w, uint32_t rel2, const uint16_t *lut) {
    const uint32_t t = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, rel2) << static_cast<uint16_t>(2));
    const uint32_t sg = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, w) >> static_cast<uint16_t>(14));
    const uint32_t off = (t & 0x1ffd1ffdu) | (sg & 0xe002e002u);
    const unsigned char *base = reinterpret_cast<const unsigned char *>(lut);
    return static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(base + (off & 0xffffu))) |
           (static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(base + (off >> 16))) << 16);
}

// GELU of a pair whose halves all have exponent fields in [2, 254] (no zero,
// subnormal, smallest-binade, inf or NaN input; gelu_pair_unusual flags the
// others): rel < kGeluLutHalf the table; |x| < 2^-12 (rel >= 0x8000)
// bf16(0.5 x), which for these exponent fields is x with its exponent field
// lowered by one, exactly; otherwise |x| >= 8, x or -0.
__device__ __forceinline__ uint32_t gelu_pair_fast(uint32_t w, uint32_t rel2, uint32_t table) {
    const uint32_t tiny = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, w) - static_cast<uint16_t>(0x80));
    const uint32_t neg = half_sign_masks(w);
    const uint32_t big = (w & ~neg) | (0x80008000u & neg);
    // rel + (0x8000 - kGeluLutHalf), saturating: bit 15 set iff rel >= kGeluLutHalf
    const u16x2 past = __builtin_elementwise_add_sat(__builtin_bit_cast(u16x2, rel2),
                                                     static_cast<u16x2>(static_cast<uint16_t>(0x8000 - kGeluLutHalf)));
    const uint32_t outside = half_sign_masks(__builtin_bit_cast(uint32_t, past));
    const uint32_t is_tiny = half_sign_masks(rel2);
    const uint32_t r = (big & outside) | (table & ~outside);
    return (tiny & is_tiny) | (r & ~is_tiny);
}

// Bit 15 of a half set iff its exponent field is 0, 1 or 255: magnitude
// bits - 0x100 (wrapping) + 0x180, saturating.
__device__ __forceinline__ uint32_t gelu_pair_unusual(uint32_t w) {
    const u16x2 mag = __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_add_sat(mag - static_cast<uint16_t>(0x100),
                                                                      static_cast<u16x2>(static_cast<uint16_t>(0x180))));
}

__device__ __forceinline__ uint32_t gelu_pair_select(uint32_t w, uint32_t rel2, uint32_t table) {
    const uint32_t tiny = hw_bf16x2_bits(0.5f * __uint_as_float(w << 16), 0.5f * __uint_as_float(w & 0xffff0000u));
    const uint32_t neg = half_sign_masks(w);
    const uint32_t big = (w & ~neg) | (0x80008000u & neg);  // x, or -0 for negative x
    const u16x2 past = __builtin_bit_cast(u16x2, rel2) - static_cast<uint16_t>(kGeluLutHalf);
    const uint32_t table_or_tiny = half_sign_masks(__builtin_bit_cast(uint32_t, past));
    const uint32_t is_tiny = half_sign_masks(rel2);
    const uint32_t r = (table & table_or_tiny) | (big & ~table_or_tiny);
    return (tiny & is_tiny) | (r & ~is_tiny);
}

// Rotation of one pass.  Lane (gi, L) holds v = the 16 consecutive columns
// 16 L .. 16 L + 15 of group gi (element index 16 L + p, p = d0 + 4 d1); on
// return z holds its rotated values after the transpose through `grp` (the
// group's slot of the wave's scratch): for G = 256, p = L and t = d2 + 4 d3 =
// 0..15 in z[t]; for G = 128, p = 2L and 2L + 1 in z[t] and z[8 + t] with
// t = d2 + 4 d3 = 0..7.
template <int G>
__device__ __forceinline__ void rotate_pass(float (&v)[16], float *grp, int L, float (&z)[16]) {
    // Digits d0 (stride 1) and d1 (stride 4) in registers (convrot_quant.cu:384-391).
#pragma unroll
    for (int d1 = 0; d1 < 4; ++d1) r4(v[4 * d1], v[4 * d1 + 1], v[4 * d1 + 2], v[4 * d1 + 3]);
#pragma unroll
    for (int d0 = 0; d0 < 4; ++d0) r4(v[d0], v[d0 + 4], v[d0 + 8], v[d0 + 12]);

    // Wave-local transpose through LDS.
    lds_wave_sync();  // earlier reads of the scratch are done
#pragma unroll
    for (int c = 0; c < 4; ++c)
        *reinterpret_cast<f32x4 *>(grp + 16 * L + 4 * ((c + (L >> 2)) & 3)) =
            f32x4{v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]};
    lds_wave_sync();
    if constexpr (G == 256) {
#pragma unroll
        for (int t = 0; t < 16; ++t) z[t] = grp[16 * t + 4 * (((L >> 2) + (t >> 2)) & 3) + (L & 3)];
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const f32x2 pair = *reinterpret_cast<const f32x2 *>(
                grp + 16 * t + 4 * (((L >> 1) + (t >> 2)) & 3) + ((2 * L) & 3));
            z[t] = pair.x;
            z[8 + t] = pair.y;
        }
    }

    // Digits d2 (stride 16) and d3 (stride 64) in registers (convrot_quant.cu:311-330).
    if constexpr (G == 256) {
#pragma unroll
        for (int d3 = 0; d3 < 4; ++d3) r4(z[4 * d3], z[4 * d3 + 1], z[4 * d3 + 2], z[4 * d3 + 3]);
#pragma unroll
        for (int d2 = 0; d2 < 4; ++d2) r4(z[d2], z[d2 + 4], z[d2 + 8], z[d2 + 12]);
    } else {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int d3 = 0; d3 < 2; ++d3)
                r4(z[8 * h + 4 * d3], z[8 * h + 4 * d3 + 1], z[8 * h + 4 * d3 + 2], z[8 * h + 4 * d3 + 3]);
            // Radix-2 digit on stride 64: (1/sqrt2) [[1, 1], [1, -1]].
#pragma unroll
            for (int d2 = 0; d2 < 4; ++d2) {
                const float a0 = z[8 * h + d2], a1 = z[8 * h + d2 + 4];
                z[8 * h + d2] = kInvSqrt2 * (a0 + a1);
                z[8 * h + d2 + 4] = kInvSqrt2 * (a0 - a1);
            }
        }
    }
}

// Codes of one pass back in column order: element 16 t + p of the lane's
// group is byte 16 t + p of `gb` (the group's slot of the wave's scratch,
// G + 16 bytes); returns the 16 codes of the lane's own columns.  `packed`
// holds the rotated values as element-type pairs in z order (G = 256:
// t = 2j, 2j + 1 of p = L; G = 128: p = 2L (low) and 2L + 1 (high) of t = j).
template <int G, bool kF16>
__device__ __forceinline__ u32x4 pass_codes(const uint32_t (&packed)[8], float rs, float ry, unsigned char *gb,
                                            int L) {
    lds_wave_sync();  // the scratch is free (transposed reads consumed)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t w = packed[j];
        uint32_t c0, c1;
        if constexpr (kF16) {
            c0 = static_cast<uint32_t>(quant_code_f16(f16_bits_to_f32(w & 0xffffu), rs)) & 0xffu;
            c1 = static_cast<uint32_t>(quant_code_f16(f16_bits_to_f32(w >> 16), rs)) & 0xffu;
        } else {
            int32_t i0, i1;
            quant_code2(bf16_bits_to_f32(w & 0xffffu), __uint_as_float(w & 0xffff0000u), ry, i0, i1);
            c0 = static_cast<uint32_t>(i0) & 0xffu;
            c1 = static_cast<uint32_t>(i1) & 0xffu;
        }
        if constexpr (G == 256) {
            gb[32 * j + L] = static_cast<unsigned char>(c0);
            gb[32 * j + 16 + L] = static_cast<unsigned char>(c1);
        } else {
            *reinterpret_cast<uint16_t *>(gb + 16 * j + 2 * L) = static_cast<uint16_t>(c0 | (c1 << 8));
        }
    }
    lds_wave_sync();
    return *reinterpret_cast<const u32x4 *>(gb + 16 * L);
}

// Raw bf16 input of one lane for one pass: 16 columns (and 16 "up" columns
// for SwiGLU).
template <int kAct>
struct LaneInput {
    u32x4 x[2];
    u32x4 up[kAct == 2 ? 2 : 1];
};

template <int kAct>
__device__ __forceinline__ void load_lane(LaneInput<kAct> &in, const uint16_t *xrow, int k, int col) {
    in.x[0] = u32x4{0u, 0u, 0u, 0u};
    in.x[1] = u32x4{0u, 0u, 0u, 0u};
    if constexpr (kAct == 2) {
        in.up[0] = u32x4{0u, 0u, 0u, 0u};
        in.up[1] = u32x4{0u, 0u, 0u, 0u};
    }
    if (col < k) {
        in.x[0] = *reinterpret_cast<const u32x4 *>(xrow + col);
        in.x[1] = *reinterpret_cast<const u32x4 *>(xrow + col + 8);
        if constexpr (kAct == 2) {
            in.up[0] = *reinterpret_cast<const u32x4 *>(xrow + k + col);
            in.up[1] = *reinterpret_cast<const u32x4 *>(xrow + k + col + 8);
        }
    }
}

// kAct: 0 none, 1 tanh-GELU, 2 SwiGLU (x rows are [gate | up], 2k wide).
// kPasses: 1024-column chunks per wave (wave w takes chunks w, w + waves, ...).
//
// Lane layout in a pass: lane l of the wave covers columns c0 + 16 l .. +15
// (c0 = chunk * 1024), i.e. group gi = l / (G/16) and, inside the group,
// element index 16 L + p with L = l % (G/16), p = d0 + 4 d1.  After the
// transpose a lane holds, for G = 256, p = L and t = d2 + 4 d3 = 0..15; for
// G = 128, p = 2L and 2L + 1 (z[t] and z[8 + t]) with t = d2 + 4 d3 = 0..7.
// rows_per_block: rows per workgroup, in order (> 1 only for the bf16 GELU
// by table, whose table build is then shared by that many rows).
// kGeluTable: bf16 GELU by the LDS table, for rows of up to
// kTableThreads / 64 waves; its launch bound leaves the kernel twice the
// registers (the 1024-thread bound capped it at 128 VGPRs, and it spilled).
template <int G, int kAct, int kPasses, bool kF16, bool kGeluTable = false>
__global__ __launch_bounds__(kGeluTable ? kTableThreads : 1024) void convrot_quant_i8_kernel(
    const uint16_t *__restrict__ x, int8_t *__restrict__ q, float *__restrict__ scales, int k, int staged_scale,
    int64_t rows, int rows_per_block) {
    static_assert(!kGeluTable || (kAct == 1 && !kF16), "the GELU table is for bf16 GELU input");
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float wave_amax[kMaxWaves];
    __shared__ uint16_t gelu_lut[kGeluTable ? kGeluLut : 1];
    constexpr int kLanesPerGroup = G / 16;
    // Transpose scratch: group gi starts at dword gi * kGroupDwords (padded so
    // the groups of a wave fall on different banks); element p of source lane
    // L sits at 16 L + 4 ((p / 4 + L / 4) % 4) + p % 4 (16-byte chunks rotated
    // by L / 4, so the 16-byte writes of lanes L and L + 4 hit different banks).
    constexpr int kGroupDwords = group_dwords<G>();
    constexpr int kCodeGroupBytes = code_group_bytes<G>();  // code scratch, padded likewise

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int waves = blockDim.x >> 6;
    const int gi = lane / kLanesPerGroup;
    const int L = lane % kLanesPerGroup;
    float *scr = reinterpret_cast<float *>(smem + wave * kScratchBytes);
    unsigned char *scr8 = smem + wave * kScratchBytes;
    float *grp = scr + gi * kGroupDwords;
    const int nchunks = (k + kChunk - 1) / kChunk;
    const int64_t in_stride = kAct == 2 ? 2 * static_cast<int64_t>(k) : k;

    if constexpr (kGeluTable) {
        for (int i = tid; i < kGeluLut; i += blockDim.x) gelu_lut[i] = static_cast<uint16_t>(gelu_lut_entry(i));
        __syncthreads();
    }
    // one row per workgroup unless the GELU table is shared by several
    const int64_t row0 = kGeluTable ? static_cast<int64_t>(blockIdx.x) * rows_per_block : blockIdx.x;
    const int64_t row_end = kGeluTable ? min(rows, row0 + rows_per_block) : row0 + 1;
    for (int64_t row = row0; row < row_end; ++row) {
        const uint16_t *xrow = x + row * in_stride;
        LaneInput<kAct> in[kPasses];
#pragma unroll
        for (int pass = 0; pass < kPasses; ++pass)
            if (wave + pass * waves < nchunks) load_lane<kAct>(in[pass], xrow, k, (wave + pass * waves) * kChunk + 16 * lane);
        float absmax = 0.0f;
        uint32_t packed[kPasses][8];
#pragma unroll
        for (int pass = 0; pass < kPasses; ++pass) {
            const int chunk = wave + pass * waves;
            if (chunk >= nchunks) break;  // uniform across the wave
            const bool active = chunk * kChunk + 16 * lane < k;  // whole groups are in or out (k % G == 0)
            float v[16];
            if constexpr (kGeluTable) {
                uint32_t unusual = 0, rel[8], table[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t w = in[pass].x[j / 4][j % 4];
                    unusual |= gelu_pair_unusual(w);
                    rel[j] = gelu_pair_rel(w);
                    table[j] = gelu_pair_lookup(w, rel[j], gelu_lut);
                }
                // The short select unless some active lane of the wave holds a
                // zero, subnormal, smallest-binade, inf or NaN input in this
                // pass (lanes past the row end hold zeros, never used).
                const bool usual = __builtin_amdgcn_ballot_w64(active && (unusual & 0x80008000u) != 0) == 0;
                uint32_t nonfinite = 0;
                if (__builtin_expect(usual, 1)) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t g = gelu_pair_fast(in[pass].x[j / 4][j % 4], rel[j], table[j]);
                        v[2 * j] = __uint_as_float(g << 16);
                        v[2 * j + 1] = __uint_as_float(g & 0xffff0000u);
                    }
                } else {
                    // A half with bit 15 of (mag + 0x80) set is inf or NaN (no
                    // carry crosses halves); such lanes recompute with activate.
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t w = in[pass].x[j / 4][j % 4];
                        nonfinite |= (w & 0x7fff7fffu) + 0x00800080u;
                        const uint32_t g = gelu_pair_select(w, rel[j], table[j]);
                        v[2 * j] = __uint_as_float(g << 16);
                        v[2 * j + 1] = __uint_as_float(g & 0xffff0000u);
                    }
                }
                if (__builtin_expect(__builtin_amdgcn_ballot_w64((nonfinite & 0x80008000u) != 0) != 0, 0)) {
                    if (nonfinite & 0x80008000u) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const uint32_t w = in[pass].x[j / 4][j % 4];
                            v[2 * j] = activate<false>(bf16_bits_to_f32(w & 0xffffu), 0.0f,
                                                       std::integral_constant<int, 1>{});
                            v[2 * j + 1] = activate<false>(__uint_as_float(w & 0xffff0000u), 0.0f,
                                                           std::integral_constant<int, 1>{});
                        }
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t w = in[pass].x[j / 4][j % 4];
                    const uint32_t u = kAct == 2 ? in[pass].up[(j / 4) % (kAct == 2 ? 2 : 1)][j % 4] : 0u;
                    v[2 * j] = activate<kF16>(elem_to_f32<kF16>(w), elem_to_f32<kF16>(u),
                                              std::integral_constant<int, kAct>{});
                    v[2 * j + 1] = activate<kF16>(elem_to_f32<kF16>(w >> 16), elem_to_f32<kF16>(u >> 16),
                                                  std::integral_constant<int, kAct>{});
                }
            }
            float z[16];
            rotate_pass<G>(v, grp, L, z);
            if (active) {
#pragma unroll
                for (int t = 0; t < 16; ++t) absmax = fmaxf(absmax, fabsf(z[t]));
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // G = 256: t = 2j, 2j + 1 of p = L.  G = 128: p = 2L (low), 2L + 1 (high) of t = j.
                const float lo = G == 256 ? z[2 * j] : z[j];
                const float hi = G == 256 ? z[2 * j + 1] : z[8 + j];
                if constexpr (kF16) packed[pass][j] = elem_bits<kF16>(lo) | (elem_bits<kF16>(hi) << 16);
                else packed[pass][j] = hw_bf16x2_bits(lo, hi);
            }
        }

        absmax = wave_max(absmax);
        if (lane == 0) wave_amax[wave] = absmax;
        __syncthreads();
        float amax = wave_amax[0];
        for (int w = 1; w < waves; ++w) amax = fmaxf(amax, wave_amax[w]);
        const float clipped = fminf(amax, kF16 ? 65504.0f : 3.38953139e38f);
        const float scale = fmaxf(staged_scale ? clipped * (1.0f / 127.0f) : clipped / 127.0f, 1.0e-30f);
        if (tid == 0) scales[row] = scale;
        const float rs = kF16 ? hw_f16_round(scale) : bf16_round(scale);
        const float ry = 1.0f / rs;

        int8_t *qrow = q + row * static_cast<int64_t>(k);
#pragma unroll
        for (int pass = 0; pass < kPasses; ++pass) {
            const int chunk = wave + pass * waves;
            if (chunk >= nchunks) break;
            const int col = chunk * kChunk + 16 * lane;
            const u32x4 codes = pass_codes<G, kF16>(packed[pass], rs, ry, scr8 + gi * kCodeGroupBytes, L);
            if (col < k) *reinterpret_cast<u32x4 *>(qrow + col) = codes;
        }
        // the next row rewrites wave_amax: every wave has read this row's first
        if (row + 1 < row_end) __syncthreads();
    }
}


// f(integral_constant<int, J>{}) for J = I, I + 1, .., N - 1, in order.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// ---------------------------------------------------------------------------
// LayerNorm fused with the G = 128 quantizer, bf16 rows of hidden = 256 per
// columns (per <= kPer).  The codes and scales are those of the bf16
// LayerNorm (AdaLN modulation, or the affine weight and bias) followed by the
// row-buffer quantizer above on its bf16 output; the normalized row never
// leaves the chip.
//
// Workgroup = 256 threads = 8 rows, one per 32-lane half-wave, as the 16-bit
// LayerNorm kernel: ln16_row_stats, then ln16_emit8 per column block (lane p
// holds columns 256 i + 8 p .. + 7 of block i).  A pass takes two blocks
// (512 columns): their outputs go through the wave's scratch so that lane p
// holds columns 512 P + 16 p .. + 15, the quantizer's layout (group
// 4 P + p / 8, lane L = p % 8 of it), and rotate_pass / pass_codes run as in
// the quantizer with the wave's 8 groups taken from its two rows.  The
// rotated values stay in registers as bf16 pairs until the row's absmax
// (a half-wave reduction) is known.
// LDS (6 B per column + kScratchBytes per wave: three workgroups per CU at
// hidden 5120): the modulation row of the workgroup's first row, m as fp32
// and the shift as bf16, then the waves' scratch.
// ---------------------------------------------------------------------------
template <int kPer, bool kAffine>
__global__ __launch_bounds__(kLnThreads) void ln_convrot_quant_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ scale, const uint16_t *__restrict__ shift,
    int8_t *__restrict__ q, float *__restrict__ scales, int64_t rows, int64_t len, int hidden, int per, int64_t steps,
    float eps, Recips rc) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int kPasses = kPer / 2;
    float *mod = reinterpret_cast<float *>(smem);
    uint16_t *mod_h16 = reinterpret_cast<uint16_t *>(smem + 4 * static_cast<size_t>(hidden));
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int p = tid & 31;  // lane of the half-wave
    const int wave = tid >> 6;
    const int gi = lane >> 3, L = lane & 7;
    unsigned char *scr8 = smem + 6 * static_cast<size_t>(hidden) + wave * kScratchBytes;
    float *grp = reinterpret_cast<float *>(scr8) + gi * group_dwords<128>();
    unsigned char *relay = scr8 + 32 * (lane & 32);  // 1 KiB per half-wave

    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * (kLnThreads / 32);
    const int64_t row_raw = row0 + (tid >> 5);
    // a half-wave past the last row computes the last row again and stores nothing
    const int64_t row = min(row_raw, rows - 1);
    const bool live = row_raw < rows;
    const int64_t mrow = modulation_row(row, len, steps);
    const int64_t mrow0 = modulation_row(row0, len, steps);
    const bool staged = mrow == mrow0;
    const uint16_t *xr = x + row * hidden + 8 * p;
    const uint16_t *sc = scale + mrow * hidden + 8 * p;
    const uint16_t *sh = shift + mrow * hidden + 8 * p;

    u32x4 xs[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (i < per) xs[i] = *reinterpret_cast<const u32x4 *>(xr + 256 * i);

    // the workgroup's first row's modulation row: m = T(1 + scale) (or the
    // weight) as fp32, the shift (or bias) as its bf16 bits
    for (int c = 8 * tid; c < hidden; c += 8 * kLnThreads) {
        const u32x4 sv = *reinterpret_cast<const u32x4 *>(scale + mrow0 * hidden + c);
        f32x4 m0, m1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float sf = unpack16<0>(sv, e);
            const float m = kAffine ? sf : t_round<0>(1.0f + sf);
            if (e < 4) m0[e] = m; else m1[e - 4] = m;
        }
        *reinterpret_cast<f32x4 *>(mod + c) = m0;
        *reinterpret_cast<f32x4 *>(mod + c + 4) = m1;
        *reinterpret_cast<u32x4 *>(mod_h16 + c) = *reinterpret_cast<const u32x4 *>(shift + mrow0 * hidden + c);
    }
    __syncthreads();

    float mu, inv;
    ln16_row_stats<0, kPer>(xs, per, hidden, eps, rc, (tid & 32) << 2, mu, inv);

    // The rotated values of pass P replace its two input blocks in xs (as bf16
    // pairs in z order: packed word j = (z[j], z[8 + j]) in xs[2P + j / 4]),
    // which keeps the row's registers at one copy.  kPer is even, so
    // xs[2P + 1] exists whenever 2P < per.
    static_assert(kPer % 2 == 0, "passes take two column blocks");
    float absmax = 0.0f;
    // passes as a compile-time sequence, so that xs[] is never indexed at run
    // time (a loop this long is not unrolled); per is uniform
    static_for<0, kPasses>([&](auto pass_c) {
        constexpr int pass = decltype(pass_c)::value;
        if (2 * pass >= per) return;
        u32x4 o[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int i = 2 * pass + b;
            o[b] = u32x4{0u, 0u, 0u, 0u};
            if (i < per) {
                float mv[8], hv[8];
                if (staged) {
                    const float *mod_m = mod + 256 * i + 8 * p;
                    const f32x4 m0 = *reinterpret_cast<const f32x4 *>(mod_m);
                    const f32x4 m1 = *reinterpret_cast<const f32x4 *>(mod_m + 4);
                    const u32x4 hw = *reinterpret_cast<const u32x4 *>(mod_h16 + 256 * i + 8 * p);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        mv[e] = m0[e]; mv[e + 4] = m1[e];
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) hv[e] = unpack16<0>(hw, e);
                } else {
                    const u32x4 sv = *reinterpret_cast<const u32x4 *>(sc + 256 * i);
                    const u32x4 shv = *reinterpret_cast<const u32x4 *>(sh + 256 * i);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float sf = unpack16<0>(sv, e);
                        mv[e] = kAffine ? sf : t_round<0>(1.0f + sf);
                        hv[e] = unpack16<0>(shv, e);
                    }
                }
                // the block's words made opaque, so that the statistics'
                // unpacked fp32 copies of them need not stay live until here
                uint32_t w0 = xs[i][0], w1 = xs[i][1], w2 = xs[i][2], w3 = xs[i][3];
                asm("" : "+v"(w0), "+v"(w1), "+v"(w2), "+v"(w3));
                o[b] = ln16_emit8<0, kAffine>(u32x4{w0, w1, w2, w3}, mv, hv, mu, inv);
            }
        }
        // blocks 2 pass and 2 pass + 1 in column order, read back 16 columns a lane
        lds_wave_sync();  // earlier reads of the scratch are done
        *reinterpret_cast<u32x4 *>(relay + 16 * p) = o[0];
        *reinterpret_cast<u32x4 *>(relay + 512 + 16 * p) = o[1];
        lds_wave_sync();
        const u32x4 y0 = *reinterpret_cast<const u32x4 *>(relay + 32 * p);
        const u32x4 y1 = *reinterpret_cast<const u32x4 *>(relay + 32 * p + 16);
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = bf16_bits_to_f32(y0[j] & 0xffffu);
            v[2 * j + 1] = __uint_as_float(y0[j] & 0xffff0000u);
            v[8 + 2 * j] = bf16_bits_to_f32(y1[j] & 0xffffu);
            v[8 + 2 * j + 1] = __uint_as_float(y1[j] & 0xffff0000u);
        }
        float z[16];
        rotate_pass<128>(v, grp, L, z);
        if (512 * pass + 16 * p < hidden) {
#pragma unroll
            for (int t = 0; t < 16; ++t) absmax = fmaxf(absmax, fabsf(z[t]));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[2 * pass + j / 4][j % 4] = hw_bf16x2_bits(z[j], z[8 + j]);
    });

    // the row's absmax over its half-wave
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) absmax = fmaxf(absmax, __shfl_xor(absmax, off, 64));
    const float clipped = fminf(absmax, 3.38953139e38f);
    const float row_scale = fmaxf(clipped / 127.0f, 1.0e-30f);
    if (p == 0 && live) scales[row] = row_scale;
    const float rs = bf16_round(row_scale);
    const float ry = 1.0f / rs;

    int8_t *qrow = q + row * static_cast<int64_t>(hidden);
    static_for<0, kPasses>([&](auto pass_c) {
        constexpr int pass = decltype(pass_c)::value;
        if (2 * pass >= per) return;
        const uint32_t packed[8] = {xs[2 * pass][0], xs[2 * pass][1], xs[2 * pass][2], xs[2 * pass][3],
                                    xs[2 * pass + 1][0], xs[2 * pass + 1][1], xs[2 * pass + 1][2], xs[2 * pass + 1][3]};
        const u32x4 codes = pass_codes<128, false>(packed, rs, ry, scr8 + gi * code_group_bytes<128>(), L);
        const int col = 512 * pass + 16 * p;
        if (live && col < hidden) *reinterpret_cast<u32x4 *>(qrow + col) = codes;
    });
}

// hidden = 256 per, per <= 20 (register-resident rows and rotated values).
constexpr int kLnQuantMaxPer = 20;

template <bool kAffine>
void launch_ln_quant(const void *x, const void *sc, const void *sh, int8_t *q, float *scales, int64_t rows,
                     int64_t len, int hidden, int64_t steps, float eps, hipStream_t s) {
    const int per = hidden / kLnThreads;
    const Recips rc = uniform_recips(per);
    const dim3 grid(static_cast<unsigned>((rows + kLnThreads / 32 - 1) / (kLnThreads / 32)));
    const size_t lds = 6 * static_cast<size_t>(hidden) + (kLnThreads / 64) * kScratchBytes;
    const auto *x16 = static_cast<const uint16_t *>(x), *sc16 = static_cast<const uint16_t *>(sc),
               *sh16 = static_cast<const uint16_t *>(sh);
#define TU_LNQ(P) \
    ln_convrot_quant_kernel<P, kAffine><<<grid, kLnThreads, lds, s>>>(x16, sc16, sh16, q, scales, rows, len, hidden, \
                                                                      per, steps, eps, rc)
    if (per <= 4) TU_LNQ(4);
    else if (per <= 8) TU_LNQ(8);
    else if (per <= 12) TU_LNQ(12);
    else if (per <= 16) TU_LNQ(16);
    else TU_LNQ(20);
#undef TU_LNQ
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_convrot_quant_i8(const void *x_bf16, int8_t *q, float *scale, int64_t rows,
                                       int64_t cols, int32_t group, int32_t act, void *stream) {
    using namespace tu;
    TU_REQUIRE(group == 128 || group == 256, "ConvRot group_size must be 128 or 256, got %d", group);
    const int staged_scale = (act & TU_CONVROT_STAGED_SCALE) != 0;
    const bool f16 = (act & TU_CONVROT_FP16_INPUT) != 0;
    act &= ~(TU_CONVROT_STAGED_SCALE | TU_CONVROT_FP16_INPUT);
    TU_REQUIRE(act >= TU_ACT_NONE && act <= TU_ACT_SWIGLU,
               "ConvRot input activation must be 0 (none), 1 (tanh-GELU) or 2 (SwiGLU), got %d", act);
    TU_REQUIRE(rows >= 0 && cols > 0 && cols % group == 0,
               "ConvRot width must be positive and divisible by %d, got %lld", group,
               static_cast<long long>(cols));
    TU_REQUIRE(rows <= 0x7fffffff && cols <= (1 << 20), "ConvRot dimensions out of range");
    TU_REQUIRE(x_bf16 && q && scale, "ConvRot pointers must be non-null");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(x_bf16) & 15) == 0 && (reinterpret_cast<uintptr_t>(q) & 15) == 0,
               "ConvRot input and codes must be 16-byte aligned");
    if (require_gfx950()) return -1;
    if (rows == 0) return 0;
    const int k = static_cast<int>(cols);
    TU_REQUIRE(k <= kMaxCols, "ConvRot row of %d columns exceeds the %d-column limit", k, kMaxCols);
    // Few waves per row, each carrying up to kMaxPasses chunks: measured
    // faster than one chunk per wave (shorter barrier, more rows per CU).
    const int nchunks = (k + kChunk - 1) / kChunk;
    const int passes = nchunks < kMaxPasses ? nchunks : kMaxPasses;
    const int waves = (nchunks + passes - 1) / passes;
    const size_t lds = static_cast<size_t>(waves) * kScratchBytes;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const auto *xp = static_cast<const uint16_t *>(x_bf16);
    // The bf16 GELU of rows up to 8 waves builds a 7.5 KiB table per
    // workgroup, which 8 rows share; wider rows compute every GELU.
    const bool table = act == TU_ACT_GELU_TANH && !f16 && waves * 64 <= kTableThreads;
    const int rpb = table ? 8 : 1;
    const dim3 grid(static_cast<unsigned>((rows + rpb - 1) / rpb));
#define TU_CONVROT_LAUNCH_T(G, A, F, T)                                                                          \
    do {                                                                                                         \
        switch (passes) {                                                                                        \
            case 1: convrot_quant_i8_kernel<G, A, 1, F, T><<<grid, waves * 64, lds, s>>>(xp, q, scale, k, staged_scale, rows, rpb); break; \
            case 2: convrot_quant_i8_kernel<G, A, 2, F, T><<<grid, waves * 64, lds, s>>>(xp, q, scale, k, staged_scale, rows, rpb); break; \
            case 3: convrot_quant_i8_kernel<G, A, 3, F, T><<<grid, waves * 64, lds, s>>>(xp, q, scale, k, staged_scale, rows, rpb); break; \
            default: convrot_quant_i8_kernel<G, A, 4, F, T><<<grid, waves * 64, lds, s>>>(xp, q, scale, k, staged_scale, rows, rpb); break; \
        }                                                                                                        \
    } while (0)
#define TU_CONVROT_LAUNCH(G, A)                                         \
    do {                                                                \
        if (f16) TU_CONVROT_LAUNCH_T(G, A, true, false);                \
        else if (table) TU_CONVROT_LAUNCH_T(G, A, false, (A == 1));     \
        else TU_CONVROT_LAUNCH_T(G, A, false, false);                   \
    } while (0)
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
#undef TU_CONVROT_LAUNCH_T
    return check_launch("tu_convrot_quant_i8");
}

namespace {
int32_t check_ln_quant(const void *x, const void *sc, const void *sh, const int8_t *q, const float *scales,
                       int64_t rows, int64_t hidden, float eps, const char *what) {
    TU_REQUIRE(rows >= 0 && rows <= 0x7fffffff, "%s rows must be in [0, 2^31)", what);
    TU_REQUIRE(hidden > 0 && hidden % tu::kLnThreads == 0 && hidden <= tu::kLnThreads * tu::kLnQuantMaxPer,
               "%s hidden must be a multiple of %d in [%d, %d], got %lld", what, tu::kLnThreads, tu::kLnThreads,
               tu::kLnThreads * tu::kLnQuantMaxPer, static_cast<long long>(hidden));
    TU_REQUIRE(eps > 0.0f && eps <= 3.4e38f, "%s epsilon must be finite and positive", what);
    TU_REQUIRE(x && sc && sh && q && scales, "%s pointers must be non-null", what);
    TU_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(sc) | reinterpret_cast<uintptr_t>(sh) |
                 reinterpret_cast<uintptr_t>(q)) & 15) == 0,
               "%s input, modulation and codes must be 16-byte aligned", what);
    return 0;
}
}  // namespace

extern "C" int32_t tu_layer_norm_adaln_convrot_quant_i8(const void *x, const void *scale, const void *shift,
                                                        int8_t *q, float *row_scale, int64_t batch, int64_t len,
                                                        int64_t hidden, int64_t steps, float eps, void *stream) {
    using namespace tu;
    TU_REQUIRE(batch > 0 && len > 0 && steps > 0 && steps <= 0x7fffffff,
               "LayerNorm+AdaLN ConvRot dimensions must be positive");
    TU_REQUIRE(batch <= 0x7fffffff / len, "LayerNorm+AdaLN ConvRot rows exceed the kernel range");
    if (check_ln_quant(x, scale, shift, q, row_scale, batch * len, hidden, eps, "LayerNorm+AdaLN ConvRot")) return -1;
    if (require_gfx950()) return -1;
    launch_ln_quant<false>(x, scale, shift, q, row_scale, batch * len, len, static_cast<int>(hidden), steps, eps,
                           static_cast<hipStream_t>(stream));
    return check_launch("tu_layer_norm_adaln_convrot_quant_i8");
}

extern "C" int32_t tu_layer_norm_affine_convrot_quant_i8(const void *x, const void *weight, const void *bias,
                                                         int8_t *q, float *row_scale, int64_t rows, int64_t hidden,
                                                         float eps, void *stream) {
    using namespace tu;
    if (check_ln_quant(x, weight, bias, q, row_scale, rows, hidden, eps, "LayerNorm ConvRot")) return -1;
    if (require_gfx950()) return -1;
    if (rows == 0) return 0;
    // one batch of `rows` tokens and a single "modulation" row: weight / bias
    launch_ln_quant<true>(x, weight, bias, q, row_scale, rows, rows, static_cast<int>(hidden), 1, eps,
                          static_cast<hipStream_t>(stream));
    return check_launch("tu_layer_norm_affine_convrot_quant_i8");
}
