// Device pieces of the W8A8 Q/K transform shared by the standalone W8A8
// quantizer (w8a8_quant.hip) and the fused RMSNorm + RoPE producer
// (qk_preprocess.hip): the sign-diagonal Walsh-Hadamard rotation of one
// 8-channel pack across a token's lanes, the K-anchor decision, and the
// cross-lane helpers they use (DPP lane exchanges, wave maxima).
#pragma once

#include "attn_common.h"

namespace tu {

// Sign words of the shared Q/K transform (kernel/csrc/turing/sage/
// fused.cu:206-212): channel c is negated when bit (c & 31) of word c >> 5 is 0.
__device__ __forceinline__ bool w8a8_sign_negative(int c) {
    constexpr uint32_t kSigns[4] = {0x1035997bu, 0x8087f5eeu, 0xee2e4e1au, 0x71132418u};
    return ((kSigns[c >> 5] >> (c & 31)) & 1u) == 0u;
}

// Maximum over the wave of non-negative floats that are not NaN, compared as
// integers (their bit patterns order as the values do): DPP within rows of
// 16, then the permlane swaps across rows.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    int b = __float_as_int(v);
    b = max(b, __builtin_amdgcn_mov_dpp(b, 0x128, 0xf, 0xf, false));   // row_ror:8
    b = max(b, __builtin_amdgcn_mov_dpp(b, 0x124, 0xf, 0xf, false));   // row_ror:4
    b = max(b, __builtin_amdgcn_mov_dpp(b, 0x4E, 0xf, 0xf, false));
    b = max(b, __builtin_amdgcn_mov_dpp(b, 0xB1, 0xf, 0xf, false));
    return __int_as_float(xmax_i32(b));
}

// v of lane i ^ kBit (kBit < 16) with no index arithmetic: DPP quad
// permutations for 1 and 2; for 4 the mirror of each 8-lane half (lane
// 7 - i) and then the reversal of each quad, which together give i ^ 4; for
// 8 the rotation of each 16-lane row by 8 ((i + 8) mod 16 = i ^ 8).
template <int kBit>
__device__ __forceinline__ float w8a8_lane_xor(float v) {
    int x = __float_as_int(v);
    if constexpr (kBit == 1) {
        x = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xf, 0xf, true);
    } else if constexpr (kBit == 2) {
        x = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xf, 0xf, true);
    } else if constexpr (kBit == 4) {
        x = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xf, 0xf, true);   // row_half_mirror
        x = __builtin_amdgcn_update_dpp(0, x, 0x1B, 0xf, 0xf, true);    // quad (3, 2, 1, 0)
    } else {
        static_assert(kBit == 8, "lane xor of 1, 2, 4 or 8");
        x = __builtin_amdgcn_update_dpp(0, x, 0x128, 0xf, 0xf, true);   // row_ror:8
    }
    return __int_as_float(x);
}

// One cross-pack butterfly stage: v = other - v on lanes with bit `kBit` of
// the pack index set, v + other elsewhere, as other + (+-1 * v): IEEE
// subtraction is addition of the negation, and addition commutes, so the
// bits are those of the two-sided form.
template <int kBit>
__device__ __forceinline__ void w8a8_cross_stage(float (&v)[8], int p) {
    float sgn = (p & kBit) ? -1.0f : 1.0f;
    // opaque to the compiler, which would otherwise form both sums and select
    asm("" : "+v"(sgn));
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = w8a8_lane_xor<kBit>(v[j]) + sgn * v[j];
}

// The transform of one pack (8 channels of pack index p) across the lanes of
// a token (attention_hadamard8, fused.cu:214-260): signs, the in-pack
// butterfly with spans 1, 2, 4, the cross-pack butterfly over lane bits (the
// D / 8 packs of a token are consecutive lanes), the 1/sqrt(D) factor.
// Every lane of the token's group must execute it.
template <int D>
__device__ __forceinline__ void w8a8_hadamard_pack(float (&v)[8], int p) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
        if (w8a8_sign_negative(8 * p + j)) v[j] = -v[j];
#pragma unroll
    for (int span = 1; span < 8; span <<= 1)
#pragma unroll
        for (int base = 0; base < 8; base += 2 * span)
#pragma unroll
            for (int o = 0; o < span; ++o) {
                const float l = v[base + o], r = v[base + o + span];
                v[base + o] = l + r;
                v[base + o + span] = l - r;
            }
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    w8a8_cross_stage<1>(v, p);
    w8a8_cross_stage<2>(v, p);
    w8a8_cross_stage<4>(v, p);
    if constexpr (D == 128) w8a8_cross_stage<8>(v, p);
    constexpr float kNorm = D == 64 ? 0.125f : 0.08838834764831845f;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= kNorm;
}

// Lane 0 / lane 32 of a wave64 end with the sum (max) of their 32-lane half,
// formed in the order of a shfl_down tree (offsets 16 .. 1): the xor partner
// of every lane below the offset is the lane the down-shift would read.
__device__ __forceinline__ float w8a8_tree32_sum(float v) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) v = v + __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float w8a8_tree32_max(float v) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

constexpr int kAnchorThreads = 128;
constexpr int kAnchorSamples = 9;

// The K-anchor decision of a 128-thread workgroup over nine sample rows in
// LDS (samples[s][c], channels >= dim zero), in the reference's order
// (fused.cu:447-575, qk_preprocess.cu:302-414): one channel per thread,
// E = fma chain of x^2, M = max |x|, S = sequential sum, per candidate
// dist = fma(9 x_j - S, 9 x_j - S, 0); 32-lane trees; the four tree results
// added from 0 in order.  Returns (to every thread) the selected sample
// 0..8 when centring on it lowers E without growing M by more than 12.5 %,
// else -1.
__device__ __forceinline__ int w8a8_anchor_decide(const float (*samples)[128], int dim) {
    __shared__ float tree_e[4], tree_m[4], tree_d[kAnchorSamples][4], tree_be[4], tree_bm[4];
    __shared__ int selected;
    const int c = threadIdx.x;
    const int lane = c & 31, tree = c >> 5;
    float e = 0.0f, m = 0.0f, sum = 0.0f, dist[kAnchorSamples];
#pragma unroll
    for (int j = 0; j < kAnchorSamples; ++j) dist[j] = 0.0f;
    if (c < dim) {
#pragma unroll
        for (int s = 0; s < kAnchorSamples; ++s) {
            const float v = samples[s][c];
            e = __builtin_fmaf(v, v, e);
            m = fmaxf(m, fabsf(v));
            sum = sum + v;
        }
#pragma unroll
        for (int j = 0; j < kAnchorSamples; ++j) {
            const float d = 9.0f * samples[j][c] - sum;
            dist[j] = __builtin_fmaf(d, d, 0.0f);
        }
    }
    e = w8a8_tree32_sum(e);
    m = w8a8_tree32_max(m);
#pragma unroll
    for (int j = 0; j < kAnchorSamples; ++j) dist[j] = w8a8_tree32_sum(dist[j]);
    if (lane == 0) {
        tree_e[tree] = e;
        tree_m[tree] = m;
#pragma unroll
        for (int j = 0; j < kAnchorSamples; ++j) tree_d[j][tree] = dist[j];
    }
    __syncthreads();
    if (c == 0) {
        int best = 0;
        float best_d = 3.402823466e+38F;
        for (int j = 0; j < kAnchorSamples; ++j) {
            float d = 0.0f;
            for (int t = 0; t < 4; ++t) d = d + tree_d[j][t];
            if (d < best_d) {
                best = j;
                best_d = d;
            }
        }
        selected = best;
    }
    __syncthreads();
    const int best = selected;
    float be = 0.0f, bm = 0.0f;
    if (c < dim) {
        const float a = samples[best][c];
#pragma unroll
        for (int s = 0; s < kAnchorSamples; ++s) {
            const float r = samples[s][c] - a;
            be = __builtin_fmaf(r, r, be);
            bm = fmaxf(bm, fabsf(r));
        }
    }
    be = w8a8_tree32_sum(be);
    bm = w8a8_tree32_max(bm);
    if (lane == 0) {
        tree_be[tree] = be;
        tree_bm[tree] = bm;
    }
    __syncthreads();
    if (c == 0) {
        float te = 0.0f, tm = 0.0f, tbe = 0.0f, tbm = 0.0f;
        for (int t = 0; t < 4; ++t) {
            te = te + tree_e[t];
            tm = fmaxf(tm, tree_m[t]);
            tbe = tbe + tree_be[t];
            tbm = fmaxf(tbm, tree_bm[t]);
        }
        selected = (tbe < te && tbm <= tm * 1.125f) ? best : -1;
    }
    __syncthreads();
    return selected;
}

}  // namespace tu
