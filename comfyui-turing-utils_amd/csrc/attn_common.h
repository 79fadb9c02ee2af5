// Device helpers shared by the two gfx950 attention kernels (Sage bf16-PV
// and dense W8A8): cross-lane row reductions, the workgroup barrier
// of the two-group schedule and the biased-accumulator constants.
#pragma once

#include "tu_common.h"

namespace tu {

typedef __attribute__((address_space(3))) void lds_void;

constexpr float kLog2e = 1.4426950408889634f;

// Row maxima / sums across the 4 lane groups (xor 16, xor 32) with the
// gfx950 permlane swaps: VALU only, no LDS traffic.
__device__ __forceinline__ int xmax_i32(int v) {
    auto a = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
    v = max(static_cast<int>(a[0]), static_cast<int>(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v), false, false);
    return max(static_cast<int>(b[0]), static_cast<int>(b[1]));
}
__device__ __forceinline__ float xmax_f32(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xsum_f32(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ int imax3(int a, int b, int c) { return max(max(a, b), c); }

// The QK^T accumulators start at kBias, the bit pattern of 1.5 * 2^23, so
// each int32 result is the float 1.5 * 2^23 + dot exactly (|dot| <= 2^21 for
// D = 128 int8 codes): float(dot) is then one exact subtraction instead of a
// conversion, and integer comparisons of the biased values still order the
// dots.
constexpr int kBias = 0x4B400000;
constexpr float kBiasF = 12582912.0f;

// Workgroup barrier that does not wait for memory (the LDS ring hand-off is
// ordered by an explicit s_waitcnt vmcnt before it) and that no instruction
// is scheduled across: the two groups' MFMA and softmax clusters must keep
// their places relative to the barrier.
__device__ __forceinline__ void wg_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

}  // namespace tu
