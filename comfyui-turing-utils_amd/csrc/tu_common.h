// Shared device/host helpers for the gfx950 kernels of libtu_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/tu_hip.h"

namespace tu {

// ---------------------------------------------------------------------------
// Host-side error reporting: every C entry point returns 0 or sets a message
// retrievable through tu_last_error() on the calling thread.
// ---------------------------------------------------------------------------
void set_error(const std::string &msg);
int32_t fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
int32_t check_launch(const char *what);
// Returns 0 if the current device is gfx950, otherwise sets an error.
int32_t require_gfx950();
// Compute units of the current device (cached per device id); 0 or an error.
int32_t device_cus(int &cus);

#define TU_REQUIRE(cond, ...)          \
    do {                               \
        if (!(cond)) return tu::fail(__VA_ARGS__); \
    } while (0)

// ---------------------------------------------------------------------------
// Vector types for MFMA operands.
// ---------------------------------------------------------------------------
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// bf16 <-> fp32.  Round-to-nearest-even with a canonical NaN (0x7fff), the
// conversion of kernel/csrc/turing/convrot_quant.cu:293-305.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t bf16_rne_bits(float v) {
    const uint32_t bits = __float_as_uint(v);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return 0x7fffu;
    // bits + 0x7fff + lsb, then truncate: RNE for finite values (no overflow
    // past inf: the largest finite fp32 rounds to bf16 inf as RNE requires).
    const uint32_t lsb = (bits >> 16) & 1u;
    return (bits + 0x7fffu + lsb) >> 16;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_f32(bf16_rne_bits(v)); }

// Packs two floats to two bf16 (low = a) with the same rounding.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return bf16_rne_bits(a) | (bf16_rne_bits(b) << 16);
}

// Two floats to two bf16 (low = a) by one v_cvt_pk_bf16_f32: RNE, equal to
// pack_bf16x2 for every non-NaN input; a NaN keeps an unspecified NaN
// payload instead of 0x7fff.
__device__ __forceinline__ uint32_t hw_bf16x2_bits(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), bf16x2_t));
}

// fp16 <-> fp32.  Two floats to two fp16 (low = a) by the hardware
// conversion: round-to-nearest-even, overflow to +-inf, fp16 subnormals kept;
// a NaN keeps an unspecified NaN payload.
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t hw_f16x2_bits(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{a, b}), f16x2_t));
}
// The same with every NaN written as 0x7e00 (quiet, positive).
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    uint32_t r = hw_f16x2_bits(a, b);
    if (a != a) r = (r & 0xffff0000u) | 0x7e00u;
    if (b != b) r = (r & 0x0000ffffu) | 0x7e000000u;
    return r;
}

// s_waitcnt immediate that waits until at most n vector-memory operations are
// outstanding and leaves the other counters alone (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_imm(int n) { return (n & 0xf) | (0x7 << 4) | (0xf << 8) | ((n >> 4) << 14); }
// s_waitcnt immediate: at most n LDS/scalar-memory operations outstanding.
constexpr int lgkmcnt_imm(int n) { return 0xf | (0x7 << 4) | ((n & 0xf) << 8) | (0x3 << 14); }

// Buffer resource over [base, base + bytes): raw (stride 0) dword access;
// reads at or past `bytes` return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), static_cast<int>(bytes),
                                             0x00020000);
}

}  // namespace tu
