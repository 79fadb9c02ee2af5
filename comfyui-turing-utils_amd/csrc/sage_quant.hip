// Sage attention prologue for gfx950: K channel mean (smoothing) and
// per-block symmetric INT8 quantization of Q and K.
//
// Quantizer semantics: QuantInt8Kernel (kernel/csrc/turing/sage/fused.cu
// :66-200) with sub_mean (:97-128):
//   v = float(x) - float(mean[d]);  amax = max(1e-7, max|v| over the block)
//   scale = amax / 127;  q = cvt.rni.sat.s8(v * (127 / amax))
// The reference compiles this with --use_fast_math; here both divisions are
// IEEE, as in the CPU oracle.
//
// The K mean is not defined by the reference (its production Sage path has
// smoothing switched off, turing_sage/core.py:421).  This build defines it as
// bf16_rn(sum_t k[t][d] / L) with a fixed fp32 summation order, so that the
// oracle can restate it bit for bit:
//   chunk c = tokens [128c, 128c + 128); a 256-thread workgroup gives each
//   thread 8 channels of every rows-th token (rows = 256 / (D/8));
//   per-thread sums run over ascending tokens, the rows partial sums of a
//   chunk are added in ascending row order, and the chunk sums in ascending
//   chunk order by a second kernel.
#include <mutex>

#include "tu_common.h"

namespace tu {
namespace {

constexpr int kThreads = 256;

// Chunk-sum scratch of tu_sage_kmean_noalloc: a file-scope device array that
// every GPU running this library holds until the process ends.  In host code
// `scratch` names a host-side stand-in, not a device address; the device
// address comes from hipGetSymbolAddress, once per device (scratch_ptr).
constexpr int64_t kNoAllocScratchFloats = int64_t{1} << 22;  // 16 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

template <int D>
__global__ __launch_bounds__(kThreads) void kmean_chunk_kernel(const uint16_t *__restrict__ k, int64_t len,
                                                               int64_t s_b, int64_t s_h, int64_t s_l,
                                                               float *__restrict__ chunk_sums) {
    constexpr int kLanesPerRow = D / 8;
    constexpr int kRows = kThreads / kLanesPerRow;
    constexpr int kPer = 128 / kRows;
    __shared__ float partial[kRows][D];

    const int tid = threadIdx.x;
    const int r = tid / kLanesPerRow;
    const int c8 = tid % kLanesPerRow;
    const int64_t chunk = blockIdx.x;
    const int64_t h = blockIdx.y, b = blockIdx.z, heads = gridDim.y, chunks = gridDim.x;
    const uint16_t *base = k + b * s_b + h * s_h;

    float s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int64_t t = chunk * 128 + r + static_cast<int64_t>(kRows) * j;
        if (t < len) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(base + t * s_l + c8 * 8);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                s[2 * e] = s[2 * e] + bf16_bits_to_f32(v[e] & 0xffffu);
                s[2 * e + 1] = s[2 * e + 1] + bf16_bits_to_f32(v[e] >> 16);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) partial[r][c8 * 8 + e] = s[e];
    __syncthreads();
    if (tid < D) {
        float acc = 0.0f;
#pragma unroll 8
        for (int rr = 0; rr < kRows; ++rr) acc = acc + partial[rr][tid];
        chunk_sums[((b * heads + h) * chunks + chunk) * D + tid] = acc;
    }
}

// One thread per (batch*head, channel): sum of the chunk sums in ascending
// order, divided by len, rounded to bf16.
__global__ __launch_bounds__(128) void kmean_final_kernel(const float *__restrict__ chunk_sums, int64_t chunks,
                                                          int64_t len, int dim, uint16_t *__restrict__ mean) {
    const int d = threadIdx.x;
    if (d >= dim) return;
    const int64_t bh = blockIdx.x;
    const float *src = chunk_sums + bh * chunks * dim + d;
    // Loads are issued 16 at a time to hide their latency; the additions stay
    // in ascending chunk order.
    float tot = 0.0f;
    int64_t c = 0;
    for (; c + 16 <= chunks; c += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = src[(c + j) * dim];
#pragma unroll
        for (int j = 0; j < 16; ++j) tot = tot + v[j];
    }
    for (; c < chunks; ++c) tot = tot + src[c * dim];
    mean[bh * dim + d] = static_cast<uint16_t>(bf16_rne_bits(tot / static_cast<float>(len)));
}

__device__ __forceinline__ int32_t sat_rne_s8(float v) {
    if (v != v) return 0;
    const float r = fminf(127.0f, fmaxf(-128.0f, __builtin_rintf(v)));
    return static_cast<int32_t>(r);
}

// One workgroup per (token block, head, batch).  Each thread owns 8
// contiguous channels of every (256 / (D/8))-th token row of the block; the
// block is held in registers between the absmax and the quantization pass.
template <int D, int BLK, bool kSubMean>
__global__ __launch_bounds__(kThreads) void sage_quant_kernel(
    const uint16_t *__restrict__ x, const uint16_t *__restrict__ mean, int64_t len, int64_t s_b,
    int64_t s_h, int64_t s_l, int8_t *__restrict__ q, int64_t q_b, int64_t q_h, int64_t q_l,
    float *__restrict__ scale) {
    constexpr int kLanesPerRow = D / 8;
    constexpr int kRowsPerPass = kThreads / kLanesPerRow;
    constexpr int kPasses = (BLK + kRowsPerPass - 1) / kRowsPerPass;
    __shared__ float wave_amax[kThreads / 64];

    const int tid = threadIdx.x;
    const int r = tid / kLanesPerRow;
    const int c8 = tid % kLanesPerRow;
    const int64_t blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z, heads = gridDim.y, nblk = gridDim.x;
    const uint16_t *xb = x + b * s_b + h * s_h;
    int8_t *qb = q + b * q_b + h * q_h;

    float mu[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) mu[e] = 0.0f;
    if constexpr (kSubMean) {
        const u32x4 mv = *reinterpret_cast<const u32x4 *>(mean + (b * heads + h) * D + c8 * 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            mu[2 * e] = bf16_bits_to_f32(mv[e] & 0xffffu);
            mu[2 * e + 1] = bf16_bits_to_f32(mv[e] >> 16);
        }
    }

    float v[kPasses][8];
    float amax = 0.0000001f;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int row = r + p * kRowsPerPass;
        const int64_t t = blk * BLK + row;
        if (row < BLK && t < len) {
            const u32x4 xv = *reinterpret_cast<const u32x4 *>(xb + t * s_l + c8 * 8);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[p][2 * e] = bf16_bits_to_f32(xv[e] & 0xffffu);
                v[p][2 * e + 1] = bf16_bits_to_f32(xv[e] >> 16);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if constexpr (kSubMean) v[p][e] = v[p][e] - mu[e];
                amax = fmaxf(amax, fabsf(v[p][e]));
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[p][e] = 0.0f;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if ((tid & 63) == 0) wave_amax[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wave_amax[0], wave_amax[1]), fmaxf(wave_amax[2], wave_amax[3]));
    if (tid == 0) scale[(b * heads + h) * nblk + blk] = amax / 127.0f;
    const float mult = 127.0f / amax;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        const int row = r + p * kRowsPerPass;
        const int64_t t = blk * BLK + row;
        if (row < BLK && t < len) {
            u32x2 out;
            uint32_t w[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                uint32_t acc = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc |= (static_cast<uint32_t>(sat_rne_s8(v[p][4 * hh + e] * mult)) & 0xffu) << (8 * e);
                w[hh] = acc;
            }
            out.x = w[0];
            out.y = w[1];
            *reinterpret_cast<u32x2 *>(qb + t * q_l + c8 * 8) = out;
        }
    }
}

template <int D>
int32_t launch_quant(const uint16_t *x, const uint16_t *mean, int64_t batch, int64_t heads, int64_t len,
                     int64_t s_b, int64_t s_h, int64_t s_l, int64_t blk, int8_t *q, int64_t q_b, int64_t q_h,
                     int64_t q_l, float *scale, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((len + blk - 1) / blk), static_cast<unsigned>(heads),
                    static_cast<unsigned>(batch));
#define TU_QUANT_CASE(B)                                                                                \
    case B:                                                                                             \
        if (mean)                                                                                       \
            sage_quant_kernel<D, B, true><<<grid, kThreads, 0, s>>>(x, mean, len, s_b, s_h, s_l, q, q_b, \
                                                                    q_h, q_l, scale);                   \
        else                                                                                            \
            sage_quant_kernel<D, B, false><<<grid, kThreads, 0, s>>>(x, mean, len, s_b, s_h, s_l, q,     \
                                                                     q_b, q_h, q_l, scale);             \
        break;
    switch (blk) {
        TU_QUANT_CASE(16)
        TU_QUANT_CASE(32)
        TU_QUANT_CASE(64)
        TU_QUANT_CASE(128)
        default:
            return fail("Sage quantization block must be 16, 32, 64 or 128, got %lld", static_cast<long long>(blk));
    }
#undef TU_QUANT_CASE
    return check_launch("tu_sage_quant");
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_sage_kmean(const void *k_bf16, int64_t batch, int64_t heads, int64_t len, int64_t dim,
                                 int64_t s_b, int64_t s_h, int64_t s_l, float *chunk_sums, void *mean_bf16,
                                 void *stream) {
    using namespace tu;
    TU_REQUIRE(dim == 64 || dim == 128, "K mean requires head_dim 64 or 128, got %lld", static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && heads > 0 && len > 0, "K mean requires positive batch, heads and length");
    TU_REQUIRE(heads <= 65535 && batch <= 65535 && (len + 127) / 128 <= 0x7fffffff, "K mean grid too large");
    TU_REQUIRE(k_bf16 && chunk_sums && mean_bf16, "K mean pointers must be non-null");
    TU_REQUIRE(s_l % 8 == 0 && s_h % 8 == 0 && s_b % 8 == 0 && (reinterpret_cast<uintptr_t>(k_bf16) & 15) == 0,
               "K mean needs 16-byte aligned token rows");
    if (require_gfx950()) return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t chunks = (len + 127) / 128;
    const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(heads), static_cast<unsigned>(batch));
    const auto *k = static_cast<const uint16_t *>(k_bf16);
    if (dim == 128) kmean_chunk_kernel<128><<<grid, kThreads, 0, s>>>(k, len, s_b, s_h, s_l, chunk_sums);
    else kmean_chunk_kernel<64><<<grid, kThreads, 0, s>>>(k, len, s_b, s_h, s_l, chunk_sums);
    if (check_launch("tu_sage_kmean(chunks)")) return -1;
    kmean_final_kernel<<<dim3(static_cast<unsigned>(batch * heads)), 128, 0, s>>>(
        chunk_sums, chunks, len, static_cast<int>(dim), static_cast<uint16_t *>(mean_bf16));
    return check_launch("tu_sage_kmean(final)");
}

namespace tu {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up on the first
// call on that device (with the device current) and kept per device.
int32_t scratch_ptr(float **out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return fail("hipGetDevice failed: %s", hipGetErrorString(err));
    if (dev < 0 || dev >= kMaxDevices) return fail("device %d is beyond the %d devices this library serves", dev,
                                                   kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p)
            return fail("hipGetSymbolAddress(scratch) on device %d failed: %s", dev, hipGetErrorString(err));
        g_scratch_ptr[dev] = static_cast<float *>(p);
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_sage_kmean_noalloc(const void *k_bf16, int64_t batch, int64_t heads, int64_t len,
                                         int64_t dim, int64_t s_b, int64_t s_h, int64_t s_l, void *mean_bf16,
                                         void *stream) {
    using namespace tu;
    TU_REQUIRE(dim == 64 || dim == 128, "K mean requires head_dim 64 or 128, got %lld", static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && heads > 0 && len > 0, "K mean requires positive batch, heads and length");
    TU_REQUIRE(heads <= 65535 && batch <= 65535 && (len + 127) / 128 <= 0x7fffffff, "K mean grid too large");
    TU_REQUIRE(k_bf16 && mean_bf16, "K mean pointers must be non-null");
    TU_REQUIRE(s_l % 8 == 0 && s_h % 8 == 0 && s_b % 8 == 0 && (reinterpret_cast<uintptr_t>(k_bf16) & 15) == 0,
               "K mean needs 16-byte aligned token rows");
    const int64_t chunks = (len + 127) / 128;
    // batch, heads <= 65535 and chunks < 2^31 cannot overflow the product in
    // steps: check each factor against the limit first
    TU_REQUIRE(chunks <= kNoAllocScratchFloats / dim &&
                   batch * heads <= kNoAllocScratchFloats / (chunks * dim),
               "K mean without allocation: batch*heads*ceil(len/128)*dim = %lld*%lld*%lld*%lld exceeds the "
               "%lld-float scratch (use tu_sage_kmean with caller scratch)",
               static_cast<long long>(batch), static_cast<long long>(heads), static_cast<long long>(chunks),
               static_cast<long long>(dim), static_cast<long long>(kNoAllocScratchFloats));
    if (require_gfx950()) return -1;
    float *chunk_sums = nullptr;
    if (scratch_ptr(&chunk_sums)) return -1;
    // Every chunk sum the final kernel reads is written by the chunk kernel
    // of the same call first, so nothing needs clearing.
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(heads), static_cast<unsigned>(batch));
    const auto *k = static_cast<const uint16_t *>(k_bf16);
    if (dim == 128) kmean_chunk_kernel<128><<<grid, kThreads, 0, s>>>(k, len, s_b, s_h, s_l, chunk_sums);
    else kmean_chunk_kernel<64><<<grid, kThreads, 0, s>>>(k, len, s_b, s_h, s_l, chunk_sums);
    if (check_launch("tu_sage_kmean_noalloc(chunks)")) return -1;
    kmean_final_kernel<<<dim3(static_cast<unsigned>(batch * heads)), 128, 0, s>>>(
        chunk_sums, chunks, len, static_cast<int>(dim), static_cast<uint16_t *>(mean_bf16));
    return check_launch("tu_sage_kmean_noalloc(final)");
}

extern "C" int32_t tu_sage_quant(const void *x_bf16, const void *mean_bf16, int64_t batch, int64_t heads,
                                 int64_t len, int64_t dim, int64_t s_b, int64_t s_h, int64_t s_l, int64_t blk,
                                 int8_t *q, int64_t q_b, int64_t q_h, int64_t q_l, float *scale, void *stream) {
    using namespace tu;
    TU_REQUIRE(dim == 64 || dim == 128, "Sage quantization requires head_dim 64 or 128, got %lld",
               static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && heads > 0 && len > 0, "Sage quantization requires positive batch, heads and length");
    TU_REQUIRE(heads <= 65535 && batch <= 65535, "Sage quantization grid too large");
    TU_REQUIRE(x_bf16 && q && scale, "Sage quantization pointers must be non-null");
    TU_REQUIRE(s_l % 8 == 0 && s_h % 8 == 0 && s_b % 8 == 0 && (reinterpret_cast<uintptr_t>(x_bf16) & 15) == 0,
               "Sage quantization needs 16-byte aligned token rows");
    TU_REQUIRE(q_l % 8 == 0 && q_h % 8 == 0 && q_b % 8 == 0 && (reinterpret_cast<uintptr_t>(q) & 7) == 0,
               "Sage quantization output needs 8-byte aligned token rows");
    TU_REQUIRE(!mean_bf16 || (reinterpret_cast<uintptr_t>(mean_bf16) & 15) == 0, "K mean must be 16-byte aligned");
    if (require_gfx950()) return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const auto *x = static_cast<const uint16_t *>(x_bf16);
    const auto *mean = static_cast<const uint16_t *>(mean_bf16);
    if (dim == 128) return launch_quant<128>(x, mean, batch, heads, len, s_b, s_h, s_l, blk, q, q_b, q_h, q_l, scale, s);
    return launch_quant<64>(x, mean, batch, heads, len, s_b, s_h, s_l, blk, q, q_b, q_h, q_l, scale, s);
}
