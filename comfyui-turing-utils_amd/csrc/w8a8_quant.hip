// Prologue of the dense W8A8 attention for gfx950: K stabilisation anchor,
// Hadamard-rotated per-tile INT8 Q/K, and channel-wise INT8 V.
//
// Reference semantics (kernel/csrc/turing/sage/):
//   anchor  DetectKAnchorKernel (fused.cu:409-575): nine keys at rows
//           s (L - 1) / 8 are sampled; the sampled key nearest their mean is
//           the anchor when centring on it lowers the energy of the samples
//           without growing their range by more than 12.5 %, else -1.
//   Q/K     quant_int8_tile with ROTATE (fused.cu:202-407): v = x - x[anchor]
//           (K only), v = H v with H the sign-diagonal normalised
//           Walsh-Hadamard transform (attention_hadamard8, :206-260), then
//           per tile (Q 16 tokens, K 64 tokens) amax = max(1e-7, max |v|),
//           scale = amax / 127, q = cvt.rni.sat.s8(v * (127 / amax)).
//   V       quantize_value_kernel (quant_v_int8_cuda_sm75.cu:58-164):
//           scale[c] = max(amax_c / 127, 1e-12) over all tokens,
//           q = cvt.rni.sat.s8(v * (1 / scale[c])).
// Every reduction here is a max (exact in any order) except the anchor's
// energy sums, which keep the reference's order: one channel per thread,
// 32-lane trees, the four tree results added from 0 in order.
//
// MI355X layout of V: channel-major codes [B][H][D][Lpad] with keys in
// natural order (the INT8 PV MFMA reads 16 consecutive keys of one channel
// per lane).
#include "w8a8_common.h"

namespace tu {
namespace {

template <bool kFp16>
__device__ __forceinline__ float h_to_f32(uint32_t bits16) {
    if constexpr (kFp16) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
    else return __uint_as_float(bits16 << 16);
}

// cvt.rni.sat.s8.f32: round half to even, saturate to [-128, 127].
__device__ __forceinline__ int32_t sat_rne_s8(float v) {
    const float r = __builtin_rintf(v);
    return static_cast<int32_t>(fminf(127.0f, fmaxf(-128.0f, r)));
}

// sat_rne_s8 of four values packed little-endian, without conversions: the
// clamp comes first (the bounds are integers, so clamping and rounding
// commute; NaN clamps to -128 as above), then adding 1.5 * 2^23 rounds half
// to even to an integer whose two's complement sits in the low byte.
__device__ __forceinline__ uint32_t sat_rne_s8x4(float a, float b, float c, float d) {
    const float vs[4] = {a, b, c, d};
    uint32_t w = 0u;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float x = fminf(127.0f, fmaxf(-128.0f, vs[k]));
        w |= (__float_as_uint(x + 12582912.0f) & 0xffu) << (8 * k);
    }
    return w;
}

__device__ __forceinline__ uint32_t pack_s8x4(int32_t a, int32_t b, int32_t c, int32_t d) {
    return (static_cast<uint32_t>(a) & 0xffu) | ((static_cast<uint32_t>(b) & 0xffu) << 8) |
           ((static_cast<uint32_t>(c) & 0xffu) << 16) | (static_cast<uint32_t>(d) << 24);
}

// ---------------------------------------------------------------------------
// K anchor: one workgroup of 128 threads (two wave64 = four 32-lane trees)
// per (kv head, batch).
// ---------------------------------------------------------------------------
template <bool kFp16>
__global__ __launch_bounds__(kAnchorThreads) void anchor_kernel(const uint16_t *__restrict__ k, int64_t len, int dim,
                                                                int64_t s_b, int64_t s_h, int64_t s_l,
                                                                int32_t *__restrict__ anchors) {
    __shared__ float samples[kAnchorSamples][128];
    const int c = threadIdx.x;
    const int64_t h = blockIdx.x, b = blockIdx.y, heads = gridDim.x;
    const uint16_t *kb = k + b * s_b + h * s_h;
#pragma unroll
    for (int s = 0; s < kAnchorSamples; ++s) {
        const int64_t row = static_cast<int64_t>(s) * (len - 1) / (kAnchorSamples - 1);
        samples[s][c] = c < dim ? h_to_f32<kFp16>(kb[row * s_l + c]) : 0.0f;
    }
    __syncthreads();
    const int sel = w8a8_anchor_decide(samples, dim);
    if (c == 0)
        anchors[b * heads + h] =
            sel >= 0 ? static_cast<int32_t>(static_cast<int64_t>(sel) * (len - 1) / (kAnchorSamples - 1)) : -1;
}

// ---------------------------------------------------------------------------
// Rotated Q/K quantizer: one workgroup (4 wave64) per 64-token chunk of a
// head, Q heads first, then K heads.  A thread owns one pack of 8 channels
// of kIters tokens; the D / 8 packs of a token are consecutive lanes, so the
// transform's cross-pack butterfly is a lane xor.  A Q tile (16 tokens) is
// covered by whole wave-passes, so its amax is a wave max plus an exchange
// through LDS.
// ---------------------------------------------------------------------------
constexpr int kQkThreads = 256;
constexpr int kChunk = 64;

struct RotArgs {
    const uint16_t *x[2];
    int8_t *out[2];
    float *scale[2];
    const int32_t *anchors;  // [B][Hk] or null
    int64_t heads[2], len[2], ntiles[2];
    int64_t x_sb[2], x_sh[2], x_sl[2];
    int64_t o_sb[2], o_sh[2], o_sl[2];
    int rotate;
};

template <bool kFp16, int D>
__global__ __launch_bounds__(kQkThreads) void rot_quant_kernel(RotArgs args) {
    constexpr int kPacks = D / 8;
    constexpr int kTokPerPass = kQkThreads / kPacks;   // 16 (D 128) or 32 (D 64)
    constexpr int kIters = kChunk / kTokPerPass;        // 4 or 2
    constexpr int kWaveTok = 64 / kPacks;               // tokens of one wave-pass
    __shared__ float wave_amax[kIters][kQkThreads / 64];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int pack = tid % kPacks;
    const int64_t b = blockIdx.y;
    int64_t task = blockIdx.x;
    const int64_t nch_q = (args.len[0] + kChunk - 1) / kChunk;
    const int which = task < args.heads[0] * nch_q ? 0 : 1;
    if (which) task -= args.heads[0] * nch_q;
    const int64_t len = args.len[which];
    const int64_t nch = (len + kChunk - 1) / kChunk;
    const int64_t head = task / nch;
    const int64_t chunk = task - head * nch;
    const int64_t t0 = chunk * kChunk;
    const uint16_t *xbase = args.x[which] + b * args.x_sb[which] + head * args.x_sh[which];

    float anchor[8];
    bool anchored = false;
    if (which == 1 && args.anchors != nullptr) {
        const int32_t a = args.anchors[b * args.heads[1] + head];
        anchored = a >= 0;
        if (anchored) {
            const u32x4 raw = *reinterpret_cast<const u32x4 *>(xbase + static_cast<int64_t>(a) * args.x_sl[1] + pack * 8);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                anchor[2 * j] = h_to_f32<kFp16>(raw[j] & 0xffffu);
                anchor[2 * j + 1] = h_to_f32<kFp16>(raw[j] >> 16);
            }
        }
    }

    float v[kIters][8];
    float amax[kIters];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
        const int64_t t = t0 + it * kTokPerPass + tid / kPacks;
        u32x4 raw = u32x4{0u, 0u, 0u, 0u};
        if (t < len) raw = *reinterpret_cast<const u32x4 *>(xbase + t * args.x_sl[which] + pack * 8);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[it][2 * j] = h_to_f32<kFp16>(raw[j] & 0xffffu);
            v[it][2 * j + 1] = h_to_f32<kFp16>(raw[j] >> 16);
        }
        if (anchored && t < len) {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[it][j] = v[it][j] - anchor[j];
        }
        if (args.rotate) w8a8_hadamard_pack<D>(v[it], pack);
        float a = 0.0000001f;
#pragma unroll
        for (int j = 0; j < 8; ++j) a = fmaxf(a, fabsf(v[it][j]));
        amax[it] = wave_max_nonneg(a);   // a >= 1e-7 and never NaN (fmaxf passes NaN over)
    }
    if ((tid & 63) == 0) {
#pragma unroll
        for (int it = 0; it < kIters; ++it) wave_amax[it][wave] = amax[it];
    }
    __syncthreads();

    // Scale of each token's tile: Q tiles of 16 tokens, one K tile per chunk.
    float mult[kIters];
    if (which == 0) {
        // Q tile s = tokens [16 s, 16 s + 16) of the chunk: the max of the
        // wave-passes inside it.
        constexpr int kSubs = kChunk / 16;
        float sub_amax[kSubs];
#pragma unroll
        for (int s = 0; s < kSubs; ++s) sub_amax[s] = 0.0f;
#pragma unroll
        for (int w = 0; w < kQkThreads / 64; ++w)
#pragma unroll
            for (int i2 = 0; i2 < kIters; ++i2) {
                const int s = (i2 * kTokPerPass + w * kWaveTok) / 16;
                sub_amax[s] = fmaxf(sub_amax[s], wave_amax[i2][w]);
            }
#pragma unroll
        for (int it = 0; it < kIters; ++it) {
            const int mine = (it * kTokPerPass + wave * kWaveTok) / 16;
            float a = sub_amax[0];
#pragma unroll
            for (int s = 1; s < kSubs; ++s) a = mine == s ? sub_amax[s] : a;
            mult[it] = 127.0f / a;
        }
        if (tid < kSubs) {
            float a = sub_amax[0];
#pragma unroll
            for (int s = 1; s < kSubs; ++s) a = tid == s ? sub_amax[s] : a;
            args.scale[0][(b * args.heads[0] + head) * args.ntiles[0] + chunk * kSubs + tid] = a / 127.0f;
        }
    } else {
        float a = 0.0f;
#pragma unroll
        for (int w = 0; w < kQkThreads / 64; ++w)
#pragma unroll
            for (int i2 = 0; i2 < kIters; ++i2) a = fmaxf(a, wave_amax[i2][w]);
#pragma unroll
        for (int it = 0; it < kIters; ++it) mult[it] = 127.0f / a;
        if (tid == 0) args.scale[1][(b * args.heads[1] + head) * args.ntiles[1] + chunk] = a / 127.0f;
    }

    int8_t *obase = args.out[which] + b * args.o_sb[which] + head * args.o_sh[which];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
        const int64_t t = t0 + it * kTokPerPass + tid / kPacks;
        if (t >= len) continue;
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = v[it][j] * mult[it];
        const u32x2 packed{sat_rne_s8x4(y[0], y[1], y[2], y[3]), sat_rne_s8x4(y[4], y[5], y[6], y[7])};
        *reinterpret_cast<u32x2 *>(obase + t * args.o_sl[which] + pack * 8) = packed;
    }
}

// ---------------------------------------------------------------------------
// V: per-channel amax over token chunks, scales, codes.
// ---------------------------------------------------------------------------
constexpr int kVThreads = 256;
constexpr int kVChunk = 1024;  // tokens per amax workgroup

template <bool kFp16, int D>
__global__ __launch_bounds__(kVThreads) void v_amax_kernel(const uint16_t *__restrict__ v, int64_t len, int64_t s_b,
                                                          int64_t s_h, int64_t s_l, float *__restrict__ partial) {
    constexpr int kPacks = D / 8;
    constexpr int kRows = kVThreads / kPacks;
    __shared__ float wave_max[kVThreads / 64][D];
    const int tid = threadIdx.x;
    const int pack = tid % kPacks;
    const int64_t chunk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int64_t chunks = gridDim.x, heads = gridDim.y;
    const uint16_t *base = v + b * s_b + h * s_h;
    float m[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) m[j] = 0.0f;
    const int64_t t_end = min(len, (chunk + 1) * kVChunk);
#pragma unroll 4
    for (int64_t t = chunk * kVChunk + tid / kPacks; t < t_end; t += kRows) {
        const u32x4 raw = *reinterpret_cast<const u32x4 *>(base + t * s_l + pack * 8);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            m[2 * j] = fmaxf(m[2 * j], fabsf(h_to_f32<kFp16>(raw[j] & 0xffffu)));
            m[2 * j + 1] = fmaxf(m[2 * j + 1], fabsf(h_to_f32<kFp16>(raw[j] >> 16)));
        }
    }
    // lanes l, l + kPacks, ... of a wave hold the same channels
#pragma unroll
    for (int off = kPacks; off < 64; off <<= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] = fmaxf(m[j], __shfl_xor(m[j], off));
    if ((tid & 63) < kPacks) {
#pragma unroll
        for (int j = 0; j < 8; ++j) wave_max[tid >> 6][pack * 8 + j] = m[j];
    }
    __syncthreads();
    if (tid < D) {
        float a = 0.0f;
#pragma unroll
        for (int w = 0; w < kVThreads / 64; ++w) a = fmaxf(a, wave_max[w][tid]);
        partial[((b * heads + h) * chunks + chunk) * D + tid] = a;
    }
}

template <int D>
__global__ __launch_bounds__(D) void v_scale_kernel(const float *__restrict__ partial, int64_t chunks,
                                                    float *__restrict__ scale) {
    const int c = threadIdx.x;
    const int64_t bh = blockIdx.x;
    float a = 0.0f;
    for (int64_t i = 0; i < chunks; ++i) a = fmaxf(a, partial[(bh * chunks + i) * D + c]);
    scale[bh * D + c] = fmaxf(a / 127.0f, 1.0e-12f);
}

// One workgroup per 64-key tile: codes through an LDS byte tile (rows of D
// + 16 bytes), written channel-major as 16-byte key runs.
template <bool kFp16, int D>
__global__ __launch_bounds__(kVThreads) void v_quant_kernel(const uint16_t *__restrict__ v, int64_t len, int64_t lpad,
                                                           int64_t s_b, int64_t s_h, int64_t s_l,
                                                           const float *__restrict__ scale, int8_t *__restrict__ vq) {
    constexpr int kPacks = D / 8;
    constexpr int kRows = kVThreads / kPacks;
    constexpr int kRowBytes = D + 16;
    __shared__ __align__(16) int8_t tile[64 * kRowBytes];
    const int tid = threadIdx.x;
    const int pack = tid % kPacks;
    const int64_t tix = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int64_t heads = gridDim.y;
    const int64_t bh = b * heads + h;
    const uint16_t *base = v + b * s_b + h * s_h;
    float inv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) inv[j] = 1.0f / scale[bh * D + pack * 8 + j];
#pragma unroll
    for (int r0 = 0; r0 < 64; r0 += kRows) {
        const int r = r0 + tid / kPacks;
        const int64_t t = tix * 64 + r;
        u32x4 raw = u32x4{0u, 0u, 0u, 0u};
        if (t < len) raw = *reinterpret_cast<const u32x4 *>(base + t * s_l + pack * 8);
        int32_t q[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            q[2 * j] = sat_rne_s8(h_to_f32<kFp16>(raw[j] & 0xffffu) * inv[2 * j]);
            q[2 * j + 1] = sat_rne_s8(h_to_f32<kFp16>(raw[j] >> 16) * inv[2 * j + 1]);
        }
        u32x2 packed;
        packed.x = pack_s8x4(q[0], q[1], q[2], q[3]);
        packed.y = pack_s8x4(q[4], q[5], q[6], q[7]);
        *reinterpret_cast<u32x2 *>(tile + r * kRowBytes + pack * 8) = packed;
    }
    __syncthreads();
    // item = (channel, 16-key run)
#pragma unroll
    for (int item = tid; item < D * 4; item += kVThreads) {
        const int c = item >> 2, run = item & 3;
        u32x4 out;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int8_t code = tile[(run * 16 + 4 * w + e) * kRowBytes + c];
                word |= (static_cast<uint32_t>(code) & 0xffu) << (8 * e);
            }
            out[w] = word;
        }
        *reinterpret_cast<u32x4 *>(vq + (bh * D + c) * lpad + tix * 64 + run * 16) = out;
    }
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_w8a8_quant_qk(const void *q, const void *k, int32_t dtype, int64_t batch, int64_t hq,
                                    int64_t hk, int64_t lq, int64_t lk, int64_t dim, int64_t q_sb, int64_t q_sh,
                                    int64_t q_sl, int64_t k_sb, int64_t k_sh, int64_t k_sl, int8_t *q8,
                                    int64_t q8_sb, int64_t q8_sh, int64_t q8_sl, int8_t *k8, int64_t k8_sb,
                                    int64_t k8_sh, int64_t k8_sl, float *q_scale, float *k_scale,
                                    int32_t *anchors, int32_t rotate, void *stream) {
    using namespace tu;
    TU_REQUIRE(dtype == 0 || dtype == 1, "W8A8 Q/K dtype must be 0 (bf16) or 1 (fp16)");
    TU_REQUIRE(dim == 64 || dim == 128, "W8A8 Q/K quantizer requires head_dim 64 or 128, got %lld",
               static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && hq > 0 && hk > 0 && lq > 0 && lk > 0 && batch <= 65535,
               "W8A8 Q/K quantizer dimensions out of range");
    TU_REQUIRE(q && k && q8 && k8 && q_scale && k_scale, "W8A8 Q/K quantizer pointers must be non-null");
    const int64_t nq = (lq + kChunk - 1) / kChunk, nk = (lk + kChunk - 1) / kChunk;
    TU_REQUIRE(hq * nq + hk * nk <= 0x7fffffff, "W8A8 Q/K quantizer grid too large");
    TU_REQUIRE(q_sb % 8 == 0 && q_sh % 8 == 0 && q_sl % 8 == 0 && k_sb % 8 == 0 && k_sh % 8 == 0 && k_sl % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(q) & 15) == 0 && (reinterpret_cast<uintptr_t>(k) & 15) == 0,
               "W8A8 Q/K inputs need 16-byte aligned rows");
    TU_REQUIRE(q8_sb % 8 == 0 && q8_sh % 8 == 0 && q8_sl % 8 == 0 && k8_sb % 8 == 0 && k8_sh % 8 == 0 &&
                   k8_sl % 8 == 0 && (reinterpret_cast<uintptr_t>(q8) & 7) == 0 &&
                   (reinterpret_cast<uintptr_t>(k8) & 7) == 0,
               "W8A8 Q/K codes need 8-byte aligned rows");
    if (require_gfx950()) return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (anchors != nullptr) {
        const dim3 grid(static_cast<unsigned>(hk), static_cast<unsigned>(batch));
        if (dtype) anchor_kernel<true><<<grid, kAnchorThreads, 0, s>>>(static_cast<const uint16_t *>(k), lk,
                                                                        static_cast<int>(dim), k_sb, k_sh, k_sl, anchors);
        else anchor_kernel<false><<<grid, kAnchorThreads, 0, s>>>(static_cast<const uint16_t *>(k), lk,
                                                                   static_cast<int>(dim), k_sb, k_sh, k_sl, anchors);
        if (int32_t rc = check_launch("tu_w8a8_quant_qk (anchor)")) return rc;
    }
    RotArgs a{};
    a.x[0] = static_cast<const uint16_t *>(q);
    a.x[1] = static_cast<const uint16_t *>(k);
    a.out[0] = q8;
    a.out[1] = k8;
    a.scale[0] = q_scale;
    a.scale[1] = k_scale;
    a.anchors = anchors;
    a.heads[0] = hq;
    a.heads[1] = hk;
    a.len[0] = lq;
    a.len[1] = lk;
    a.ntiles[0] = nq * 4;
    a.ntiles[1] = nk;
    a.x_sb[0] = q_sb; a.x_sh[0] = q_sh; a.x_sl[0] = q_sl;
    a.x_sb[1] = k_sb; a.x_sh[1] = k_sh; a.x_sl[1] = k_sl;
    a.o_sb[0] = q8_sb; a.o_sh[0] = q8_sh; a.o_sl[0] = q8_sl;
    a.o_sb[1] = k8_sb; a.o_sh[1] = k8_sh; a.o_sl[1] = k8_sl;
    a.rotate = rotate != 0;
    const dim3 grid(static_cast<unsigned>(hq * nq + hk * nk), static_cast<unsigned>(batch));
    if (dtype) {
        if (dim == 128) rot_quant_kernel<true, 128><<<grid, kQkThreads, 0, s>>>(a);
        else rot_quant_kernel<true, 64><<<grid, kQkThreads, 0, s>>>(a);
    } else {
        if (dim == 128) rot_quant_kernel<false, 128><<<grid, kQkThreads, 0, s>>>(a);
        else rot_quant_kernel<false, 64><<<grid, kQkThreads, 0, s>>>(a);
    }
    return check_launch("tu_w8a8_quant_qk");
}

extern "C" int64_t tu_w8a8_quant_v_workspace(int64_t batch, int64_t heads, int64_t len, int64_t dim) {
    if (batch <= 0 || heads <= 0 || len <= 0 || dim <= 0) return -1;
    const int64_t chunks = (len + tu::kVChunk - 1) / tu::kVChunk;
    // partial maxima (fp32)
    return batch * heads * dim * chunks * 4;
}

extern "C" int32_t tu_w8a8_quant_v(const void *v, int32_t dtype, int64_t batch, int64_t heads, int64_t len,
                                   int64_t dim, int64_t s_b, int64_t s_h, int64_t s_l, int8_t *vq, int64_t lpad,
                                   float *scale, void *workspace, int64_t workspace_bytes,
                                   void *stream) {
    using namespace tu;
    TU_REQUIRE(dtype == 0 || dtype == 1, "W8A8 V dtype must be 0 (bf16) or 1 (fp16)");
    TU_REQUIRE(dim == 64 || dim == 128, "W8A8 V quantizer requires head_dim 64 or 128, got %lld",
               static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && heads > 0 && len > 0 && batch <= 65535 && heads <= 65535,
               "W8A8 V quantizer dimensions out of range");
    TU_REQUIRE(lpad == (len + 63) / 64 * 64, "W8A8 V padded length must be ceil(len / 64) * 64");
    TU_REQUIRE(v && vq && scale && workspace, "W8A8 V quantizer pointers must be non-null");
    TU_REQUIRE(workspace_bytes >= tu_w8a8_quant_v_workspace(batch, heads, len, dim),
               "W8A8 V quantizer workspace too small");
    TU_REQUIRE(s_b % 8 == 0 && s_h % 8 == 0 && s_l % 8 == 0 && (reinterpret_cast<uintptr_t>(v) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(vq) & 15) == 0 && (reinterpret_cast<uintptr_t>(workspace) & 3) == 0,
               "W8A8 V quantizer needs 16-byte aligned rows");
    if (require_gfx950()) return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t chunks = (len + kVChunk - 1) / kVChunk;
    const int64_t ntiles = lpad / 64;
    float *partial = static_cast<float *>(workspace);
    const uint16_t *vp = static_cast<const uint16_t *>(v);
    const dim3 g1(static_cast<unsigned>(chunks), static_cast<unsigned>(heads), static_cast<unsigned>(batch));
    const dim3 g3(static_cast<unsigned>(ntiles), static_cast<unsigned>(heads), static_cast<unsigned>(batch));
    const unsigned bh = static_cast<unsigned>(batch * heads);
#define TU_V_LAUNCH(F16, DD)                                                                                  \
    do {                                                                                                      \
        v_amax_kernel<F16, DD><<<g1, kVThreads, 0, s>>>(vp, len, s_b, s_h, s_l, partial);                     \
        v_scale_kernel<DD><<<bh, DD, 0, s>>>(partial, chunks, scale);                                         \
        v_quant_kernel<F16, DD><<<g3, kVThreads, 0, s>>>(vp, len, lpad, s_b, s_h, s_l, scale, vq);            \
    } while (0)
    if (dtype) {
        if (dim == 128) TU_V_LAUNCH(true, 128);
        else TU_V_LAUNCH(true, 64);
    } else {
        if (dim == 128) TU_V_LAUNCH(false, 128);
        else TU_V_LAUNCH(false, 64);
    }
#undef TU_V_LAUNCH
    return check_launch("tu_w8a8_quant_v");
}
