// Fused Q/K RMSNorm + RoPE + per-tile INT8 quantization for gfx950: the
// producer of Sage attention's Q/K in a Wan block.
//
// Semantics follow the reference's quantize_qk_kernel / quantize_tile
// (kernel/csrc/turing/sage/qk_preprocess.cu:417-629) without its Hadamard /
// anchor variant:
//   rrms = 1 / sqrt(sumsq / n + eps)   per token: over the head's D channels
//          (head scope) or over all H*D channels of the token (row scope)
//   a_c  = T((x_c * rrms) * w_c)       T = the input type (bf16 or fp16)
//   y_c  = T(fma(f1, a_second, f0 * a_first)) for c < rot_dim (interleaved
//          or split-half pairs; (f0, f1) the row of the pair's 2x2 matrix
//          that produces channel c), y_c = a_c otherwise
//   per tile (Q: 16 tokens, K: 64 tokens) of one (batch, head):
//   amax = max(1e-7, max |y|), scale = amax / 127,
//   q = clamp(rint(y * (127 / amax)), -127, 127).
// The sum of squares has a fixed order (8-channel FMA chains, then a
// butterfly across a head's packs; heads added in order for the row scope),
// and square root and divisions are IEEE, so the CPU oracle restates it bit
// for bit.  The reference uses rsqrtf, which is not reproduced.
//
// MI355X mapping: one workgroup (4 wave64) per 64-token chunk of a head (four
// Q tiles or one K tile; a Q tile is whole waves, so its amax is a wave max
// plus one LDS exchange shared by the four).  A thread owns 8
// consecutive channels ("pack") of a token; the packs of one token are
// consecutive lanes, so the head-scope sum is a lane butterfly.  The
// normalized tile goes through LDS once so RoPE can take its pair partner
// from any pack (split-half pairs and partial rot_dim included).  Row-scope
// rrms comes from a pre-pass into caller scratch.  Interleaved RoPE over the
// whole head (or none) takes a fast path that processes a group of heads per
// workgroup (qk_rope_quant_heads_kernel).
#include <type_traits>

#include "attn_common.h"
#include "w8a8_common.h"

namespace tu {
namespace {

constexpr int kQkThreads = 256;
constexpr int kQTile = 16;   // Q scale granularity (tokens)
constexpr int kChunk = 64;   // tokens per workgroup = the K scale granularity

// bf16 (kFp16 = false) or fp16 bit patterns <-> fp32.
template <bool kFp16>
__device__ __forceinline__ float t_to_f32(uint32_t bits16) {
    if constexpr (kFp16) return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
    else return __uint_as_float(bits16 << 16);
}
// Round to the input type (RNE, the hardware conversion) and back.  The
// empty asm pins v as an fp32 value first: without it the compiler folds the
// conversion into the producing multiply or FMA (v_fma_mixlo_f16), which
// rounds the exact result to fp16 once instead of rounding to fp32 and then
// to fp16 as the reference does, and differs at fp32 values that are fp16
// rounding ties.
template <bool kFp16>
__device__ __forceinline__ float t_round(float v) {
    asm volatile("" : "+v"(v));
    if constexpr (kFp16) return static_cast<float>(static_cast<_Float16>(v));
    else return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(v))) << 16);
}

// t_round of a pair: bf16 rounds both with one v_cvt_pk_bf16_f32 (the
// conversion t_round's cast compiles to), fp16 one value at a time.
template <bool kFp16>
__device__ __forceinline__ void t_round2(float &a, float &b) {
    asm volatile("" : "+v"(a), "+v"(b));
    if constexpr (kFp16) {
        a = static_cast<float>(static_cast<_Float16>(a));
        b = static_cast<float>(static_cast<_Float16>(b));
    } else {
        const uint32_t w = hw_bf16x2_bits(a, b);
        a = __uint_as_float(w << 16);
        b = __uint_as_float(w & 0xffff0000u);
    }
}

// t_round2 that also returns the rounded pair as packed T bits (low = a),
// for kernels that keep rounded values packed.  The fp16 pair conversion is
// the same round-to-nearest-even as the single-value cast.
template <bool kFp16>
__device__ __forceinline__ uint32_t t_round2w(float &a, float &b) {
    asm volatile("" : "+v"(a), "+v"(b));
    uint32_t w;
    if constexpr (kFp16) w = hw_f16x2_bits(a, b);
    else w = hw_bf16x2_bits(a, b);
    a = t_to_f32<kFp16>(w & 0xffffu);
    b = t_to_f32<kFp16>(w >> 16);
    return w;
}

// INT8 codes of four values, packed little-endian: clamp(rint(y * inv),
// -127, 127).  The clamp comes first (the bounds are integers, so clamping
// and rounding commute; a NaN product clamps to -127 as fminf(127,
// fmaxf(-127, rint(NaN))) does), then adding 1.5 * 2^23 rounds half to even
// to an integer whose two's complement sits in the low byte of the sum.
__device__ __forceinline__ uint32_t quant_pack4(float y0, float y1, float y2, float y3, float inv) {
    const float ys[4] = {y0, y1, y2, y3};
    uint32_t w = 0u;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float c = fminf(127.0f, fmaxf(-127.0f, ys[k] * inv));
        w |= (__float_as_uint(c + 12582912.0f) & 0xffu) << (8 * k);
    }
    return w;
}

// v + (v of lane i ^ kOff), the step of a butterfly sum over the P lanes of a
// token (P = 8 or 16 consecutive lanes, kOff < P), as __shfl_xor(v, kOff, P)
// gives it but without index arithmetic: DPP quad permutations for 1 and 2,
// row rotation by 8 (lane (i + 8) mod 16 is lane i ^ 8), and a bit-mode
// ds_swizzle for 4.  Addition is commutative, so the sums are bit-identical.
template <int kOff>
__device__ __forceinline__ float butterfly_add(float v) {
    int o;
    if constexpr (kOff == 1) o = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false);
    else if constexpr (kOff == 2) o = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false);
    else if constexpr (kOff == 8) o = __builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false);
    else o = __builtin_amdgcn_ds_swizzle(__float_as_int(v), (kOff << 10) | 0x1f);
    return v + __int_as_float(o);
}
template <int kPacks>
__device__ __forceinline__ float pack_sum(float v) {
    if constexpr (kPacks == 16) v = butterfly_add<8>(v);
    v = butterfly_add<4>(v);
    v = butterfly_add<2>(v);
    return butterfly_add<1>(v);
}

// max(m, |a|, |b|) in one instruction.  A quiet NaN operand is passed over
// (IEEE maxNum), as fmaxf passes it over; a and b are never signalling NaNs
// here (they come out of hardware conversions).
__device__ __forceinline__ float max3_abs(float m, float a, float b) {
    float r;
    asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
    return r;
}

struct QkArgs {
    const uint16_t *x[2];        // Q, K
    const uint16_t *norm[2];
    float *rrms[2];              // row scope: [B, L] per tensor
    int8_t *out[2];
    float *scale[2];
    const uint16_t *freqs;
    int64_t heads[2], len[2];
    int64_t x_sb[2], x_sh[2], x_sl[2];
    int64_t o_sb[2], o_sh[2], o_sl[2];
    int64_t ntiles[2];           // scale entries per (batch, head)
    int64_t f_sb, f_sl, f_sp, f_sr, f_sc;
    int f_contig;                // [.., pair, 2, 2] contiguous, 16-byte aligned rows
    int64_t f_batches, f_len;
    int rot_dim;
    float eps;
    const int32_t *anchors;   // K stabilisation [B][Hk] (W8A8 variant) or null
    float *anchor_values;     // [B][Hk][D]: the anchor row's processed values
    int k_only;               // row pre-pass / head-group kernel: K's tasks only
};

template <bool kFp16, int D, bool kSplit, bool kRow, bool kRotate>
__global__ __launch_bounds__(kQkThreads) void qk_rope_quant_kernel(QkArgs args) {
    constexpr int kPacks = D / 8;                        // lanes per token
    constexpr int kIters = kChunk * kPacks / kQkThreads;  // packs per thread
    constexpr int kSubs = kChunk / kQTile;                // 16-token sub-tiles per chunk
    // Split-half pairs take their partner from another pack through LDS;
    // interleaved pairs are inside a pack and stay in registers.
    __shared__ __align__(16) float tile_a[kSplit ? kChunk * D : 4];
    __shared__ float wave_amax[kQkThreads / 64][kSubs];

    const int tid = threadIdx.x;
    const int64_t b = blockIdx.y;
    // Tasks: 64-token chunks of every Q head first, then of every K head.
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
    const uint16_t *norm = args.norm[which] + (kRow ? head * D : 0);
    const int pairs = args.rot_dim / 2;

    // W8A8 variant: K rows are centred on the head's anchor row before the
    // rotation.  A thread's pack index is fixed (256 is a multiple of D / 8).
    float anc[8];
    bool anchored = false;
    if constexpr (kRotate) {
        if (which == 1 && args.anchors != nullptr) {
            anchored = args.anchors[b * args.heads[1] + head] >= 0;
            const float *ap = args.anchor_values + (b * args.heads[1] + head) * D + (tid % kPacks) * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j) anc[j] = anchored ? ap[j] : 0.0f;
        }
    }

    // Pass 1: RMSNorm (into the LDS tile for split-half pairs).
    float av[kIters][8];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
        const int pidx = tid + it * kQkThreads;
        const int to = pidx / kPacks, pack = pidx % kPacks;
        const int64_t t = t0 + to;
        const bool valid = t < len;
        u32x4 raw = u32x4{0u, 0u, 0u, 0u};
        if (valid) raw = *reinterpret_cast<const u32x4 *>(xbase + t * args.x_sl[which] + pack * 8);
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = t_to_f32<kFp16>(raw[j] & 0xffffu);
            v[2 * j + 1] = t_to_f32<kFp16>(raw[j] >> 16);
        }
        float rrms;
        if constexpr (kRow) {
            rrms = valid ? args.rrms[which][b * len + t] : 0.0f;
        } else {
            // Every lane of the token's pack group takes part, valid or not.
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) s = __builtin_fmaf(v[c], v[c], s);
#pragma unroll
            for (int off = kPacks / 2; off > 0; off >>= 1) s = s + __shfl_xor(s, off, kPacks);
            rrms = 1.0f / __builtin_sqrtf(s / static_cast<float>(D) + args.eps);
        }
        const u32x4 wraw = *reinterpret_cast<const u32x4 *>(norm + pack * 8);
        float *a = av[it];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            a[2 * j] = t_round<kFp16>((v[2 * j] * rrms) * t_to_f32<kFp16>(wraw[j] & 0xffffu));
            a[2 * j + 1] = t_round<kFp16>((v[2 * j + 1] * rrms) * t_to_f32<kFp16>(wraw[j] >> 16));
        }
        if constexpr (kSplit) {
            float *dst = tile_a + to * D + pack * 8;
            *reinterpret_cast<f32x4 *>(dst) = f32x4{a[0], a[1], a[2], a[3]};
            *reinterpret_cast<f32x4 *>(dst + 4) = f32x4{a[4], a[5], a[6], a[7]};
        }
    }
    if constexpr (kSplit) __syncthreads();

    // Pass 2: RoPE, amax per 16-token sub-tile (a sub-tile is whole waves:
    // 16 tokens x kPacks lanes = 256 or 128 lanes).
    float y[kIters][8];
    float amax[kSubs];
#pragma unroll
    for (int sub = 0; sub < kSubs; ++sub) amax[sub] = 0.0000001f;
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
        const int pidx = tid + it * kQkThreads;
        const int to = pidx / kPacks, pack = pidx % kPacks;
        const int64_t t = t0 + to;
        const uint16_t *frow = args.rot_dim == 0 ? nullptr
                                                 : args.freqs + (args.f_batches == 1 ? 0 : b) * args.f_sb +
                                                       (args.f_len == 1 ? 0 : t) * args.f_sl;
        const float *a = av[it];
        float pmax = 0.0f;
        const bool rope = t < len && pack * 8 < args.rot_dim;
        if (rope && args.f_contig && pack * 8 + 8 <= args.rot_dim && (!kSplit || pairs % 8 == 0)) {
            // The pack's frequency rows as 16-byte loads ([pair][row][col]
            // contiguous): interleaved, pairs 4 pack .. + 3 (all four values);
            // split-half, 8 pairs of one row.
            if constexpr (!kSplit) {
                const u32x4 f01 = *reinterpret_cast<const u32x4 *>(frow + pack * 16);
                const u32x4 f23 = *reinterpret_cast<const u32x4 *>(frow + pack * 16 + 8);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int i = j >> 1, comp = j & 1;
                    const uint32_t word = (i < 2 ? f01 : f23)[(i & 1) * 2 + comp];
                    const float f0 = t_to_f32<kFp16>(word & 0xffffu), f1 = t_to_f32<kFp16>(word >> 16);
                    const float val = t_round<kFp16>(__builtin_fmaf(f1, a[2 * i + 1], f0 * a[2 * i]));
                    y[it][j] = val;
                    pmax = fmaxf(pmax, fabsf(val));
                }
            } else {
                const int comp = pack * 8 >= pairs;
                const int pb = pack * 8 - (comp ? pairs : 0);
                const float *arow = tile_a + to * D;
                u32x4 fv[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) fv[r] = *reinterpret_cast<const u32x4 *>(frow + pb * 4 + r * 8);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t word = fv[j >> 1][(j & 1) * 2 + comp];
                    const float f0 = t_to_f32<kFp16>(word & 0xffffu), f1 = t_to_f32<kFp16>(word >> 16);
                    const float val = t_round<kFp16>(__builtin_fmaf(f1, arow[pb + j + pairs], f0 * arow[pb + j]));
                    y[it][j] = val;
                    pmax = fmaxf(pmax, fabsf(val));
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = pack * 8 + j;
                float val = a[j];
                if (c < args.rot_dim && t < len) {
                    const int pair = kSplit ? (c < pairs ? c : c - pairs) : c >> 1;
                    const int comp = kSplit ? (c >= pairs) : (c & 1);
                    const uint16_t *fp = frow + pair * args.f_sp + comp * args.f_sr;
                    const float f0 = t_to_f32<kFp16>(fp[0]);
                    const float f1 = t_to_f32<kFp16>(fp[args.f_sc]);
                    float x0, x1;
                    if constexpr (kSplit) {
                        x0 = tile_a[to * D + pair];
                        x1 = tile_a[to * D + pair + pairs];
                    } else {
                        x0 = a[j & ~1];
                        x1 = a[j | 1];
                    }
                    val = t_round<kFp16>(__builtin_fmaf(f1, x1, f0 * x0));
                }
                y[it][j] = val;
                pmax = fmaxf(pmax, fabsf(val));
            }
        }
        if constexpr (kRotate) {
            // v = hadamard(y - anchor), every lane of the token's group
            // taking part (tokens past L are zero)
            if (anchored && t < len) {
#pragma unroll
                for (int j = 0; j < 8; ++j) y[it][j] -= anc[j];
            }
            w8a8_hadamard_pack<D>(y[it], pack);
            pmax = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) pmax = fmaxf(pmax, fabsf(y[it][j]));
        }
        if (t < len) {
            const int sub = to / kQTile;
#pragma unroll
            for (int s2 = 0; s2 < kSubs; ++s2) amax[s2] = sub == s2 ? fmaxf(amax[s2], pmax) : amax[s2];
        }
    }
#pragma unroll
    for (int sub = 0; sub < kSubs; ++sub) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) amax[sub] = fmaxf(amax[sub], __shfl_xor(amax[sub], off, 64));
        if ((tid & 63) == 0) wave_amax[tid >> 6][sub] = amax[sub];
    }
    __syncthreads();
    float inv[kSubs];
    float kmax = 0.0000001f;
#pragma unroll
    for (int sub = 0; sub < kSubs; ++sub) {
        const float m = fmaxf(fmaxf(wave_amax[0][sub], wave_amax[1][sub]), fmaxf(wave_amax[2][sub], wave_amax[3][sub]));
        kmax = fmaxf(kmax, m);
        inv[sub] = 127.0f / m;
        if (which == 0 && tid == sub)
            args.scale[0][(b * args.heads[0] + head) * args.ntiles[0] + chunk * kSubs + sub] = m / 127.0f;
    }
    if (which == 1) {
        if (tid == 0) args.scale[1][(b * args.heads[1] + head) * args.ntiles[1] + chunk] = kmax / 127.0f;
        const float kinv = 127.0f / kmax;
#pragma unroll
        for (int sub = 0; sub < kSubs; ++sub) inv[sub] = kinv;
    }

    // Pass 3: codes, one 8-byte store per pack.
    int8_t *obase = args.out[which] + b * args.o_sb[which] + head * args.o_sh[which];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
        const int pidx = tid + it * kQkThreads;
        const int to = pidx / kPacks, pack = pidx % kPacks;
        const int64_t t = t0 + to;
        if (t >= len) continue;
        float iv = inv[0];
#pragma unroll
        for (int sub = 1; sub < kSubs; ++sub) iv = to / kQTile == sub ? inv[sub] : iv;
        uint32_t w[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float r = fminf(127.0f, fmaxf(-127.0f, __builtin_rintf(y[it][j] * iv)));
            w[j >> 2] |= (static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu) << (8 * (j & 3));
        }
        *reinterpret_cast<u32x2 *>(obase + t * args.o_sl[which] + pack * 8) = u32x2{w[0], w[1]};
    }
}

// Fast path for interleaved RoPE over the whole head (or no RoPE) with the
// frequencies in their contiguous [.., pair, 2, 2] layout: one workgroup
// (4 wave64) per 64-token chunk and group of kHeadGroup heads of Q or of K,
// chunk-major.  Wave w owns tokens 16 w .. 16 w + 15 of the chunk (one Q
// scale tile); lane l owns pack l % P of tokens 16 w + l / P + (64 / P) i,
// i < kItems (P = D / 8 packs a token).  A lane's frequency words and
// row-scope rrms do not depend on the head, so they are loaded once per chunk
// and kept in registers for the group's heads (the general kernel reads the
// frequency table again for every head).  The Q amax is a wave reduction;
// K's 64-token amax adds one LDS exchange per head.  Per element the
// arithmetic is the general kernel's, operation for operation.
#ifndef TU_QK_HEAD_GROUP
#define TU_QK_HEAD_GROUP 8
#endif
constexpr int kHeadGroup = TU_QK_HEAD_GROUP;

template <bool kFp16, int D, bool kRow, bool kRope>
__global__ __launch_bounds__(kQkThreads) void qk_rope_quant_heads_kernel(QkArgs args) {
    constexpr int kPacks = D / 8;
    constexpr int kTokStep = 64 / kPacks;   // tokens one lane row of a wave covers
    constexpr int kItems = 16 / kTokStep;   // (token, pack) items per lane
    __shared__ float kamax[2][kQkThreads / 64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t b = blockIdx.y;
    const int64_t nch_q = (args.len[0] + kChunk - 1) / kChunk;
    const int64_t grp_q = (args.heads[0] + kHeadGroup - 1) / kHeadGroup;
    int64_t task = blockIdx.x + (args.k_only ? grp_q * nch_q : 0);
    const int which = task < grp_q * nch_q ? 0 : 1;
    if (which) task -= grp_q * nch_q;
    const int64_t len = args.len[which];
    const int64_t heads = args.heads[which];
    const int64_t groups = (heads + kHeadGroup - 1) / kHeadGroup;
    const int64_t chunk = task / groups;
    const int64_t h0 = (task - chunk * groups) * kHeadGroup;
    const int hn = static_cast<int>(min<int64_t>(kHeadGroup, heads - h0));
    const int pack = lane % kPacks;
    const int64_t tok0 = chunk * kChunk + 16 * wave + lane / kPacks;

    bool valid[kItems];
    float rr[kItems];
    u32x4 fa[kItems], fb[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int64_t t = tok0 + kTokStep * i;
        valid[i] = t < len;
        rr[i] = 0.0f;
        if constexpr (kRow) rr[i] = valid[i] ? args.rrms[which][b * len + t] : 0.0f;
        fa[i] = fb[i] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (kRope) {
            if (valid[i]) {
                const uint16_t *frow = args.freqs + (args.f_batches == 1 ? 0 : b) * args.f_sb +
                                       (args.f_len == 1 ? 0 : t) * args.f_sl + pack * 16;
                fa[i] = *reinterpret_cast<const u32x4 *>(frow);
                fb[i] = *reinterpret_cast<const u32x4 *>(frow + 8);
            }
        }
    }
    // the frequency words as fp32, once for all of the group's heads:
    // fr[i][2 j], fr[i][2 j + 1] = (f0, f1) of output channel j of the pack
    float fr[kRope ? kItems : 1][16];
    if constexpr (kRope) {
#pragma unroll
        for (int i = 0; i < kItems; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int pi = j >> 1, comp = j & 1;
                const uint32_t word = (pi < 2 ? fa[i] : fb[i])[(pi & 1) * 2 + comp];
                fr[i][2 * j] = t_to_f32<kFp16>(word & 0xffffu);
                fr[i][2 * j + 1] = t_to_f32<kFp16>(word >> 16);
            }
    }
    const int64_t nt = args.ntiles[which];
    // the group's rows one head ahead: head hh + 1's loads are in flight
    // while head hh is computed
    const uint16_t *xtok = args.x[which] + b * args.x_sb[which] + pack * 8;
    const int64_t x_sh = args.x_sh[which], x_sl = args.x_sl[which];
    auto load_head = [&](int64_t h, u32x4 (&r)[kItems]) {
#pragma unroll
        for (int i = 0; i < kItems; ++i)
            r[i] = valid[i] ? *reinterpret_cast<const u32x4 *>(xtok + h * x_sh + (tok0 + kTokStep * i) * x_sl)
                            : u32x4{0u, 0u, 0u, 0u};
    };
    u32x4 next[kItems];
    load_head(h0, next);
    for (int hh = 0; hh < hn; ++hh) {
        const int64_t h = h0 + hh;
        const u32x4 wraw = *reinterpret_cast<const u32x4 *>(args.norm[which] + (kRow ? h * D : 0) + pack * 8);
        u32x4 raw[kItems];
#pragma unroll
        for (int i = 0; i < kItems; ++i) raw[i] = next[i];
        if (hh + 1 < hn) load_head(h + 1, next);
        float y[kItems][8];
        float amax = 0.0000001f;
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[2 * j] = t_to_f32<kFp16>(raw[i][j] & 0xffffu);
                v[2 * j + 1] = t_to_f32<kFp16>(raw[i][j] >> 16);
            }
            float rrms;
            if constexpr (kRow) {
                rrms = rr[i];
            } else {
                // every lane of the token's pack group takes part, valid or not
                float sq = 0.0f;
#pragma unroll
                for (int c = 0; c < 8; ++c) sq = __builtin_fmaf(v[c], v[c], sq);
                sq = pack_sum<kPacks>(sq);
                rrms = 1.0f / __builtin_sqrtf(sq / static_cast<float>(D) + args.eps);
            }
            float a[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a[2 * j] = (v[2 * j] * rrms) * t_to_f32<kFp16>(wraw[j] & 0xffffu);
                a[2 * j + 1] = (v[2 * j + 1] * rrms) * t_to_f32<kFp16>(wraw[j] >> 16);
                t_round2<kFp16>(a[2 * j], a[2 * j + 1]);
            }
            float pmax = 0.0f;
#pragma unroll
            for (int pi = 0; pi < 4; ++pi) {
                float v0 = a[2 * pi], v1 = a[2 * pi + 1];
                if constexpr (kRope) {
                    // pair pi of the pack: output channel 2 pi + comp takes
                    // row comp of the pair's matrix
                    v0 = __builtin_fmaf(fr[i][4 * pi + 1], a[2 * pi + 1], fr[i][4 * pi] * a[2 * pi]);
                    v1 = __builtin_fmaf(fr[i][4 * pi + 3], a[2 * pi + 1], fr[i][4 * pi + 2] * a[2 * pi]);
                    t_round2<kFp16>(v0, v1);
                }
                y[i][2 * pi] = v0;
                y[i][2 * pi + 1] = v1;
                pmax = max3_abs(pmax, v0, v1);
            }
            if (valid[i]) amax = __int_as_float(max(__float_as_int(amax), __float_as_int(pmax)));
        }
        amax = wave_max_nonneg(amax);
        float inv;
        if (which == 0) {
            if (lane == 0) args.scale[0][(b * heads + h) * nt + chunk * 4 + wave] = amax / 127.0f;
            inv = 127.0f / amax;
        } else {
            if (lane == 0) kamax[hh & 1][wave] = amax;
            __syncthreads();
            float kmax = 0.0000001f;
#pragma unroll
            for (int w = 0; w < kQkThreads / 64; ++w)
                kmax = __int_as_float(max(__float_as_int(kmax), __float_as_int(kamax[hh & 1][w])));
            if (tid == 0) args.scale[1][(b * heads + h) * nt + chunk] = kmax / 127.0f;
            inv = 127.0f / kmax;
        }
        int8_t *obase = args.out[which] + b * args.o_sb[which] + h * args.o_sh[which];
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            if (!valid[i]) continue;
            const u32x2 w2{quant_pack4(y[i][0], y[i][1], y[i][2], y[i][3], inv),
                           quant_pack4(y[i][4], y[i][5], y[i][6], y[i][7], inv)};
            *reinterpret_cast<u32x2 *>(obase + (tok0 + kTokStep * i) * args.o_sl[which] + pack * 8) = w2;
        }
    }
}

// Row-scope Q in one pass over HBM.  A Q scale tile is 16 tokens of one
// head, so one workgroup (4 wave64) takes a 16-token tile of every head:
// wave w owns heads w, w + 4, .. (at most kHPW), each as kItems (token, pack)
// items per lane laid out as in the head-group kernel.  First pass: each
// head's sum of squares per token, computed as the row pre-pass computes it
// (8-channel FMA chain, butterfly across the token's packs), into LDS; the
// first 16 lanes add each token's heads in order and publish rrms.  Second
// pass: every head is read again -- the workgroup's 160 KB (Wan: 40 heads)
// was just read, so this comes from L2 or MALL, not HBM -- then normalized,
// rotated and quantized with the head-group kernel's arithmetic.  Keeping the
// rows in registers instead needs 253 VGPRs, one workgroup per CU, and ran
// slower (0.369 against 0.342 ms for the two-pass path).  K keeps the
// pre-pass: a K scale tile is 64 tokens, and 64 tokens of every head do not
// stay in the caches between two passes.
constexpr int kRowQThreads = 256;

template <bool kFp16, int D, bool kRope, int kHPW>
__global__ __launch_bounds__(kRowQThreads) __attribute__((amdgpu_waves_per_eu(3))) void qk_rowq_kernel(QkArgs args) {
    constexpr int kPacks = D / 8;
    constexpr int kTokStep = 64 / kPacks;   // tokens one lane row of a wave covers
    constexpr int kItems = kQTile / kTokStep;
    constexpr int kWaves = kRowQThreads / 64;
    __shared__ float hsum[kQTile][kWaves * kHPW];
    __shared__ float rr_s[kQTile];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t b = blockIdx.y;
    const int64_t tile = blockIdx.x;
    const int64_t len = args.len[0], heads = args.heads[0];
    const int pack = lane % kPacks, trow = lane / kPacks;
    const int64_t tok0 = tile * kQTile + trow;
    const int64_t x_sh = args.x_sh[0], x_sl = args.x_sl[0];
    const uint16_t *xtok = args.x[0] + b * args.x_sb[0] + pack * 8;

    bool valid[kItems];
    u32x4 fa[kItems], fb[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int64_t t = tok0 + kTokStep * i;
        valid[i] = t < len;
        fa[i] = fb[i] = u32x4{0u, 0u, 0u, 0u};
        if constexpr (kRope) {
            if (valid[i]) {
                const uint16_t *frow = args.freqs + (args.f_batches == 1 ? 0 : b) * args.f_sb +
                                       (args.f_len == 1 ? 0 : t) * args.f_sl + pack * 16;
                fa[i] = *reinterpret_cast<const u32x4 *>(frow);
                fb[i] = *reinterpret_cast<const u32x4 *>(frow + 8);
            }
        }
    }
    auto load_head = [&](int64_t h, u32x4 (&r)[kItems]) {
#pragma unroll
        for (int i = 0; i < kItems; ++i)
            r[i] = valid[i] && h < heads
                       ? *reinterpret_cast<const u32x4 *>(xtok + h * x_sh + (tok0 + kTokStep * i) * x_sl)
                       : u32x4{0u, 0u, 0u, 0u};
    };
    // two head buffers: head k + 1's loads are in flight while head k is used
    u32x4 xr[2][kItems];
    load_head(wave, xr[0]);
#pragma unroll
    for (int k = 0; k < kHPW; ++k) {
        const int h = wave + kWaves * k;
        if (k + 1 < kHPW) load_head(wave + kWaves * (k + 1), xr[(k + 1) & 1]);
        const u32x4 (&xk)[kItems] = xr[k & 1];
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            float sq = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = t_to_f32<kFp16>(xk[i][j] & 0xffffu), hi = t_to_f32<kFp16>(xk[i][j] >> 16);
                sq = __builtin_fmaf(lo, lo, sq);
                sq = __builtin_fmaf(hi, hi, sq);
            }
            sq = pack_sum<kPacks>(sq);
            if (pack == 0 && h < heads) hsum[kTokStep * i + trow][h] = sq;
        }
    }
    __syncthreads();
    if (tid < kQTile) {
        float total = 0.0f;
        for (int h = 0; h < heads; ++h) total = total + hsum[tid][h];
        rr_s[tid] = 1.0f / __builtin_sqrtf(total / static_cast<float>(heads * D) + args.eps);
    }
    __syncthreads();
    float rr[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) rr[i] = rr_s[kTokStep * i + trow];

    const int64_t nt = args.ntiles[0];
    load_head(wave, xr[0]);
#pragma unroll
    for (int k = 0; k < kHPW; ++k) {
        const int64_t h = wave + kWaves * k;
        if (h >= heads) break;
        if (k + 1 < kHPW) load_head(wave + kWaves * (k + 1), xr[(k + 1) & 1]);
        const u32x4 (&xk)[kItems] = xr[k & 1];
        const u32x4 wraw = *reinterpret_cast<const u32x4 *>(args.norm[0] + h * D + pack * 8);
        float y[kItems][8];
        float amax = 0.0000001f;
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            float a[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a[2 * j] = (t_to_f32<kFp16>(xk[i][j] & 0xffffu) * rr[i]) * t_to_f32<kFp16>(wraw[j] & 0xffffu);
                a[2 * j + 1] = (t_to_f32<kFp16>(xk[i][j] >> 16) * rr[i]) * t_to_f32<kFp16>(wraw[j] >> 16);
                t_round2<kFp16>(a[2 * j], a[2 * j + 1]);
            }
            float pmax = 0.0f;
#pragma unroll
            for (int pi = 0; pi < 4; ++pi) {
                float v0 = a[2 * pi], v1 = a[2 * pi + 1];
                if constexpr (kRope) {
                    // row comp of pair pi is word 2 (pi & 1) + comp of fa
                    // (pi < 2) or fb, kept packed to save registers
                    const uint32_t w0 = (pi < 2 ? fa[i] : fb[i])[(pi & 1) * 2];
                    const uint32_t w1 = (pi < 2 ? fa[i] : fb[i])[(pi & 1) * 2 + 1];
                    v0 = __builtin_fmaf(t_to_f32<kFp16>(w0 >> 16), a[2 * pi + 1], t_to_f32<kFp16>(w0 & 0xffffu) * a[2 * pi]);
                    v1 = __builtin_fmaf(t_to_f32<kFp16>(w1 >> 16), a[2 * pi + 1], t_to_f32<kFp16>(w1 & 0xffffu) * a[2 * pi]);
                    t_round2<kFp16>(v0, v1);
                }
                y[i][2 * pi] = v0;
                y[i][2 * pi + 1] = v1;
                pmax = max3_abs(pmax, v0, v1);
            }
            if (valid[i]) amax = __int_as_float(max(__float_as_int(amax), __float_as_int(pmax)));
        }
        amax = wave_max_nonneg(amax);
        if (lane == 0) args.scale[0][(b * heads + h) * nt + tile] = amax / 127.0f;
        const float inv = 127.0f / amax;
        int8_t *obase = args.out[0] + b * args.o_sb[0] + h * args.o_sh[0];
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            if (!valid[i]) continue;
            const u32x2 w2{quant_pack4(y[i][0], y[i][1], y[i][2], y[i][3], inv),
                           quant_pack4(y[i][4], y[i][5], y[i][6], y[i][7], inv)};
            *reinterpret_cast<u32x2 *>(obase + (tok0 + kTokStep * i) * args.o_sl[0] + pack * 8) = w2;
        }
    }
}

// Row-scope Q, streamed (17 to 48 heads): one workgroup of 16 wave64 per CU
// walks 16-token Q tiles (task k, k + grid, .. over batch x tiles), every
// head of a tile at once as in qk_rowq_kernel, but each row is read from HBM
// once and the next tile's reads are in flight while the current tile is
// normalized and quantized.  Wave w owns heads w, w + 16 and w + 32: head w
// arrives in registers (two buffers, alternate tiles), the other two through
// buffer_load ... lds into two LDS regions of the wave's own, each reloaded
// with the next tile's rows as soon as the wave has read it.  Per tile:
// (1) each head's per-token sum of squares, computed as the row pre-pass
// computes it, into LDS; (2) wave t adds token t's heads in order and
// publishes rrms; (3) every head is normalized, rotated and quantized with
// the head-group kernel's arithmetic.  Two barriers a tile.  Buffer offsets
// are 32-bit: the host requires a batch's rows to span less than 2 GiB, and
// rows past the sequence read as zeros (their offsets are past the range).
constexpr int kRowSWaves = 16;
constexpr int kRowSThreads = kRowSWaves * 64;
constexpr int kRowSMaxHeads = 3 * kRowSWaves;
constexpr uint32_t kRowSPast = 0x80000000u;   // an offset past every range

__device__ __forceinline__ u32x4 rows_load16(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
}
// 64 lanes x 16 B into 1 KiB of LDS at `dst` (wave-uniform), lane order.
__device__ __forceinline__ void rows_load16_lds(__amdgpu_buffer_rsrc_t rs, int8_t *dst, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16, off, 0, 0, 0);
}

template <bool kFp16, int D, bool kRope>
__global__ __launch_bounds__(kRowSThreads) void qk_rowq_stream_kernel(QkArgs args, uint32_t ntasks, uint32_t span,
                                                                    uint32_t f_span) {
    constexpr int kPacks = D / 8;
    constexpr int kTokStep = 64 / kPacks;   // tokens one lane row of a wave covers
    constexpr int kItems = kQTile / kTokStep;
    constexpr int kHeadBytes = kItems * 1024;
    __shared__ __align__(1024) int8_t ring[2 * kRowSWaves * kHeadBytes];
    __shared__ __align__(16) float hsum[kQTile][kRowSMaxHeads];
    __shared__ float rr_s[kQTile];
    // The tile's frequency rows: fstage receives them as stored (chunk 2 i + c
    // holds lane l's 16 bytes c of item i's row segment), fconv holds them
    // as fp32, converted once per tile for all heads (chunk 4 i + p holds
    // pair p's 2x2 row-major matrix of lane l's item i).
    constexpr int kStageBytes = kRope ? 2 * kItems * 1024 : 16;
    constexpr int kConvBytes = kRope ? 4 * kItems * 1024 : 16;
    __shared__ __align__(1024) int8_t fstage[kStageBytes];
    __shared__ __align__(1024) int8_t fconv[kConvBytes];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // 32-bit task arithmetic: batch x tiles < 2^31 (checked on the host)
    const uint32_t len = static_cast<uint32_t>(args.len[0]), heads = static_cast<uint32_t>(args.heads[0]);
    const uint32_t nt = static_cast<uint32_t>(args.ntiles[0]);
    const int pack = lane % kPacks, trow = lane / kPacks;
    const uint32_t x_sh2 = static_cast<uint32_t>(args.x_sh[0] * 2), x_sl2 = static_cast<uint32_t>(args.x_sl[0] * 2);
    int8_t *const region[2] = {ring + wave * kHeadBytes, ring + (kRowSWaves + wave) * kHeadBytes};
    const uint32_t nheads_w = (heads - wave + kRowSWaves - 1) / kRowSWaves;
    const int nmine = static_cast<int>(nheads_w < 3u ? nheads_w : 3u);

    // the task's rows: head `wave` into xa, the wave's other heads into its
    // LDS regions; `from` selects which of those (0 registers, 1 + r region r)
    auto issue_rows = [&](uint32_t task, int from, int upto, u32x4 (&xa)[kItems]) {
        const uint32_t b = task / nt, tile = task - b * nt;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(args.x[0] + b * args.x_sb[0], span);
        uint32_t off[kItems];
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const uint32_t t = tile * kQTile + trow + kTokStep * i;
            off[i] = t < len ? t * x_sl2 + pack * 16 : kRowSPast;
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            if (k < from || k >= upto) continue;
            const uint32_t hoff = static_cast<uint32_t>(wave + kRowSWaves * k) * x_sh2;
            if (k == 0) {
#pragma unroll
                for (int i = 0; i < kItems; ++i) xa[i] = rows_load16(rs, off[i] + hoff);
            } else {
#pragma unroll
                for (int i = 0; i < kItems; ++i) rows_load16_lds(rs, region[k - 1] + i * 1024, off[i] + hoff);
            }
        }
    };
    // wave n < 2 kItems loads chunk n of the task's frequency rows
    auto issue_freqs = [&](uint32_t task) {
        if constexpr (kRope) {
            if (wave < 2 * kItems) {
                const uint32_t b = task / nt, tile = task - b * nt;
                const __amdgpu_buffer_rsrc_t rs =
                    make_rsrc(args.freqs + (args.f_batches == 1 ? 0 : b) * args.f_sb, f_span);
                const int i = wave >> 1;
                const uint32_t t = tile * kQTile + trow + kTokStep * i;
                const uint32_t off = t >= len ? kRowSPast
                                              : (args.f_len == 1 ? 0u : t) * static_cast<uint32_t>(args.f_sl * 2) +
                                                    pack * 32 + (wave & 1) * 16;
                rows_load16_lds(rs, fstage + wave * 1024, off);
            }
        }
    };
    auto read_region = [&](int r, u32x4 (&xk)[kItems]) {
#pragma unroll
        for (int i = 0; i < kItems; ++i)
            xk[i] = *reinterpret_cast<const u32x4 *>(region[r] + i * 1024 + lane * 16);
    };

    auto run = [&](uint32_t task, u32x4 (&xa)[kItems], u32x4 (&xa_next)[kItems]) {
        const uint32_t b = task / nt, tile = task - b * nt;
        const uint32_t next = task + gridDim.x;
        const bool more = next < ntasks;
        bool valid[kItems];
#pragma unroll
        for (int i = 0; i < kItems; ++i) valid[i] = tile * kQTile + trow + kTokStep * i < len;
        // this task's rows (and frequencies) have arrived
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        // (1) per-head sums of squares
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            if (k >= nmine) break;
            const int h = wave + kRowSWaves * k;
            u32x4 xk[kItems];
            if (k == 0) {
#pragma unroll
                for (int i = 0; i < kItems; ++i) xk[i] = xa[i];
            } else {
                read_region(k - 1, xk);
            }
#pragma unroll
            for (int i = 0; i < kItems; ++i) {
                float sq = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float lo = t_to_f32<kFp16>(xk[i][j] & 0xffffu), hi = t_to_f32<kFp16>(xk[i][j] >> 16);
                    sq = __builtin_fmaf(lo, lo, sq);
                    sq = __builtin_fmaf(hi, hi, sq);
                }
                sq = pack_sum<kPacks>(sq);
                if (pack == 0) hsum[kTokStep * i + trow][h] = sq;
            }
        }
        __syncthreads();
        if constexpr (kRope) {
            // every wave is past the last tile's reads of fconv, and this
            // tile's rows are in fstage
            if (tid < 4 * kItems * 64) {
                const int i = tid >> 8, p = (tid >> 6) & 3, l = tid & 63;
                const u32x2 w = *reinterpret_cast<const u32x2 *>(fstage + (2 * i + (p >> 1)) * 1024 + l * 16 +
                                                                 (p & 1) * 8);
                *reinterpret_cast<f32x4 *>(fconv + (4 * i + p) * 1024 + l * 16) =
                    f32x4{t_to_f32<kFp16>(w[0] & 0xffffu), t_to_f32<kFp16>(w[0] >> 16),
                          t_to_f32<kFp16>(w[1] & 0xffffu), t_to_f32<kFp16>(w[1] >> 16)};
            }
        }
        // (2) wave t: token t's heads in order
        {
            float total = 0.0f;
            for (uint32_t h = 0; h < heads; ++h) total = total + hsum[wave][h];
            if (lane == 0) rr_s[wave] = 1.0f / __builtin_sqrtf(total / static_cast<float>(heads * D) + args.eps);
        }
        __syncthreads();
        float rr[kItems];
#pragma unroll
        for (int i = 0; i < kItems; ++i) rr[i] = rr_s[kTokStep * i + trow];

        // (3) normalize, rotate, quantize; the next task's loads go out as
        // each head's source is free.  The LDS heads go first, so their
        // regions are refilled early; the register head (double-buffered)
        // goes last.
        // fstage was read before the barrier above
        if (more) issue_freqs(next);
#pragma unroll
        for (int kk = 0; kk < 3; ++kk) {
            const int k = (kk + 1) % 3;
            if (k >= nmine) continue;
            if (k == 0 && more) issue_rows(next, 0, 1, xa_next);
            const uint32_t h = wave + kRowSWaves * k;
            const u32x4 wraw = *reinterpret_cast<const u32x4 *>(args.norm[0] + h * D + pack * 8);
            float y[kItems][8];
            float amax = 0.0000001f;
#pragma unroll
            for (int i = 0; i < kItems; ++i) {
                const u32x4 xi = k == 0 ? xa[i] : *reinterpret_cast<const u32x4 *>(region[k - 1] + i * 1024 + lane * 16);
                float a[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    a[2 * j] = (t_to_f32<kFp16>(xi[j] & 0xffffu) * rr[i]) * t_to_f32<kFp16>(wraw[j] & 0xffffu);
                    a[2 * j + 1] = (t_to_f32<kFp16>(xi[j] >> 16) * rr[i]) * t_to_f32<kFp16>(wraw[j] >> 16);
                    t_round2<kFp16>(a[2 * j], a[2 * j + 1]);
                }
                float pmax = 0.0f;
#pragma unroll
                for (int pi = 0; pi < 4; ++pi) {
                    float v0 = a[2 * pi], v1 = a[2 * pi + 1];
                    if constexpr (kRope) {
                        const f32x4 f = *reinterpret_cast<const f32x4 *>(fconv + (4 * i + pi) * 1024 + lane * 16);
                        v0 = __builtin_fmaf(f[1], a[2 * pi + 1], f[0] * a[2 * pi]);
                        v1 = __builtin_fmaf(f[3], a[2 * pi + 1], f[2] * a[2 * pi]);
                        t_round2<kFp16>(v0, v1);
                    }
                    y[i][2 * pi] = v0;
                    y[i][2 * pi + 1] = v1;
                    pmax = max3_abs(pmax, v0, v1);
                }
                if (valid[i]) amax = __int_as_float(max(__float_as_int(amax), __float_as_int(pmax)));
            }
            amax = wave_max_nonneg(amax);
            if (k > 0 && more) {
                // the region's reads have returned before it is refilled
                __builtin_amdgcn_s_waitcnt(lgkmcnt_imm(0));
                issue_rows(next, k, k + 1, xa_next);
            }
            if (lane == 0) args.scale[0][(static_cast<int64_t>(b) * heads + h) * nt + tile] = amax / 127.0f;
            const float inv = 127.0f / amax;
            int8_t *obase = args.out[0] + b * args.o_sb[0] + h * args.o_sh[0];
#pragma unroll
            for (int i = 0; i < kItems; ++i) {
                if (!valid[i]) continue;
                const u32x2 w2{quant_pack4(y[i][0], y[i][1], y[i][2], y[i][3], inv),
                               quant_pack4(y[i][4], y[i][5], y[i][6], y[i][7], inv)};
                *reinterpret_cast<u32x2 *>(obase + (tile * kQTile + trow + kTokStep * i) * args.o_sl[0] + pack * 8) = w2;
            }
        }
    };

    uint32_t task = blockIdx.x;
    if (task >= ntasks) return;
    u32x4 xa0[kItems], xa1[kItems];
    issue_rows(task, 0, nmine, xa0);
    issue_freqs(task);
    for (;;) {
        run(task, xa0, xa1);
        task += gridDim.x;
        if (task >= ntasks) break;
        run(task, xa1, xa0);
        task += gridDim.x;
        if (task >= ntasks) break;
    }
}

// Row-scope rrms, batched: one wave per 64 / P tokens (P = D / 8 packs a
// token), four waves a workgroup, Q tokens then K tokens.  Each lane group of
// P lanes owns a token; the heads' loads go out kRrmsBatch at a time, and the
// per-head sums are the general pre-pass's (8-channel FMA chain, butterfly
// across the packs), added to the token's total in head order.
constexpr int kRrmsBatch = 8;

template <bool kFp16, int D>
__global__ __launch_bounds__(kQkThreads) void row_rrms_batched_kernel(QkArgs args) {
    constexpr int kPacks = D / 8;
    constexpr int kTokPerWave = 64 / kPacks;
    constexpr int kTokPerBlock = kTokPerWave * kQkThreads / 64;
    const int tid = threadIdx.x, lane = tid & 63;
    const int64_t b = blockIdx.y;
    const int64_t nblk_q = (args.len[0] + kTokPerBlock - 1) / kTokPerBlock;
    int64_t blk = blockIdx.x + (args.k_only ? nblk_q : 0);
    const int which = blk < nblk_q ? 0 : 1;
    if (which) blk -= nblk_q;
    const int64_t len = args.len[which];
    const int64_t t = blk * kTokPerBlock + (tid >> 6) * kTokPerWave + lane / kPacks;
    const int pack = lane % kPacks;
    const bool valid = t < len;
    const int64_t heads = args.heads[which];
    const uint16_t *xrow = args.x[which] + b * args.x_sb[which] + (valid ? t : 0) * args.x_sl[which] + pack * 8;
    float total = 0.0f;
    // one batch of heads ahead: batch n + 1's loads are in flight while
    // batch n is summed
    const int64_t x_sh = args.x_sh[which];
    auto load_batch = [&](int64_t h0, u32x4 (&r)[kRrmsBatch]) {
#pragma unroll
        for (int g = 0; g < kRrmsBatch; ++g)
            r[g] = valid && h0 + g < heads ? *reinterpret_cast<const u32x4 *>(xrow + (h0 + g) * x_sh)
                                           : u32x4{0u, 0u, 0u, 0u};
    };
    u32x4 next[kRrmsBatch];
    load_batch(0, next);
    for (int64_t h0 = 0; h0 < heads; h0 += kRrmsBatch) {
        u32x4 raw[kRrmsBatch];
#pragma unroll
        for (int g = 0; g < kRrmsBatch; ++g) raw[g] = next[g];
        if (h0 + kRrmsBatch < heads) load_batch(h0 + kRrmsBatch, next);
#pragma unroll
        for (int g = 0; g < kRrmsBatch; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float lo = t_to_f32<kFp16>(raw[g][j] & 0xffffu), hi = t_to_f32<kFp16>(raw[g][j] >> 16);
                s = __builtin_fmaf(lo, lo, s);
                s = __builtin_fmaf(hi, hi, s);
            }
            s = pack_sum<kPacks>(s);
            if (h0 + g < heads) total = total + s;
        }
    }
    if (valid && pack == 0) {
        const float r = 1.0f / __builtin_sqrtf(total / static_cast<float>(heads * D) + args.eps);
        args.rrms[which][b * len + t] = r;
    }
}

// processed_value (qk_preprocess.cu:97-145) of channel c of K row xrow:
// RMSNorm then RoPE, rounded to the input type, with strided frequencies.
template <bool kFp16, bool kSplit>
__device__ __forceinline__ float processed_value(const QkArgs &args, const uint16_t *xrow, const uint16_t *norm,
                                                 int c, float rrms, int64_t b, int64_t t) {
    const float ac = t_round<kFp16>((t_to_f32<kFp16>(xrow[c]) * rrms) * t_to_f32<kFp16>(norm[c]));
    if (c >= args.rot_dim) return ac;
    const int pairs = args.rot_dim / 2;
    const int pair = kSplit ? (c < pairs ? c : c - pairs) : c >> 1;
    const int first = kSplit ? pair : 2 * pair;
    const int second = kSplit ? pair + pairs : first + 1;
    const int comp = kSplit ? (c >= pairs) : (c & 1);
    const float x0 = t_round<kFp16>((t_to_f32<kFp16>(xrow[first]) * rrms) * t_to_f32<kFp16>(norm[first]));
    const float x1 = t_round<kFp16>((t_to_f32<kFp16>(xrow[second]) * rrms) * t_to_f32<kFp16>(norm[second]));
    const uint16_t *fp = args.freqs + (args.f_batches == 1 ? 0 : b) * args.f_sb + (args.f_len == 1 ? 0 : t) * args.f_sl +
                         pair * args.f_sp + comp * args.f_sr;
    const float f0 = t_to_f32<kFp16>(fp[0]);
    const float f1 = t_to_f32<kFp16>(fp[args.f_sc]);
    return t_round<kFp16>(__builtin_fmaf(f1, x1, f0 * x0));
}

// K anchor of the fused producer (detect_anchor_kernel, qk_preprocess.cu
// :250-416): one 128-thread workgroup per (K head, batch).  The nine samples
// are processed values; their rrms is the row-scope pre-pass value, or for
// the head scope 1 / sqrt(S / D + eps) with S a sequential fma chain over the
// head's channels (the reference's order; it takes rsqrtf, here IEEE).
template <bool kFp16, int D, bool kSplit, bool kRow>
__global__ __launch_bounds__(kAnchorThreads) void qk_anchor_kernel(QkArgs args) {
    __shared__ float samples[kAnchorSamples][128];
    __shared__ float rr[kAnchorSamples];
    const int c = threadIdx.x;
    const int64_t head = blockIdx.x, b = blockIdx.y;
    const int64_t len = args.len[1];
    const uint16_t *xbase = args.x[1] + b * args.x_sb[1] + head * args.x_sh[1];
    const uint16_t *norm = args.norm[1] + (kRow ? head * D : 0);
    if (c < kAnchorSamples) {
        const int64_t t = static_cast<int64_t>(c) * (len - 1) / (kAnchorSamples - 1);
        if constexpr (kRow) {
            rr[c] = args.rrms[1][b * len + t];
        } else {
            const uint16_t *xrow = xbase + t * args.x_sl[1];
            float sq = 0.0f;
            for (int ch = 0; ch < D; ++ch) {
                const float v = t_to_f32<kFp16>(xrow[ch]);
                sq = __builtin_fmaf(v, v, sq);
            }
            rr[c] = 1.0f / __builtin_sqrtf(sq / static_cast<float>(D) + args.eps);
        }
    }
    __syncthreads();
#pragma unroll
    for (int sm = 0; sm < kAnchorSamples; ++sm) {
        const int64_t t = static_cast<int64_t>(sm) * (len - 1) / (kAnchorSamples - 1);
        samples[sm][c] = c < D ? processed_value<kFp16, kSplit>(args, xbase + t * args.x_sl[1], norm, c, rr[sm], b, t)
                               : 0.0f;
    }
    __syncthreads();
    const int sel = w8a8_anchor_decide(samples, D);
    const int64_t bh = b * args.heads[1] + head;
    if (c == 0)
        const_cast<int32_t *>(args.anchors)[bh] =
            sel >= 0 ? static_cast<int32_t>(static_cast<int64_t>(sel) * (len - 1) / (kAnchorSamples - 1)) : -1;
    if (c < D) args.anchor_values[bh * D + c] = sel >= 0 ? samples[sel][c] : 0.0f;
}

template <bool kFp16, int D, bool kRotate>
void launch_quant(const QkArgs &args, dim3 grid, bool split, bool row, hipStream_t s) {
    if (split) {
        if (row) qk_rope_quant_kernel<kFp16, D, true, true, kRotate><<<grid, kQkThreads, 0, s>>>(args);
        else qk_rope_quant_kernel<kFp16, D, true, false, kRotate><<<grid, kQkThreads, 0, s>>>(args);
    } else {
        if (row) qk_rope_quant_kernel<kFp16, D, false, true, kRotate><<<grid, kQkThreads, 0, s>>>(args);
        else qk_rope_quant_kernel<kFp16, D, false, false, kRotate><<<grid, kQkThreads, 0, s>>>(args);
    }
}

template <bool kFp16, int D>
int32_t launch_qk(const QkArgs &args, int64_t batch, bool split, bool row, bool rotate, hipStream_t s) {
    // interleaved RoPE over the whole head (contiguous frequencies) or none,
    // no rotation: the head-group fast path
    const bool fast = !rotate && !split && (args.rot_dim == 0 || (args.rot_dim == D && args.f_contig));
    // the streamed Q kernel: a batch's Q rows within 2 GiB of 32-bit offsets
    // (non-negative head, token and frequency strides)
    const bool q_strides_ok = args.x_sh[0] >= 0 && args.x_sl[0] >= 0 && (args.rot_dim == 0 || args.f_sl >= 0);
    const int64_t q_span = ((args.heads[0] - 1) * args.x_sh[0] + (args.len[0] - 1) * args.x_sl[0] + D) * 2;
    // and its frequency rows (one batch of them) likewise
    const int64_t f_span = args.rot_dim == 0 ? 0 : ((args.f_len - 1) * args.f_sl + 2 * D) * 2;
    const bool stream = fast && row && q_strides_ok && args.heads[0] > 16 && args.heads[0] <= kRowSMaxHeads &&
                        q_span < (1ll << 31) &&
                        f_span < (1ll << 31) && args.ntiles[0] * batch < (1ll << 31);
    if (fast && row && (stream || args.heads[0] <= 40)) {
        // Q in one pass; K: its row pre-pass, then the head-group kernel
        QkArgs ka = args;
        ka.k_only = 1;
        constexpr int kTokPerBlock = 64 / (D / 8) * kQkThreads / 64;
        const dim3 gr(static_cast<unsigned>((args.len[1] + kTokPerBlock - 1) / kTokPerBlock),
                      static_cast<unsigned>(batch));
        row_rrms_batched_kernel<kFp16, D><<<gr, kQkThreads, 0, s>>>(ka);
        if (stream) {
            int cus = 0;
            if (device_cus(cus)) return -1;
            const uint32_t ntasks = static_cast<uint32_t>(args.ntiles[0] * batch);
            const unsigned grid = ntasks < static_cast<uint32_t>(cus) ? ntasks : static_cast<unsigned>(cus);
            const uint32_t span = static_cast<uint32_t>(q_span);
            if (args.rot_dim == 0)
                qk_rowq_stream_kernel<kFp16, D, false><<<grid, kRowSThreads, 0, s>>>(args, ntasks, span, 0u);
            else
                qk_rowq_stream_kernel<kFp16, D, true><<<grid, kRowSThreads, 0, s>>>(args, ntasks, span,
                                                                                   static_cast<uint32_t>(f_span));
        } else {
            const dim3 gq(static_cast<unsigned>(args.ntiles[0]), static_cast<unsigned>(batch));
            const bool small = args.heads[0] <= 16;
            constexpr int kSmall = 16 / (kRowQThreads / 64), kLarge = 40 / (kRowQThreads / 64);
#define TU_ROWQ(R) \
    if (small) qk_rowq_kernel<kFp16, D, R, kSmall><<<gq, kRowQThreads, 0, s>>>(args); \
    else qk_rowq_kernel<kFp16, D, R, kLarge><<<gq, kRowQThreads, 0, s>>>(args)
            if (args.rot_dim == 0) { TU_ROWQ(false); }
            else { TU_ROWQ(true); }
#undef TU_ROWQ
        }
        const int64_t gk = (args.heads[1] + kHeadGroup - 1) / kHeadGroup;
        const dim3 grid(static_cast<unsigned>(gk * ((args.len[1] + kChunk - 1) / kChunk)), static_cast<unsigned>(batch));
        if (args.rot_dim == 0) qk_rope_quant_heads_kernel<kFp16, D, true, false><<<grid, kQkThreads, 0, s>>>(ka);
        else qk_rope_quant_heads_kernel<kFp16, D, true, true><<<grid, kQkThreads, 0, s>>>(ka);
        return check_launch("tu_qk_rms_rope_int8");
    }
    if (row) {
        constexpr int kTokPerBlock = 64 / (D / 8) * kQkThreads / 64;
        const dim3 g(static_cast<unsigned>((args.len[0] + kTokPerBlock - 1) / kTokPerBlock +
                                           (args.len[1] + kTokPerBlock - 1) / kTokPerBlock),
                     static_cast<unsigned>(batch));
        row_rrms_batched_kernel<kFp16, D><<<g, kQkThreads, 0, s>>>(args);
    }
    if (fast) {
        const int64_t gq = (args.heads[0] + kHeadGroup - 1) / kHeadGroup;
        const int64_t gk = (args.heads[1] + kHeadGroup - 1) / kHeadGroup;
        const dim3 grid(static_cast<unsigned>(gq * ((args.len[0] + kChunk - 1) / kChunk) +
                                              gk * ((args.len[1] + kChunk - 1) / kChunk)),
                        static_cast<unsigned>(batch));
        if (args.rot_dim == 0) {
            if (row) qk_rope_quant_heads_kernel<kFp16, D, true, false><<<grid, kQkThreads, 0, s>>>(args);
            else qk_rope_quant_heads_kernel<kFp16, D, false, false><<<grid, kQkThreads, 0, s>>>(args);
        } else {
            if (row) qk_rope_quant_heads_kernel<kFp16, D, true, true><<<grid, kQkThreads, 0, s>>>(args);
            else qk_rope_quant_heads_kernel<kFp16, D, false, true><<<grid, kQkThreads, 0, s>>>(args);
        }
        return check_launch("tu_qk_rms_rope_int8");
    }
    if (args.anchors != nullptr) {
        const dim3 ga(static_cast<unsigned>(args.heads[1]), static_cast<unsigned>(batch));
        if (split) {
            if (row) qk_anchor_kernel<kFp16, D, true, true><<<ga, kAnchorThreads, 0, s>>>(args);
            else qk_anchor_kernel<kFp16, D, true, false><<<ga, kAnchorThreads, 0, s>>>(args);
        } else {
            if (row) qk_anchor_kernel<kFp16, D, false, true><<<ga, kAnchorThreads, 0, s>>>(args);
            else qk_anchor_kernel<kFp16, D, false, false><<<ga, kAnchorThreads, 0, s>>>(args);
        }
    }
    // one workgroup per 64-token chunk of each head: ntiles is 4 chunks' worth for Q, one for K
    const dim3 grid(static_cast<unsigned>(args.heads[0] * (args.ntiles[0] / 4) + args.heads[1] * args.ntiles[1]),
                    static_cast<unsigned>(batch));
    if (rotate) launch_quant<kFp16, D, true>(args, grid, split, row, s);
    else launch_quant<kFp16, D, false>(args, grid, split, row, s);
    return check_launch("tu_qk_rms_rope_int8");
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_qk_rms_rope_int8(
    const void *q, const void *k, int32_t dtype, int64_t batch, int64_t hq, int64_t hk, int64_t lq, int64_t lk,
    int64_t dim, int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb, int64_t k_sh, int64_t k_sl,
    const void *q_norm, const void *k_norm, int32_t norm_scope, float eps, const void *freqs, int64_t rot_dim,
    int32_t split_half, int64_t f_batches, int64_t f_len, int64_t f_sb, int64_t f_sl, int64_t f_sp, int64_t f_sr,
    int64_t f_sc, float *q_rrms, float *k_rrms, int8_t *q8, int64_t qo_sb, int64_t qo_sh, int64_t qo_sl,
    int8_t *k8, int64_t ko_sb, int64_t ko_sh, int64_t ko_sl, float *q_scale, float *k_scale, int32_t rotate,
    int32_t *anchors, float *anchor_values, void *stream) {
    using namespace tu;
    TU_REQUIRE(dtype == 0 || dtype == 1, "Q/K preprocessing dtype must be 0 (bf16) or 1 (fp16), got %d", dtype);
    TU_REQUIRE(dim == 64 || dim == 128, "Q/K preprocessing requires head_dim 64 or 128, got %lld",
               static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && batch <= 65535 && hq > 0 && hk > 0 && lq > 0 && lk > 0,
               "Q/K preprocessing dimensions must be positive");
    TU_REQUIRE(norm_scope == 0 || norm_scope == 1, "norm_scope must be 0 (head) or 1 (row)");
    TU_REQUIRE(rot_dim >= 0 && rot_dim <= dim && rot_dim % 2 == 0, "rot_dim must be even and within head_dim");
    TU_REQUIRE(q && k && q_norm && k_norm && q8 && k8 && q_scale && k_scale, "Q/K preprocessing pointers must be non-null");
    TU_REQUIRE(rot_dim == 0 || freqs, "RoPE frequencies are required when rot_dim > 0");
    TU_REQUIRE(rot_dim == 0 || ((f_batches == 1 || f_batches == batch) &&
                                (f_len == 1 || (f_len == lq && lq == lk))),
               "RoPE batch/sequence broadcasting is incompatible");
    TU_REQUIRE(norm_scope == 0 || (q_rrms && k_rrms), "row-scope RMSNorm needs rrms scratch");
    TU_REQUIRE((anchors == nullptr) == (anchor_values == nullptr), "K anchors need both the index and value buffers");
    TU_REQUIRE(anchors == nullptr || rotate, "K stabilisation is part of the rotated (W8A8) variant");
    const auto aligned16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    TU_REQUIRE(aligned16(q) && aligned16(k) && aligned16(q_norm) && aligned16(k_norm) && q_sl % 8 == 0 &&
                   q_sh % 8 == 0 && q_sb % 8 == 0 && k_sl % 8 == 0 && k_sh % 8 == 0 && k_sb % 8 == 0,
               "Q/K preprocessing inputs must be 16-byte aligned rows");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(q8) & 7) == 0 && (reinterpret_cast<uintptr_t>(k8) & 7) == 0 &&
                   qo_sl % 8 == 0 && qo_sh % 8 == 0 && qo_sb % 8 == 0 && ko_sl % 8 == 0 && ko_sh % 8 == 0 &&
                   ko_sb % 8 == 0,
               "Q/K preprocessing outputs must be 8-byte aligned rows");
    const int64_t nqt = (lq + 63) / 64 * 4, nkt = (lk + 63) / 64;
    TU_REQUIRE(hq * nqt + hk * nkt < 0x7fffffff && lq + lk < 0x7fffffff, "Q/K preprocessing grid too large");
    if (require_gfx950()) return -1;
    QkArgs a{};
    a.x[0] = static_cast<const uint16_t *>(q);
    a.x[1] = static_cast<const uint16_t *>(k);
    a.norm[0] = static_cast<const uint16_t *>(q_norm);
    a.norm[1] = static_cast<const uint16_t *>(k_norm);
    a.rrms[0] = q_rrms;
    a.rrms[1] = k_rrms;
    a.out[0] = q8;
    a.out[1] = k8;
    a.scale[0] = q_scale;
    a.scale[1] = k_scale;
    a.freqs = static_cast<const uint16_t *>(freqs);
    a.heads[0] = hq;
    a.heads[1] = hk;
    a.len[0] = lq;
    a.len[1] = lk;
    a.x_sb[0] = q_sb, a.x_sh[0] = q_sh, a.x_sl[0] = q_sl;
    a.x_sb[1] = k_sb, a.x_sh[1] = k_sh, a.x_sl[1] = k_sl;
    a.o_sb[0] = qo_sb, a.o_sh[0] = qo_sh, a.o_sl[0] = qo_sl;
    a.o_sb[1] = ko_sb, a.o_sh[1] = ko_sh, a.o_sl[1] = ko_sl;
    a.ntiles[0] = nqt;
    a.ntiles[1] = nkt;
    a.f_sb = f_sb, a.f_sl = f_sl, a.f_sp = f_sp, a.f_sr = f_sr, a.f_sc = f_sc;
    a.f_batches = f_batches;
    a.f_contig = rot_dim > 0 && f_sc == 1 && f_sr == 2 && f_sp == 4 && f_sl % 8 == 0 && f_sb % 8 == 0 &&
                 (reinterpret_cast<uintptr_t>(freqs) & 15) == 0;
    a.f_len = f_len;
    a.rot_dim = static_cast<int>(rot_dim);
    a.eps = eps;
    a.anchors = anchors;
    a.anchor_values = anchor_values;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool split = split_half != 0, row = norm_scope == 1;
    const bool rot = rotate != 0;
    if (dtype == 1)
        return dim == 128 ? launch_qk<true, 128>(a, batch, split, row, rot, s) : launch_qk<true, 64>(a, batch, split, row, rot, s);
    return dim == 128 ? launch_qk<false, 128>(a, batch, split, row, rot, s)
                      : launch_qk<false, 64>(a, batch, split, row, rot, s);
}
