// Sage INT8 attention forward for gfx950: INT8 QK^T on MFMA, online softmax
// in base 2, P rounded to bf16, PV on bf16 MFMA with fp32 accumulation.
//
// Reference semantics: qk_int_sv_f16_attn_kernel
// (kernel/csrc/turing/sage/qk_int_sv_f16_cuda_sm75.cu:48-830) with
// update_mdo / normalize_d (sage/attn_utils.cuh:464-568, :920-973):
//   s   = float(q8 . k8) * (sm_scale * log2 e) * q_scale * k_scale
//   p   = 2^(s - m) with m a running row maximum, O = O * 2^(m_old - m) + P V
//   out = O / sum(p)
// The reference rounds P to fp16 for its Turing fp16 MMA; here P is rounded
// to bf16 for the CDNA4 bf16 MFMA.
//
// MI355X mapping
//   * Workgroup = 4 wave64 = 64 QT query rows (16 QT per wave, QT = 2 by
//     default) of one (batch, head); two workgroups per CU (256 registers per
//     lane each), so the two waves sharing a SIMD overlap one's softmax VALU
//     work with the other's MFMAs.
//   * Keys stream in tiles of 64 through a 3-stage LDS ring (24 KiB a stage)
//     filled with global_load_lds_dwordx4 (no staging registers), two tiles
//     ahead of the MFMAs.  For pairs of unmasked tiles the QK^T of the next
//     tile is issued before the softmax and PV of the current one.  V arrives
//     pre-transposed (V^T, [d][key], keys padded to a multiple of 64 with
//     zeros) from tu_sage_v_prep, so every MFMA operand is a plain LDS read.
//   * Each tile is processed in two 32-key halves.  S^T = K Q^T runs on
//     v_mfma_i32_16x16x64_i8 with the wave's Q rows resident as the B
//     operand; a lane then holds 4 keys x 1 query per 16x16 block, so the row
//     max is an integer max3 tree plus two cross-lane steps.  O^T = V^T P runs
//     on v_mfma_f32_16x16x32_bf16 with P taken straight from registers.
//   * Masking (Lk tail, causal diagonal) is compiled only into the tiles
//     that need it.  The O rescale is lazy: the exponent base m_used only
//     moves when a row maximum exceeds it by more than 8 (p <= 2^8), which
//     after the first tiles is rare.
//   * LDS rows are 128 B with 16-byte chunks XOR-swizzled by row bits 1..3,
//     conflict-free for the 16 lanes that read one chunk column.
#include <type_traits>

#ifndef TU_ATTN_QT
#define TU_ATTN_QT 2
#endif

#include "tu_common.h"

namespace tu {
namespace {

constexpr int kThreads = 256;
constexpr int kD = 128;
// Query rows per wave = 16 * QT (template parameter); 4 waves per workgroup.
constexpr int kBKey = 64;     // keys per tile
constexpr int kKTileBytes = kBKey * kD;      // int8 K tile, 8 KiB
constexpr int kVTileBytes = kD * kBKey * 2;  // bf16 V^T tile, 16 KiB
constexpr int kStageBytes = kKTileBytes + kVTileBytes;
constexpr int kStages = 3;                   // LDS ring: current tile plus two in flight
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleSlack = 8.0f;        // log2 of the largest p allowed

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt immediate that waits until at most n vector-memory operations are
// outstanding and leaves the other counters alone (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_imm(int n) { return (n & 0xf) | (0x7 << 4) | (0xf << 8) | ((n >> 4) << 14); }

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

__device__ __forceinline__ int imax3(int a, int b, int c) { return max(max(a, b), c); }

// K tile LDS row p holds key kperm(p): within each 32-key half, row
// 16 kt + i holds key 8 (i >> 2) + 4 kt + (i & 3).  The QK MFMA reads 16
// consecutive rows per 16-key block, so output row 4 g + r of block kt (of
// half h) is key 32 h + 8 g + 4 (kt & 1) + r, and each lane group g owns the
// 8 contiguous keys 32 h + 8 g .. +7: exactly one 16-byte V^T chunk.
__device__ __forceinline__ int kperm(int p) {
    const int i = p & 15, kt = (p >> 4) & 1;
    return (p & ~31) + 8 * (i >> 2) + 4 * kt + (i & 3);
}

// Per-lane constants of the tile loads and the MFMA operand reads.
struct LaneGeom {
    int k_row[2];        // K tile LDS row filled by this lane's two loads
    uint32_t k_src[2];   // kperm(row) and byte offset of the source chunk
    uint32_t v_src[4];   // byte offset of this lane's four V^T source chunks
    uint32_t k_rd[2];    // LDS byte offset of the K operand, chunk g / 4 + g
    uint32_t v_rd[2];    // LDS byte offset of the V^T operand, half 0 / 1
};

__device__ __forceinline__ LaneGeom lane_geom(int wave, int lane, int64_t lpad) {
    LaneGeom gm;
    const int g = lane >> 4, lc = lane & 15, sw = (lc >> 1) & 7;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = (2 * wave + i) * 8 + (lane >> 3);
        gm.k_row[i] = kperm(row);
        gm.k_src[i] = static_cast<uint32_t>(((lane & 7) ^ ((row >> 1) & 7)) * 16);
        gm.k_rd[i] = static_cast<uint32_t>(lc * 128 + (((4 * i + g) ^ sw) << 4));
        gm.v_rd[i] = static_cast<uint32_t>(kKTileBytes + lc * 128 + (((4 * i + g) ^ sw) << 4));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = (4 * wave + i) * 8 + (lane >> 3);
        gm.v_src[i] = static_cast<uint32_t>((d * lpad + ((lane & 7) ^ ((d >> 1) & 7)) * 8) * 2);
    }
    return gm;
}

// Direct-to-LDS loads of the K and V^T tiles at key0 into one ring stage.
// Each global_load_lds_dwordx4 moves 64 lanes x 16 B into 1 KiB of contiguous
// LDS; the row permutation and chunk swizzle come from the source offsets.
__device__ __forceinline__ void issue_tile(int8_t *stage, const int8_t *__restrict__ kp,
                                           const uint16_t *__restrict__ vtp, const LaneGeom &gm, int64_t k_sl,
                                           int64_t key0, int64_t lk, int wave) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t key = min(key0 + gm.k_row[i], lk - 1);
        const uint32_t off = static_cast<uint32_t>(key * k_sl) + gm.k_src[i];
        __builtin_amdgcn_global_load_lds(kp + off, (lds_void *)(stage + (2 * wave + i) * 1024), 16, 0, 0);
    }
    const int8_t *vbase = reinterpret_cast<const int8_t *>(vtp + key0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        __builtin_amdgcn_global_load_lds(vbase + gm.v_src[i], (lds_void *)(stage + kKTileBytes + (4 * wave + i) * 1024),
                                         16, 0, 0);
}

// S^T for one tile: s[kt][qt][r] = score of key 32 (kt >> 1) + 8 g + 4 (kt & 1) + r
// and query 16 qt + lc of the wave.
template <int QT>
__device__ __forceinline__ void qk_tile(const int8_t *stage, const LaneGeom &gm, const i32x4 (&qf)[QT][2],
                                        i32x4 (&s)[4][QT]) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
        const i32x4 kf0 = *reinterpret_cast<const i32x4 *>(stage + gm.k_rd[0] + kt * 16 * 128);
        const i32x4 kf1 = *reinterpret_cast<const i32x4 *>(stage + gm.k_rd[1] + kt * 16 * 128);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const i32x4 z = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf0, qf[qt][0], i32x4{0, 0, 0, 0}, 0, 0, 0);
            s[kt][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf1, qf[qt][1], z, 0, 0, 0);
        }
    }
}

// Softmax state of the wave: exponent base per query block, O^T and the row
// sums (l, accumulated by an MFMA against a ones operand so every lane ends
// with the complete sum for its query column).
template <int QT>
struct SoftmaxState {
    float m_used[QT];
    f32x4 acc_o[8][QT];
    f32x4 acc_l[QT];
};

// Scales (and masks) the tile's raw scores into sf and returns per-query-block
// row maxima in scaled units.  Masked tiles produce -inf for padded keys and,
// for causal attention, keys after the query.
template <int QT, bool kMask, bool kCausal>
__device__ __forceinline__ void tile_rowmax(i32x4 (&s)[4][QT], const float (&f)[QT], float (&mrow)[QT], int key_lim,
                                            int q_rel, int g, int lc) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        if constexpr (kMask) {
            const int qi = q_rel + 16 * qt + lc;
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = 32 * (kt >> 1) + 8 * g + 4 * (kt & 1) + r;
                    bool masked = key >= key_lim;
                    if constexpr (kCausal) masked = masked || key > qi;
                    const float x = masked ? -INFINITY : static_cast<float>(s[kt][qt][r]);
                    s[kt][qt][r] = __float_as_int(x);  // masked tiles carry floats from here on
                    mx = fmaxf(mx, x);
                }
            mrow[qt] = xmax_f32(mx) * f[qt];
        } else {
            int mi = imax3(s[0][qt][0], s[0][qt][1], s[0][qt][2]);
            mi = imax3(mi, s[0][qt][3], s[1][qt][0]);
            mi = imax3(mi, s[1][qt][1], s[1][qt][2]);
            mi = imax3(mi, s[1][qt][3], s[2][qt][0]);
            mi = imax3(mi, s[2][qt][1], s[2][qt][2]);
            mi = imax3(mi, s[2][qt][3], s[3][qt][0]);
            mi = imax3(mi, s[3][qt][1], s[3][qt][2]);
            mi = max(mi, s[3][qt][3]);
            mrow[qt] = static_cast<float>(xmax_i32(mi)) * f[qt];
        }
    }
}

template <int QT>
__device__ __forceinline__ void maybe_rescale(SoftmaxState<QT> &st, const float (&mrow)[QT]) {
    bool need = false;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) need = need || (mrow[qt] > st.m_used[qt] + kRescaleSlack);
    if (__any(need)) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const float m_new = fmaxf(st.m_used[qt], mrow[qt]);
            const float alpha = __builtin_amdgcn_exp2f(st.m_used[qt] - m_new);
            st.m_used[qt] = m_new;
            st.acc_l[qt] *= alpha;
#pragma unroll
            for (int ds = 0; ds < 8; ++ds) st.acc_o[ds][qt] *= alpha;
        }
    }
}

// P = 2^(s f - m_used) as bf16 B operands and O^T += V^T P, l += 1 P.
template <int QT, bool kMask>
__device__ __forceinline__ void tile_pv(const int8_t *stage, const LaneGeom &gm, const i32x4 (&s)[4][QT],
                                        const float (&f)[QT], SoftmaxState<QT> &st, const bf16x8 &ones) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        bf16x8 vf[8];
#pragma unroll
        for (int ds = 0; ds < 8; ++ds)
            vf[ds] = *reinterpret_cast<const bf16x8 *>(stage + gm.v_rd[h] + ds * 16 * 128);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const float nm = -st.m_used[qt];
            u32x4 packed;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float p2[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int e = 2 * j + t;           // keys 32 h + 8 g + e
                    const int v = s[2 * h + (e >> 2)][qt][e & 3];
                    const float x = kMask ? __int_as_float(v) : static_cast<float>(v);
                    p2[t] = __builtin_amdgcn_exp2f(__builtin_fmaf(x, f[qt], nm));
                }
                packed[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{p2[0], p2[1]}), bf16x2_t));
            }
            const bf16x8 pf = __builtin_bit_cast(bf16x8, packed);
#pragma unroll
            for (int ds = 0; ds < 8; ++ds)
                st.acc_o[ds][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[ds], pf, st.acc_o[ds][qt], 0, 0, 0);
            st.acc_l[qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf, st.acc_l[qt], 0, 0, 0);
        }
    }
}

template <int QT, bool kCausal>
__global__ __launch_bounds__(kThreads, QT == 4 ? 1 : 2) void sage_attn_kernel(
    const int8_t *__restrict__ q8, const float *__restrict__ q_scale, int blkq, const int8_t *__restrict__ k8,
    const float *__restrict__ k_scale, int kscale_shift, const uint16_t *__restrict__ vt, uint16_t *__restrict__ o,
    int hq, int groups, int64_t lq, int64_t lk, int64_t lpad, int64_t q_sb, int64_t q_sh, int64_t q_sl,
    int64_t k_sb, int64_t k_sh, int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl, float sm_log2) {
    __shared__ __align__(1024) int8_t lds[kStages][kStageBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4;
    const int lc = lane & 15;

    const int64_t bh = blockIdx.y;
    const int64_t b = bh / hq, h = bh % hq, hk = h / groups;
    const int64_t hkv = hq / groups;
    constexpr int kWaveQ = 16 * QT;
    constexpr int kBQ = 4 * kWaveQ;
    const int64_t qblock0 = static_cast<int64_t>(blockIdx.x) * kBQ;
    const int64_t q0 = qblock0 + wave * kWaveQ;

    const int8_t *qp = q8 + b * q_sb + h * q_sh;
    const int8_t *kp = k8 + b * k_sb + hk * k_sh;
    const uint16_t *vtp = vt + (b * hkv + hk) * kD * lpad;
    const int64_t nbq = (lq + blkq - 1) / blkq;
    const int64_t nbk = ((lk + kBKey - 1) / kBKey + (1 << kscale_shift) - 1) >> kscale_shift;
    const float *ks_row = k_scale + (b * hkv + hk) * nbk;

    int64_t key_end = lk;
    if constexpr (kCausal) key_end = min(lk, qblock0 + kBQ);
    const int tiles = static_cast<int>((key_end + kBKey - 1) / kBKey);
    const LaneGeom gm = lane_geom(wave, lane, lpad);
    // Tiles past the last one re-load it (their results are never used), so
    // the ring needs no guards.
    auto tile_key0 = [&](int it) { return static_cast<int64_t>(min(it, tiles - 1)) * kBKey; };
    issue_tile(lds[0], kp, vtp, gm, k_sl, tile_key0(0), lk, wave);
    issue_tile(lds[1], kp, vtp, gm, k_sl, tile_key0(1), lk, wave);

    i32x4 qf[QT][2];
    float qsc[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int64_t qi = min(q0 + 16 * qt + lc, lq - 1);
#pragma unroll
        for (int ds = 0; ds < 2; ++ds)
            qf[qt][ds] = *reinterpret_cast<const i32x4 *>(qp + qi * q_sl + 64 * ds + 16 * g);
        qsc[qt] = q_scale[(b * hq + h) * nbq + qi / blkq] * sm_log2;
    }
    SoftmaxState<QT> st;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        st.m_used[qt] = -INFINITY;
        st.acc_l[qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ds = 0; ds < 8; ++ds) st.acc_o[ds][qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = static_cast<__bf16>(1.0f);

    // Tiles at or past this key index need the Lk-tail or causal mask.
    int64_t mask_from = (lk / kBKey) * kBKey;
    if constexpr (kCausal) mask_from = min(mask_from, (q0 / kBKey) * kBKey);
    const int first_masked = static_cast<int>(min<int64_t>(tiles, mask_from / kBKey));

    // Software pipeline over key tiles.  Entering step(it), S(it) is in s_cur,
    // tile it sits in stage it % 3 and tile it + 1's loads are in flight.
    // The step waits for tile it + 1, refills the stage of tile it - 1 with
    // tile it + 2, then overlaps QK(it + 1) (MFMA) with the row max of S(it)
    // (VALU) and P(it) (VALU) with PV(it) (MFMA).
    auto step = [&](int it, i32x4 (&s_cur)[4][QT], i32x4 (&s_next)[4][QT], auto mask_tag) {
        constexpr bool kMask = decltype(mask_tag)::value;
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        issue_tile(lds[(it + 2) % kStages], kp, vtp, gm, k_sl, tile_key0(it + 2), lk, wave);
        const int64_t key0 = static_cast<int64_t>(it) * kBKey;
        const float kscale = ks_row[it >> kscale_shift];
        float f[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) f[qt] = qsc[qt] * kscale;
        const int key_lim = static_cast<int>(min(lk - key0, static_cast<int64_t>(kBKey)));
        const int q_rel = static_cast<int>(max(min(q0 - key0, static_cast<int64_t>(kBKey)), static_cast<int64_t>(-kBQ)));
        qk_tile<QT>(lds[(it + 1) % kStages], gm, qf, s_next);
        float mrow[QT];
        tile_rowmax<QT, kMask, kCausal>(s_cur, f, mrow, key_lim, q_rel, g, lc);
        maybe_rescale<QT>(st, mrow);
        tile_pv<QT, kMask>(lds[it % kStages], gm, s_cur, f, st, ones);
    };
    // Non-pipelined step for the boundary tiles (Lk tail, causal diagonal) and
    // an odd leftover: it waits for every outstanding load, then computes
    // QK(it), the row max, P and PV of the same tile.
    auto step_single = [&](int it, auto mask_tag) {
        constexpr bool kMask = decltype(mask_tag)::value;
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        __syncthreads();
        issue_tile(lds[(it + 2) % kStages], kp, vtp, gm, k_sl, tile_key0(it + 2), lk, wave);
        const int64_t key0 = static_cast<int64_t>(it) * kBKey;
        const float kscale = ks_row[it >> kscale_shift];
        float f[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) f[qt] = qsc[qt] * kscale;
        const int key_lim = static_cast<int>(min(lk - key0, static_cast<int64_t>(kBKey)));
        const int q_rel = static_cast<int>(max(min(q0 - key0, static_cast<int64_t>(kBKey)), static_cast<int64_t>(-kBQ)));
        i32x4 s1[4][QT];
        qk_tile<QT>(lds[it % kStages], gm, qf, s1);
        float mrow[QT];
        tile_rowmax<QT, kMask, kCausal>(s1, f, mrow, key_lim, q_rel, g, lc);
        maybe_rescale<QT>(st, mrow);
        tile_pv<QT, kMask>(lds[it % kStages], gm, s1, f, st, ones);
    };

    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    int it = 0;
    if (first_masked >= 2) {
        i32x4 sa[4][QT], sb[4][QT];
        qk_tile<QT>(lds[0], gm, qf, sa);
#pragma clang loop unroll(disable)
        for (; it + 2 <= first_masked; it += 2) {
            step(it, sa, sb, std::false_type{});
            step(it + 1, sb, sa, std::false_type{});
        }
    }
#pragma clang loop unroll(disable)
    for (; it < first_masked; ++it) step_single(it, std::false_type{});
#pragma clang loop unroll(disable)
    for (; it < tiles; ++it) step_single(it, std::true_type{});
    __builtin_amdgcn_s_waitcnt(0);

    // acc_o[ds][qt][r] = O[q0 + 16 qt + lc][16 ds + 4 g + r]; acc_l[qt][*] = l.
    uint16_t *op = o + b * o_sb + h * o_sh;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int64_t qi = q0 + 16 * qt + lc;
        const float inv = 1.0f / st.acc_l[qt][0];
        if (qi >= lq) continue;
#pragma unroll
        for (int ds = 0; ds < 8; ++ds) {
            u32x2 packed;
            packed.x = pack_bf16x2(st.acc_o[ds][qt][0] * inv, st.acc_o[ds][qt][1] * inv);
            packed.y = pack_bf16x2(st.acc_o[ds][qt][2] * inv, st.acc_o[ds][qt][3] * inv);
            *reinterpret_cast<u32x2 *>(op + qi * o_sl + 16 * ds + 4 * g) = packed;
        }
    }
}

// V [key][d] (bf16, strides) -> V^T [b][h][d][lpad] with zero keys in [lk, lpad).
// One workgroup per 64-key tile: 64 x 128 staged through LDS (rows padded to
// 132 elements so the column reads are bank-conflict free).
__global__ __launch_bounds__(256) void v_prep_kernel(const uint16_t *__restrict__ v, int64_t lk, int64_t lpad,
                                                     int64_t v_sb, int64_t v_sh, int64_t v_sl,
                                                     uint16_t *__restrict__ vt) {
    __shared__ uint16_t tile[kBKey][kD + 4];
    const int tid = threadIdx.x;
    const int64_t key0 = static_cast<int64_t>(blockIdx.x) * kBKey;
    const int64_t h = blockIdx.y, b = blockIdx.z, heads = gridDim.y;
    const uint16_t *vp = v + b * v_sb + h * v_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = i * 16 + (tid >> 4);
        const int c = tid & 15;
        u32x4 val = u32x4{0u, 0u, 0u, 0u};
        if (key0 + row < lk) val = *reinterpret_cast<const u32x4 *>(vp + (key0 + row) * v_sl + c * 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            tile[row][c * 8 + 2 * e] = static_cast<uint16_t>(val[e] & 0xffffu);
            tile[row][c * 8 + 2 * e + 1] = static_cast<uint16_t>(val[e] >> 16);
        }
    }
    __syncthreads();
    uint16_t *dst = vt + (b * heads + h) * kD * lpad + key0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int item = tid + 256 * i;  // (d, 8-key chunk)
        const int d = item >> 3, c = item & 7;
        u32x4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            out[e] = static_cast<uint32_t>(tile[c * 8 + 2 * e][d]) | (static_cast<uint32_t>(tile[c * 8 + 2 * e + 1][d]) << 16);
        *reinterpret_cast<u32x4 *>(dst + d * lpad + c * 8) = out;
    }
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_sage_v_prep(const void *v_bf16, int64_t batch, int64_t heads, int64_t len, int64_t dim,
                                  int64_t s_b, int64_t s_h, int64_t s_l, void *vt_bf16, int64_t lpad, void *stream) {
    using namespace tu;
    TU_REQUIRE(dim == kD, "V prep requires head_dim 128, got %lld", static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && heads > 0 && len > 0 && batch <= 65535 && heads <= 65535, "V prep dimensions out of range");
    TU_REQUIRE(lpad >= len && lpad % kBKey == 0, "V prep padded length must cover len and be a multiple of 64");
    TU_REQUIRE(v_bf16 && vt_bf16, "V prep pointers must be non-null");
    TU_REQUIRE(s_l % 8 == 0 && s_h % 8 == 0 && s_b % 8 == 0 && (reinterpret_cast<uintptr_t>(v_bf16) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(vt_bf16) & 15) == 0,
               "V prep needs 16-byte aligned rows");
    if (require_gfx950()) return -1;
    const dim3 grid(static_cast<unsigned>(lpad / kBKey), static_cast<unsigned>(heads), static_cast<unsigned>(batch));
    v_prep_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const uint16_t *>(v_bf16), len, lpad,
                                                                       s_b, s_h, s_l, static_cast<uint16_t *>(vt_bf16));
    return check_launch("tu_sage_v_prep");
}

extern "C" int32_t tu_sage_attn_fwd(const int8_t *q8, const float *q_scale, int64_t blkq, const int8_t *k8,
                                    const float *k_scale, int64_t blkk, const void *vt_bf16, int64_t lpad,
                                    void *o_bf16, int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk,
                                    int64_t dim, int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb,
                                    int64_t k_sh, int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                                    float sm_scale, int32_t causal, void *stream) {
    using namespace tu;
    TU_REQUIRE(dim == kD, "Sage attention kernel requires head_dim 128, got %lld", static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "Sage attention: hq must be a positive multiple of hkv");
    TU_REQUIRE(lq > 0 && lk > 0, "Sage attention requires non-empty sequences");
    TU_REQUIRE(lpad >= lk && lpad % kBKey == 0, "Sage attention: V^T padded length must cover lk, multiple of 64");
    TU_REQUIRE(blkq > 0 && blkk > 0 && blkk % kBKey == 0 && ((blkk / kBKey) & (blkk / kBKey - 1)) == 0,
               "Sage attention needs blkq > 0 and blkk = 64 * 2^n");
    TU_REQUIRE(blkq <= 0x7fffffff && blkk <= 0x7fffffff, "Sage attention block sizes out of range");
    TU_REQUIRE((lq + 127) / 128 <= 0x7fffffff && batch * hq <= 65535, "Sage attention grid too large");
    TU_REQUIRE(q8 && q_scale && k8 && k_scale && vt_bf16 && o_bf16, "Sage attention pointers must be non-null");
    TU_REQUIRE(sm_scale > 0.0f, "Sage attention sm_scale must be positive");
    TU_REQUIRE(q_sl % 16 == 0 && q_sh % 16 == 0 && q_sb % 16 == 0 && (reinterpret_cast<uintptr_t>(q8) & 15) == 0 &&
                   k_sl % 16 == 0 && k_sh % 16 == 0 && k_sb % 16 == 0 && (reinterpret_cast<uintptr_t>(k8) & 15) == 0,
               "Sage attention Q/K rows must be 16-byte aligned");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(vt_bf16) & 15) == 0 && o_sl % 4 == 0 && o_sh % 4 == 0 && o_sb % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(o_bf16) & 7) == 0,
               "Sage attention V^T/O must be aligned");
    if (require_gfx950()) return -1;
    constexpr int kQT = TU_ATTN_QT;
    const dim3 grid(static_cast<unsigned>((lq + 64 * kQT - 1) / (64 * kQT)), static_cast<unsigned>(batch * hq));
    const float sm_log2 = sm_scale * kLog2e;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int groups = static_cast<int>(hq / hkv);
    int kscale_shift = 0;
    while ((kBKey << kscale_shift) < blkk) ++kscale_shift;
#define TU_ATTN_ARGS                                                                                             \
    q8, q_scale, static_cast<int>(blkq), k8, k_scale, kscale_shift, static_cast<const uint16_t *>(vt_bf16),      \
        static_cast<uint16_t *>(o_bf16), static_cast<int>(hq), groups, lq, lk, lpad, q_sb, q_sh, q_sl, k_sb, k_sh,  \
        k_sl, o_sb, o_sh, o_sl, sm_log2
    if (causal) sage_attn_kernel<kQT, true><<<grid, kThreads, 0, s>>>(TU_ATTN_ARGS);
    else sage_attn_kernel<kQT, false><<<grid, kThreads, 0, s>>>(TU_ATTN_ARGS);
#undef TU_ATTN_ARGS
    return check_launch("tu_sage_attn_fwd");
}
