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
//   * Workgroup = 8 wave64 = 256 query rows of one (batch, head): two groups
//     of 4 waves, 32 rows (two 16-row fragments) per wave, one wave of each
//     group per SIMD.  One workgroup barrier per key tile; within a tile's
//     interval group 0 runs its MFMA cluster then its softmax VALU cluster,
//     group 1 the softmax first, so each SIMD sees one wave's MFMAs beside the
//     other's VALU work, with the two MFMA clusters overlapping in the middle
//     (a lone wave issues 16x16 MFMAs at about 60 % of the pipe, two waves
//     together fill it).
//   * Keys stream in tiles of 64 through a 4-stage LDS ring (24 KiB a stage)
//     filled by buffer_load_dwordx4 ... lds (no staging registers) from group
//     0, three tiles ahead of the MFMAs (measured 1-2 % faster than five
//     stages; the loads land in time either way).  V arrives pre-transposed (V^T,
//     [d][key], keys padded to a multiple of 64 with zeros) from
//     tu_sage_v_prep, so every MFMA operand is a plain LDS read.
//   * S^T = K Q^T runs on v_mfma_i32_16x16x64_i8 with the wave's Q rows
//     resident as the B operand, accumulators starting at the bit pattern of
//     1.5 * 2^23 so that the result reads as a float with one subtraction; a
//     lane then holds 4 keys x 1 query per 16x16 block, so the row max is an
//     integer max3 tree plus two cross-lane steps.  O^T = V^T P runs on
//     v_mfma_f32_16x16x32_bf16 with P taken straight from registers.
//   * Masking (Lk tail, causal diagonal) is an integer pre-pass compiled only
//     into the steps that need it.  The O rescale is lazy: the exponent base
//     m_used only moves when a row maximum exceeds it by more than 8
//     (p <= 2^8), which after the first tiles is rare.
//   * LDS rows are 128 B with 16-byte chunks XOR-swizzled by row bits 1..3,
//     conflict-free for the 16 lanes that read one chunk column.
#include <type_traits>

#include "attn_common.h"

namespace tu {
namespace {

constexpr int kThreads = 512;  // 8 waves: two groups of 4
constexpr int kQT = 2;                   // 16-row query fragments per wave
constexpr int kWaveQ = 16 * kQT;         // query rows per wave
constexpr int kBQ = 8 * kWaveQ;          // query rows per workgroup
constexpr int kBKey = 64;                // keys per tile
constexpr float kRescaleSlack = 8.0f;        // log2 of the largest p allowed

// Head-dim geometry (D = 64 or 128).  K tile: 64 keys x D bytes; V^T tile:
// D channels x 64 keys of bf16 (128-byte rows); group 0's 4 waves each move
// kKLoads + kVLoads 1 KiB blocks of a tile.
template <int D>
struct Geo {
    static_assert(D == 64 || D == 128, "head_dim 64 or 128");
    static constexpr int kKTileBytes = kBKey * D;
    static constexpr int kVTileBytes = D * kBKey * 2;
    static constexpr int kStageBytes = kKTileBytes + kVTileBytes;
    static constexpr int kKSlices = D / 64;  // 64-byte QK^T slices of a key row
    static constexpr int kDS = D / 16;       // 16-channel PV blocks
    static constexpr int kKLoads = kKTileBytes / 4096;
    static constexpr int kVLoads = kVTileBytes / 4096;
    static constexpr int kLoadsPerTile = kKLoads + kVLoads;
};

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
template <int D>
struct LaneGeom {
    uint32_t k_src[Geo<D>::kKLoads];    // byte offset (from key0's row) of this lane's K source chunks
    uint32_t v_src[Geo<D>::kVLoads];    // byte offset (from key0's column) of this lane's V^T source chunks
    uint32_t k_rd[Geo<D>::kKSlices];    // LDS byte offset of the K operand of slice i
    uint32_t v_rd[2];                   // LDS byte offset of the V^T operand, half 0 / 1
};

// K rows of 128 B (D = 128) have their 16-byte chunks XOR-swizzled by row
// bits 1..3, rows of 64 B (D = 64) by row bits 2..3; either way the 16 lanes
// that read one chunk column of 16 consecutive rows hit distinct banks.
template <int D>
__device__ __forceinline__ LaneGeom<D> lane_geom(int wave, int lane, int64_t k_sl, int64_t lpad) {
    LaneGeom<D> gm;
    const int g = lane >> 4, lc = lane & 15, sw = (lc >> 1) & 7;
    if constexpr (D == 128) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = (2 * wave + i) * 8 + (lane >> 3);
            gm.k_src[i] = static_cast<uint32_t>(kperm(row) * k_sl + ((lane & 7) ^ ((row >> 1) & 7)) * 16);
            gm.k_rd[i] = static_cast<uint32_t>(lc * 128 + (((4 * i + g) ^ sw) << 4));
        }
    } else {
        const int row = wave * 16 + (lane >> 2);
        gm.k_src[0] = static_cast<uint32_t>(kperm(row) * k_sl + ((lane & 3) ^ ((row >> 2) & 3)) * 16);
        gm.k_rd[0] = static_cast<uint32_t>(lc * 64 + ((g ^ ((lc >> 2) & 3)) << 4));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
        gm.v_rd[i] = static_cast<uint32_t>(Geo<D>::kKTileBytes + lc * 128 + (((4 * i + g) ^ sw) << 4));
#pragma unroll
    for (int i = 0; i < Geo<D>::kVLoads; ++i) {
        const int d = (Geo<D>::kVLoads * wave + i) * 8 + (lane >> 3);
        gm.v_src[i] = static_cast<uint32_t>((d * lpad + ((lane & 7) ^ ((d >> 1) & 7)) * 8) * 2);
    }
    return gm;
}

// Direct-to-LDS buffer loads of the K and V^T tiles at key0 into one ring
// stage.  Each buffer_load_dwordx4 ... lds moves 64 lanes x 16 B into 1 KiB of
// contiguous LDS; the K row permutation and the chunk swizzle come from the
// per-lane source offsets.  The tile's key offset goes into the per-lane
// offset, not the scalar one: the buffer range check covers only the
// per-lane offset, so K rows at or past lk (the range ends at lk rows) read
// as zeros instead of the bytes past the head's rows; those keys are masked
// by the softmax.  V^T is padded to whole tiles, so its key offset can stay
// scalar.
// One overload per head dim: the host compilation pass rejects a template of
// this function (the buffer builtins only exist for the device target), a
// plain device function it accepts.
#define TU_ISSUE_TILE_BODY(D)                                                                                      \
    constexpr int kK = Geo<D>::kKLoads, kV = Geo<D>::kVLoads;                                                      \
    _Pragma("unroll") for (int i = 0; i < kK; ++i)                                                                 \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void *)(stage + (kK * wave + i) * 1024), 16,            \
                                                 gm.k_src[i] + key0 * k_sl, 0, 0, 0);                              \
    _Pragma("unroll") for (int i = 0; i < kV; ++i)                                                                 \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void *)(stage + Geo<D>::kKTileBytes + (kV * wave + i) * 1024), \
                                                 16, gm.v_src[i], key0 * 2, 0, 0);
__device__ __forceinline__ void issue_tile(int8_t *stage, __amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                           const LaneGeom<128> &gm, uint32_t k_sl, uint32_t key0, int wave) {
    TU_ISSUE_TILE_BODY(128)
}
__device__ __forceinline__ void issue_tile(int8_t *stage, __amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                           const LaneGeom<64> &gm, uint32_t k_sl, uint32_t key0, int wave) {
    TU_ISSUE_TILE_BODY(64)
}
#undef TU_ISSUE_TILE_BODY

// S^T for one tile: s[kt][qt][r] = biased score of key 32 (kt >> 1) + 8 g +
// 4 (kt & 1) + r and query 16 qt + lc of the wave.
template <int D>
__device__ __forceinline__ void qk_tile(const int8_t *stage, const LaneGeom<D> &gm,
                                        const i32x4 (&qf)[kQT][Geo<D>::kKSlices], i32x4 (&s)[4][kQT]) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
        i32x4 kf[Geo<D>::kKSlices];
#pragma unroll
        for (int i = 0; i < Geo<D>::kKSlices; ++i)
            kf[i] = *reinterpret_cast<const i32x4 *>(stage + gm.k_rd[i] + kt * 16 * D);
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
            i32x4 acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[0], qf[qt][0], i32x4{kBias, kBias, kBias, kBias},
                                                              0, 0, 0);
            if constexpr (D == 128) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[1], qf[qt][1], acc, 0, 0, 0);
            s[kt][qt] = acc;
        }
    }
}

// Softmax state of the wave: exponent base per query block, O^T and the row
// sums (l, accumulated by an MFMA against a ones operand so every lane ends
// with the complete sum for its query column).
template <int D>
struct SoftmaxState {
    float m_used[kQT];
    f32x4 acc_o[Geo<D>::kDS][kQT];
    f32x4 acc_l[kQT];
};

// Masks a tile's biased scores in place: masked keys (key >= key_lim, and for
// causal attention key > query) get the int bit pattern of -inf, which is
// below every biased score as an integer and stays -inf through the
// subtraction of the bias, so the row max ignores it and its p is 0.
template <bool kCausal>
__device__ __forceinline__ void mask_tile(i32x4 (&s)[4][kQT], int key_lim, int q_rel, int g, int lc) {
    constexpr int kNegInf = static_cast<int>(0xFF800000u);
    // key = c + 8 g with c a constant; key is masked iff c > t, with t the
    // lane's last visible key minus 8 g.  The select is done with integer
    // arithmetic (sign of t - c) to keep lane masks out of scalar registers.
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        int t = key_lim - 1 - 8 * g;
        if constexpr (kCausal) t = min(t, q_rel + 16 * qt + lc - 8 * g);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int c = 32 * (kt >> 1) + 4 * (kt & 1) + r;
                const int m = (t - c) >> 31;  // all ones when masked
                s[kt][qt][r] = (s[kt][qt][r] & ~m) | (kNegInf & m);
            }
    }
}

// Softmax of one tile: lazy rescale of O and l, then P = 2^(dot f - m_used)
// rounded to bf16, packed as the PV B operands p[h][qt] (keys 32 h + 8 g ..
// + 7 of query 16 qt + lc).
//
// The exponent base m_used of a query row only moves when some score of the
// row exceeds it by more than kRescaleSlack; each lane tests its own 16
// scores (an integer max tree on the biased values), and only when some lane
// of the wave fails is the exact row maximum reduced across the 4 lanes that
// hold the row.
//
// x = dot f - m_used is formed as fma(biased, f, c) with
// c = -(1.5 * 2^23 f + m_used) when |c| < 2^12, which keeps the rounding of c
// below 2^-13 in the exponent; otherwise the bias is subtracted exactly first.
template <int D>
__device__ __forceinline__ void softmax_tile(const i32x4 (&s)[4][kQT], const float (&f)[kQT], SoftmaxState<D> &st,
                                             bf16x8 (&p)[2][kQT]) {
    float mlane[kQT];
    bool need = false;
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        int mi = imax3(s[0][qt][0], s[0][qt][1], s[0][qt][2]);
        mi = imax3(mi, s[0][qt][3], s[1][qt][0]);
        mi = imax3(mi, s[1][qt][1], s[1][qt][2]);
        mi = imax3(mi, s[1][qt][3], s[2][qt][0]);
        mi = imax3(mi, s[2][qt][1], s[2][qt][2]);
        mi = imax3(mi, s[2][qt][3], s[3][qt][0]);
        mi = imax3(mi, s[3][qt][1], s[3][qt][2]);
        mi = max(mi, s[3][qt][3]);
        mlane[qt] = (__int_as_float(mi) - kBiasF) * f[qt];
        need = need || (mlane[qt] > st.m_used[qt] + kRescaleSlack);
    }
    if (__any(need)) {
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
            const float m_new = fmaxf(st.m_used[qt], xmax_f32(mlane[qt]));
            // a row with no visible key yet keeps m_used = -inf and alpha = 1
            const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(st.m_used[qt] - m_new);
            st.m_used[qt] = m_new;
            st.acc_l[qt] *= alpha;
#pragma unroll
            for (int ds = 0; ds < Geo<D>::kDS; ++ds) st.acc_o[ds][qt] *= alpha;
        }
    }
    float c[kQT];
    bool exact = false;
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        c[qt] = -__builtin_fmaf(kBiasF, f[qt], st.m_used[qt]);
        exact = exact || !(fabsf(c[qt]) < 4096.0f);
    }
    auto make_p = [&](auto exact_tag) {
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
            const float nm = -st.m_used[qt];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                u32x4 packed;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float p2[2];
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const int e = 2 * j + t;  // keys 32 h + 8 g + e
                        const float v = __int_as_float(s[2 * h + (e >> 2)][qt][e & 3]);
                        const float x = decltype(exact_tag)::value ? __builtin_fmaf(v - kBiasF, f[qt], nm)
                                                                   : __builtin_fmaf(v, f[qt], c[qt]);
                        p2[t] = __builtin_amdgcn_exp2f(x);
                    }
                    packed[j] =
                        __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{p2[0], p2[1]}), bf16x2_t));
                }
                p[h][qt] = __builtin_bit_cast(bf16x8, packed);
            }
        }
    };
    if (__any(exact)) make_p(std::true_type{});
    else make_p(std::false_type{});
}

// O^T += V^T P and l += 1 P for one tile.
template <int D>
__device__ __forceinline__ void pv_tile(const int8_t *stage, const LaneGeom<D> &gm, const bf16x8 (&p)[2][kQT],
                                        SoftmaxState<D> &st, const bf16x8 &ones) {
    constexpr int kDS = Geo<D>::kDS;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        bf16x8 vf[kDS];
#pragma unroll
        for (int ds = 0; ds < kDS; ++ds)
            vf[ds] = *reinterpret_cast<const bf16x8 *>(stage + gm.v_rd[h] + ds * 16 * 128);
#pragma unroll
        for (int ds = 0; ds < kDS; ++ds)
#pragma unroll
            for (int qt = 0; qt < kQT; ++qt)
                st.acc_o[ds][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[ds], p[h][qt], st.acc_o[ds][qt], 0, 0, 0);
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
            st.acc_l[qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, p[h][qt], st.acc_l[qt], 0, 0, 0);
    }
}

// MFMA cluster of a steady-state step: QK^T of the tile in kst and PV of the
// tile in vst, with the LDS fragment reads issued a group of MFMAs ahead of
// their first use.
template <int D>
__device__ __forceinline__ void mfma_cluster(const int8_t *kst, const int8_t *vst, const LaneGeom<D> &gm,
                                             const i32x4 (&qf)[kQT][Geo<D>::kKSlices], i32x4 (&s)[4][kQT],
                                             const bf16x8 (&p)[2][kQT], SoftmaxState<D> &st, const bf16x8 &ones) {
    constexpr int kDS = Geo<D>::kDS, kSl = Geo<D>::kKSlices;
    // This wave's MFMA cluster is the critical path of its interval: raise its
    // issue priority over the other group's softmax VALU on the same SIMD
    // (measured about 1 % faster; raising the softmax instead was slower).
    __builtin_amdgcn_s_setprio(3);
    i32x4 kf[4][kSl];
    bf16x8 va[kDS], vb[kDS];
    // first-slice K fragments first: the first QK^T MFMAs only need those
#pragma unroll
    for (int i = 0; i < kSl; ++i)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) kf[kt][i] = *reinterpret_cast<const i32x4 *>(kst + gm.k_rd[i] + kt * 16 * D);
#pragma unroll
    for (int ds = 0; ds < kDS; ++ds) va[ds] = *reinterpret_cast<const bf16x8 *>(vst + gm.v_rd[0] + ds * 16 * 128);
    i32x4 z[4][kQT];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
            z[kt][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[kt][0], qf[qt][0], i32x4{kBias, kBias, kBias, kBias},
                                                              0, 0, 0);
    if constexpr (D == 128) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int qt = 0; qt < kQT; ++qt)
                s[kt][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[kt][kSl - 1], qf[qt][kSl - 1], z[kt][qt], 0, 0, 0);
    } else {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int qt = 0; qt < kQT; ++qt) s[kt][qt] = z[kt][qt];
    }
#pragma unroll
    for (int ds = 0; ds < kDS; ++ds) vb[ds] = *reinterpret_cast<const bf16x8 *>(vst + gm.v_rd[1] + ds * 16 * 128);
    // PV holds each V^T fragment (the A operand) for both query fragments,
    // as QK^T holds each K fragment: measured 1 % faster at B1 H40 L32760
    // than holding P across the V^T fragments (and QK^T holding Q across the
    // K fragments was 1 % slower).
#pragma unroll
    for (int ds = 0; ds < kDS; ++ds)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
            st.acc_o[ds][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[ds], p[0][qt], st.acc_o[ds][qt], 0, 0, 0);
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt)
        st.acc_l[qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, p[0][qt], st.acc_l[qt], 0, 0, 0);
#pragma unroll
    for (int ds = 0; ds < kDS; ++ds)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
            st.acc_o[ds][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vb[ds], p[1][qt], st.acc_o[ds][qt], 0, 0, 0);
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt)
        st.acc_l[qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, p[1][qt], st.acc_l[qt], 0, 0, 0);
    // Issue order, keeping at most 12 LDS reads in flight (the wait counter
    // holds 15; past that the compiler can only wait for all of them):
    // K reads, first QK^T MFMAs, first V^T half, second QK^T MFMAs (D = 128)
    // and 4 PV MFMAs, second V^T half, remaining PV MFMAs.
    if constexpr (D == 128) {
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 12, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);
    } else {
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 9, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 15, 0);
    }
    __builtin_amdgcn_s_setprio(0);
}

// Schedule.  A workgroup is 8 waves in two groups of 4 (one wave of each
// group per SIMD), 256 query rows of one (batch, head).  Each wave runs the
// same sequence of clusters over the key tiles t = 0 .. T-1:
//   QK(0), softmax(0), then per tile M_t = { QK(t+1), PV(t) } and
//   softmax(t+1),
// with one workgroup barrier per interval: interval 0 = [QK(0), softmax(0)]
// for group 0 and [QK(0)] for group 1; interval t+1 = [M_t, softmax(t+1)]
// for group 0 and [softmax(t), M_t] for group 1.  Both groups read tiles t
// and t+1 in interval t+1.  Group 0 alone streams the K and V^T tiles
// through a kStages-deep LDS ring, kAhead tiles ahead, and waits for the
// tile the next interval reads before the barrier that opens it.
// tests/test_attn_schedule.py replays these loops on the host and checks
// equal barrier counts and ring residency for every wave.
constexpr int kStages = 4;
constexpr int kAhead = kStages - 1;

// kSplit: the workgroup covers key tiles [blockIdx.z * split_tiles, + split_tiles)
// of a non-causal attention and writes its unnormalized O with the row's
// exponent base and row sum to `part` for sage_combine_kernel.
template <int D, bool kCausal, bool kSplit = false>
__global__ __launch_bounds__(kThreads, 1) void sage_attn_kernel(
    const int8_t *__restrict__ q8, const float *__restrict__ q_scale, int blkq, const int8_t *__restrict__ k8,
    const float *__restrict__ k_scale, int kscale_shift, const uint16_t *__restrict__ vt, uint16_t *__restrict__ o,
    int hq, int groups, int64_t lq, int64_t lk, int64_t lpad, int64_t q_sb, int64_t q_sh, int64_t q_sl,
    int64_t k_sb, int64_t k_sh, int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl, float sm_log2,
    int split_tiles, float *__restrict__ part) {
    static_assert(!(kSplit && kCausal), "key splits are for non-causal attention");
    constexpr int kSl = Geo<D>::kKSlices;
    constexpr int kLoadsPerTile = Geo<D>::kLoadsPerTile;
    __shared__ __align__(1024) int8_t lds[kStages][Geo<D>::kStageBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;
    const int w4 = wave & 3;
    const int g = lane >> 4;
    const int lc = lane & 15;

    const int64_t bh = blockIdx.y;
    const int64_t b = bh / hq, h = bh % hq, hk = h / groups;
    const int64_t hkv = hq / groups;
    const int64_t qblock0 = static_cast<int64_t>(blockIdx.x) * kBQ;
    const int64_t q0 = qblock0 + grp * (kBQ / 2) + w4 * kWaveQ;

    const int8_t *qp = q8 + b * q_sb + h * q_sh;
    const int8_t *kp = k8 + b * k_sb + hk * k_sh;
    const uint16_t *vtp = vt + (b * hkv + hk) * D * lpad;
    const int64_t nbq = (lq + blkq - 1) / blkq;
    const int64_t nbk = ((lk + kBKey - 1) / kBKey + (1 << kscale_shift) - 1) >> kscale_shift;
    const float *ks_row = k_scale + (b * hkv + hk) * nbk;

    int64_t key_end = lk;
    if constexpr (kCausal) key_end = min(lk, qblock0 + kBQ);
    // first key tile of this workgroup's key range (0 unless split)
    const int tile_base = kSplit ? static_cast<int>(blockIdx.z) * split_tiles : 0;
    int tiles = static_cast<int>((key_end + kBKey - 1) / kBKey);
    if constexpr (kSplit) tiles = min(split_tiles, tiles - tile_base);
    // Tiles this wave computes: all of them, or up to its last query's
    // diagonal when causal.  Later tiles only keep the barrier count.
    int my_tiles = tiles;
    if constexpr (kCausal)
        my_tiles = static_cast<int>(min<int64_t>(tiles, max<int64_t>(1, (min(q0 + kWaveQ, lq) + kBKey - 1) / kBKey)));
    // Tiles at or past this one need the Lk-tail or causal mask.
    int64_t mask_from = lk / kBKey - tile_base;
    if constexpr (kCausal) mask_from = min(mask_from, q0 / kBKey);
    const int first_masked = static_cast<int>(min<int64_t>(tiles, mask_from));

    const LaneGeom<D> gm = lane_geom<D>(w4, lane, k_sl, lpad);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kp, static_cast<uint32_t>(lk * k_sl));
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vtp, static_cast<uint32_t>(D * lpad * 2));
    const uint32_t k_sl32 = static_cast<uint32_t>(k_sl);
    auto tile_key0 = [&](int it) { return static_cast<uint32_t>((tile_base + min(it, tiles - 1)) * kBKey); };

    i32x4 qf[kQT][kSl];
    float qsc[kQT];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        const int64_t qi = min(q0 + 16 * qt + lc, lq - 1);
#pragma unroll
        for (int ds = 0; ds < kSl; ++ds)
            qf[qt][ds] = *reinterpret_cast<const i32x4 *>(qp + qi * q_sl + 64 * ds + 16 * g);
        qsc[qt] = q_scale[(b * hq + h) * nbq + qi / blkq] * sm_log2;
    }
    if (grp == 0) {
#pragma unroll
        for (int j = 0; j < kAhead; ++j) issue_tile(lds[j], krs, vrs, gm, k_sl32, tile_key0(j), w4);
    }
    SoftmaxState<D> st;
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        st.m_used[qt] = -INFINITY;
        st.acc_l[qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ds = 0; ds < Geo<D>::kDS; ++ds) st.acc_o[ds][qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    bf16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = static_cast<__bf16>(1.0f);

    i32x4 s[4][kQT];
    bf16x8 pb[2][kQT];

    // softmax of tile it (it < my_tiles) into pb; mask_tag false promises
    // it < first_masked.
    auto softmax = [&](int it, auto mask_tag) {
        const float kscale = ks_row[(tile_base + it) >> kscale_shift];
        float f[kQT];
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) f[qt] = qsc[qt] * kscale;
        if (decltype(mask_tag)::value && it >= first_masked) {
            const int64_t key0 = static_cast<int64_t>(tile_base + it) * kBKey;
            const int key_lim = static_cast<int>(min(lk - key0, static_cast<int64_t>(kBKey)));
            const int q_rel =
                static_cast<int>(max(min(q0 - key0, static_cast<int64_t>(kBKey)), static_cast<int64_t>(-kBQ)));
            mask_tile<kCausal>(s, key_lim, q_rel, g, lc);
        }
        softmax_tile(s, f, st, pb);
    };

    // Group 0 has tile 0 (and the Q loads) resident before the first barrier.
    if (grp == 0) __builtin_amdgcn_s_waitcnt(vmcnt_imm((kAhead - 1) * kLoadsPerTile));
    wg_barrier();
    // Interval 0: QK(0); group 0 also runs softmax(0) and waits for tile 1.
    // Group 1 runs softmax(0) right after the barrier, opening interval 1.
    qk_tile(lds[0], gm, qf, s);
    const int main_steps = max(0, min(my_tiles, first_masked) - 1);
    if (grp == 0) {
        softmax(0, std::true_type{});
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((kAhead - 2) * kLoadsPerTile));
    }
    wg_barrier();
    if (grp == 1) softmax(0, std::true_type{});
    // Intervals 1 .. main_steps, one barrier each.  Both groups run the same
    // sequence M_it = {QK(it + 1), PV(it)}, softmax(it + 1); group 0's
    // barrier follows the softmax, group 1's precedes it, so interval it + 1
    // is [M_it, softmax(it + 1)] for group 0 and [softmax(it), M_it] for
    // group 1: on each SIMD the second half of one wave's MFMA cluster
    // overlaps the first half of the other's.  Group 0 issues tile
    // it + kAhead after its MFMA cluster (its stage held tile it - 1, which
    // both groups last read in the previous interval) and, before its
    // barrier, waits for tile it + 2, which interval it + 2 reads.
#pragma clang loop unroll(disable)
    for (int it = 0; it < main_steps; ++it) {
        mfma_cluster(lds[(it + 1) % kStages], lds[it % kStages], gm, qf, s, pb, st, ones);
        if (grp == 0) issue_tile(lds[(it + kAhead) % kStages], krs, vrs, gm, k_sl32, tile_key0(it + kAhead), w4);
        else wg_barrier();
        softmax(it + 1, std::false_type{});
        if (grp == 0) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((kAhead - 2) * kLoadsPerTile));
            wg_barrier();
        }
    }
    // Remaining intervals: masked tiles, the last tile, and (causal) tiles
    // past this wave's diagonal, which only keep the barrier count.  Group 1
    // has already run softmax(main_steps).
#pragma clang loop unroll(disable)
    for (int it = main_steps; it < tiles; ++it) {
        if (grp == 0)
            issue_tile(lds[(it + kAhead) % kStages], krs, vrs, gm, k_sl32, tile_key0(it + kAhead), w4);
        if (it + 1 < my_tiles) qk_tile(lds[(it + 1) % kStages], gm, qf, s);
        if (it < my_tiles) pv_tile(lds[it % kStages], gm, pb, st, ones);
        if (grp == 1) wg_barrier();
        if (it + 1 < my_tiles) softmax(it + 1, std::true_type{});
        if (grp == 0) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((kAhead - 2) * kLoadsPerTile));
            wg_barrier();
        }
    }
    __builtin_amdgcn_s_waitcnt(0);

    // acc_o[ds][qt][r] = O[q0 + 16 qt + lc][16 ds + 4 g + r]; acc_l[qt][*] = l.
    if constexpr (kSplit) {
        // unnormalized O of this key range, then (m_used, l) per row:
        // part = [splits][B * H][lq][D] fp32, followed by [splits][B * H][lq][2]
        const int64_t rows = static_cast<int64_t>(gridDim.y) * lq;
        const int64_t row0 = (static_cast<int64_t>(blockIdx.z) * gridDim.y + bh) * lq;
        float *po = part + row0 * D;
        float *pml = part + static_cast<int64_t>(gridDim.z) * rows * D + row0 * 2;
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
            const int64_t qi = q0 + 16 * qt + lc;
            if (qi >= lq) continue;
#pragma unroll
            for (int ds = 0; ds < Geo<D>::kDS; ++ds)
                *reinterpret_cast<f32x4 *>(po + qi * D + 16 * ds + 4 * g) = st.acc_o[ds][qt];
            if (g == 0) *reinterpret_cast<f32x2 *>(pml + qi * 2) = f32x2{st.m_used[qt], st.acc_l[qt][0]};
        }
        return;
    }
    uint16_t *op = o + b * o_sb + h * o_sh;
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        const int64_t qi = q0 + 16 * qt + lc;
        const float inv = 1.0f / st.acc_l[qt][0];
        if (qi >= lq) continue;
#pragma unroll
        for (int ds = 0; ds < Geo<D>::kDS; ++ds) {
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
template <int D>
__global__ __launch_bounds__(256) void v_prep_kernel(const uint16_t *__restrict__ v, int64_t lk, int64_t lpad,
                                                     int64_t v_sb, int64_t v_sh, int64_t v_sl,
                                                     uint16_t *__restrict__ vt) {
    constexpr int kChunks = D / 8;             // 16-byte chunks of a key row
    constexpr int kRowsPerPass = 256 / kChunks;
    __shared__ uint16_t tile[kBKey][D + 4];
    const int tid = threadIdx.x;
    const int64_t key0 = static_cast<int64_t>(blockIdx.x) * kBKey;
    const int64_t h = blockIdx.y, b = blockIdx.z, heads = gridDim.y;
    const uint16_t *vp = v + b * v_sb + h * v_sh;
#pragma unroll
    for (int i = 0; i < kBKey / kRowsPerPass; ++i) {
        const int row = i * kRowsPerPass + tid / kChunks;
        const int c = tid % kChunks;
        u32x4 val = u32x4{0u, 0u, 0u, 0u};
        if (key0 + row < lk) val = *reinterpret_cast<const u32x4 *>(vp + (key0 + row) * v_sl + c * 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            tile[row][c * 8 + 2 * e] = static_cast<uint16_t>(val[e] & 0xffffu);
            tile[row][c * 8 + 2 * e + 1] = static_cast<uint16_t>(val[e] >> 16);
        }
    }
    __syncthreads();
    uint16_t *dst = vt + (b * heads + h) * D * lpad + key0;
#pragma unroll
    for (int i = 0; i < D * 8 / 256; ++i) {
        const int item = tid + 256 * i;  // (d, 8-key chunk)
        const int d = item >> 3, c = item & 7;
        u32x4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            out[e] = static_cast<uint32_t>(tile[c * 8 + 2 * e][d]) | (static_cast<uint32_t>(tile[c * 8 + 2 * e + 1][d]) << 16);
        *reinterpret_cast<u32x4 *>(dst + d * lpad + c * 8) = out;
    }
}

// Merges the key-range partials of sage_attn_kernel<D, false, true>: per
// row, M = max_s m_s, w_s = 2^(m_s - M), out = sum_s w_s O_s / sum_s w_s l_s
// rounded to bf16.  D / 8 threads per row, 8 channels each.
template <int D>
__global__ __launch_bounds__(256) void sage_combine_kernel(const float *__restrict__ part, int splits, int hq,
                                                           int64_t bh_rows, int64_t lq, uint16_t *__restrict__ o,
                                                           int64_t o_sb, int64_t o_sh, int64_t o_sl) {
    constexpr int kTpr = D / 8;  // threads per row
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (256 / kTpr) + threadIdx.x / kTpr;
    const int d0 = (threadIdx.x % kTpr) * 8;
    const int64_t rows = bh_rows * lq;
    if (row >= rows) return;
    const float *ml = part + static_cast<int64_t>(splits) * rows * D;
    float m = -INFINITY;
    for (int sp = 0; sp < splits; ++sp) m = fmaxf(m, ml[(sp * rows + row) * 2]);
    float l = 0.0f, acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int sp = 0; sp < splits; ++sp) {
        const float ms = ml[(sp * rows + row) * 2];
        const float w = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - m);
        l = __builtin_fmaf(w, ml[(sp * rows + row) * 2 + 1], l);
        const f32x4 *src = reinterpret_cast<const f32x4 *>(part + (sp * rows + row) * D + d0);
        const f32x4 a = src[0], c = src[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc[e] = __builtin_fmaf(w, a[e], acc[e]);
            acc[4 + e] = __builtin_fmaf(w, c[e], acc[4 + e]);
        }
    }
    const float inv = 1.0f / l;
    const int64_t bh = row / lq, q = row - bh * lq;
    uint16_t *dst = o + (bh / hq) * o_sb + (bh % hq) * o_sh + q * o_sl + d0;
    u32x2 lo, hi;
    lo.x = pack_bf16x2(acc[0] * inv, acc[1] * inv);
    lo.y = pack_bf16x2(acc[2] * inv, acc[3] * inv);
    hi.x = pack_bf16x2(acc[4] * inv, acc[5] * inv);
    hi.y = pack_bf16x2(acc[6] * inv, acc[7] * inv);
    reinterpret_cast<u32x2 *>(dst)[0] = lo;
    reinterpret_cast<u32x2 *>(dst)[1] = hi;
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_sage_v_prep(const void *v_bf16, int64_t batch, int64_t heads, int64_t len, int64_t dim,
                                  int64_t s_b, int64_t s_h, int64_t s_l, void *vt_bf16, int64_t lpad, void *stream) {
    using namespace tu;
    TU_REQUIRE(dim == 64 || dim == 128, "V prep requires head_dim 64 or 128, got %lld", static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && heads > 0 && len > 0 && batch <= 65535 && heads <= 65535, "V prep dimensions out of range");
    TU_REQUIRE(lpad >= len && lpad % kBKey == 0, "V prep padded length must cover len and be a multiple of 64");
    TU_REQUIRE(v_bf16 && vt_bf16, "V prep pointers must be non-null");
    TU_REQUIRE(s_l % 8 == 0 && s_h % 8 == 0 && s_b % 8 == 0 && (reinterpret_cast<uintptr_t>(v_bf16) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(vt_bf16) & 15) == 0,
               "V prep needs 16-byte aligned rows");
    if (require_gfx950()) return -1;
    const dim3 grid(static_cast<unsigned>(lpad / kBKey), static_cast<unsigned>(heads), static_cast<unsigned>(batch));
    const auto *vp = static_cast<const uint16_t *>(v_bf16);
    auto *vtp = static_cast<uint16_t *>(vt_bf16);
    if (dim == 128) v_prep_kernel<128><<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(vp, len, lpad, s_b, s_h, s_l, vtp);
    else v_prep_kernel<64><<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(vp, len, lpad, s_b, s_h, s_l, vtp);
    return check_launch("tu_sage_v_prep");
}

namespace tu {
namespace {

// Argument checks shared by the attention entry points (all on the host,
// before any HIP call).
int32_t check_attn_args(const int8_t *q8, const float *q_scale, int64_t blkq, const int8_t *k8, const float *k_scale,
                        int64_t blkk, const void *vt_bf16, int64_t lpad, void *o_bf16, int64_t batch, int64_t hq,
                        int64_t hkv, int64_t lq, int64_t lk, int64_t dim, int64_t q_sb, int64_t q_sh, int64_t q_sl,
                        int64_t k_sb, int64_t k_sh, int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                        float sm_scale) {
    TU_REQUIRE(dim == 64 || dim == 128, "Sage attention kernel requires head_dim 64 or 128, got %lld",
               static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "Sage attention: hq must be a positive multiple of hkv");
    TU_REQUIRE(lq > 0 && lk > 0, "Sage attention requires non-empty sequences");
    TU_REQUIRE(lpad >= lk && lpad % kBKey == 0, "Sage attention: V^T padded length must cover lk, multiple of 64");
    TU_REQUIRE(blkq > 0 && blkk > 0 && blkk % kBKey == 0 && ((blkk / kBKey) & (blkk / kBKey - 1)) == 0,
               "Sage attention needs blkq > 0 and blkk = 64 * 2^n");
    TU_REQUIRE(blkq <= 0x7fffffff && blkk <= 0x7fffffff, "Sage attention block sizes out of range");
    TU_REQUIRE((lq + kBQ - 1) / kBQ <= 0x7fffffff && batch * hq <= 65535, "Sage attention grid too large");
    TU_REQUIRE(lk * k_sl < (int64_t{1} << 32) && dim * lpad * 2 < (int64_t{1} << 32),
               "Sage attention: one head's K or V^T exceeds 4 GiB of addressable bytes");
    TU_REQUIRE(q8 && q_scale && k8 && k_scale && vt_bf16 && o_bf16, "Sage attention pointers must be non-null");
    TU_REQUIRE(sm_scale > 0.0f, "Sage attention sm_scale must be positive");
    TU_REQUIRE(q_sl % 16 == 0 && q_sh % 16 == 0 && q_sb % 16 == 0 && (reinterpret_cast<uintptr_t>(q8) & 15) == 0 &&
                   k_sl % 16 == 0 && k_sh % 16 == 0 && k_sb % 16 == 0 && (reinterpret_cast<uintptr_t>(k8) & 15) == 0,
               "Sage attention Q/K rows must be 16-byte aligned");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(vt_bf16) & 15) == 0 && o_sl % 4 == 0 && o_sh % 4 == 0 && o_sb % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(o_bf16) & 7) == 0,
               "Sage attention V^T/O must be aligned");
    return require_gfx950();
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_sage_attn_fwd(const int8_t *q8, const float *q_scale, int64_t blkq, const int8_t *k8,
                                    const float *k_scale, int64_t blkk, const void *vt_bf16, int64_t lpad,
                                    void *o_bf16, int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk,
                                    int64_t dim, int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb,
                                    int64_t k_sh, int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl,
                                    float sm_scale, int32_t causal, void *stream) {
    using namespace tu;
    if (check_attn_args(q8, q_scale, blkq, k8, k_scale, blkk, vt_bf16, lpad, o_bf16, batch, hq, hkv, lq, lk, dim, q_sb,
                        q_sh, q_sl, k_sb, k_sh, k_sl, o_sb, o_sh, o_sl, sm_scale))
        return -1;
    const dim3 grid(static_cast<unsigned>((lq + kBQ - 1) / kBQ), static_cast<unsigned>(batch * hq));
    const float sm_log2 = sm_scale * kLog2e;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int groups = static_cast<int>(hq / hkv);
    int kscale_shift = 0;
    while ((kBKey << kscale_shift) < blkk) ++kscale_shift;
#define TU_ATTN_ARGS                                                                                             \
    q8, q_scale, static_cast<int>(blkq), k8, k_scale, kscale_shift, static_cast<const uint16_t *>(vt_bf16),      \
        static_cast<uint16_t *>(o_bf16), static_cast<int>(hq), groups, lq, lk, lpad, q_sb, q_sh, q_sl, k_sb, k_sh,  \
        k_sl, o_sb, o_sh, o_sl, sm_log2, 0, nullptr
    if (dim == 128) {
        if (causal) sage_attn_kernel<128, true><<<grid, kThreads, 0, s>>>(TU_ATTN_ARGS);
        else sage_attn_kernel<128, false><<<grid, kThreads, 0, s>>>(TU_ATTN_ARGS);
    } else {
        if (causal) sage_attn_kernel<64, true><<<grid, kThreads, 0, s>>>(TU_ATTN_ARGS);
        else sage_attn_kernel<64, false><<<grid, kThreads, 0, s>>>(TU_ATTN_ARGS);
    }
#undef TU_ATTN_ARGS
    return check_launch("tu_sage_attn_fwd");
}

// Key splits for a grid that fills the GPU badly: a workgroup's time is about
// its key tiles plus a fixed ~4 tiles of prologue and epilogue, and the
// workgroups run in rounds of `cus`; a split also pays ~2 tiles for the
// partial write and the combine.  Splits keep at least 16 key tiles each.
extern "C" int32_t tu_sage_attn_kv_splits(int64_t batch, int64_t hq, int64_t lq, int64_t lk, int32_t causal,
                                          int32_t cus) {
    using namespace tu;
    if (causal || batch <= 0 || hq <= 0 || lq <= 0 || lk <= 0 || cus <= 0) return 1;
    const int64_t wgs = (lq + kBQ - 1) / kBQ * batch * hq;
    const int64_t tiles = (lk + kBKey - 1) / kBKey;
    int32_t best = 1;
    double best_cost = 0.0;
    for (int32_t sp = 1; sp <= 8; ++sp) {
        const int64_t per = (tiles + sp - 1) / sp;
        if (sp > 1 && (per < 16 || (tiles + per - 1) / per != sp)) continue;
        const double cost = static_cast<double>((sp * wgs + cus - 1) / cus) * (per + 4 + (sp > 1 ? 2 : 0));
        if (sp == 1 || cost < best_cost) {
            best = sp;
            best_cost = cost;
        }
    }
    return best;
}

extern "C" int32_t tu_sage_attn_fwd_split(const int8_t *q8, const float *q_scale, int64_t blkq, const int8_t *k8,
                                          const float *k_scale, int64_t blkk, const void *vt_bf16, int64_t lpad,
                                          void *o_bf16, int64_t batch, int64_t hq, int64_t hkv, int64_t lq,
                                          int64_t lk, int64_t dim, int64_t q_sb, int64_t q_sh, int64_t q_sl,
                                          int64_t k_sb, int64_t k_sh, int64_t k_sl, int64_t o_sb, int64_t o_sh,
                                          int64_t o_sl, float sm_scale, int32_t kv_splits, void *partial,
                                          int64_t partial_bytes, void *stream) {
    using namespace tu;
    const int64_t tiles = (lk + kBKey - 1) / kBKey;
    TU_REQUIRE(kv_splits >= 1 && kv_splits <= tiles && kv_splits <= 256,
               "Sage attention: kv_splits must be in [1, min(key tiles, 256)], got %d", kv_splits);
    if (kv_splits == 1)
        return tu_sage_attn_fwd(q8, q_scale, blkq, k8, k_scale, blkk, vt_bf16, lpad, o_bf16, batch, hq, hkv, lq, lk,
                                dim, q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, o_sb, o_sh, o_sl, sm_scale, 0, stream);
    // every split non-empty: split_tiles = ceil(tiles / kv_splits), and the
    // number of splits that covers
    const int64_t split_tiles = (tiles + kv_splits - 1) / kv_splits;
    const int64_t splits = (tiles + split_tiles - 1) / split_tiles;
    const int64_t need = splits * batch * hq * lq * (dim + 2) * static_cast<int64_t>(sizeof(float));
    TU_REQUIRE(partial && (reinterpret_cast<uintptr_t>(partial) & 15) == 0 && partial_bytes >= need,
               "Sage attention split workspace must be 16-byte aligned and hold %lld bytes",
               static_cast<long long>(need));
    if (check_attn_args(q8, q_scale, blkq, k8, k_scale, blkk, vt_bf16, lpad, o_bf16, batch, hq, hkv, lq, lk, dim, q_sb,
                        q_sh, q_sl, k_sb, k_sh, k_sl, o_sb, o_sh, o_sl, sm_scale))
        return -1;
    const dim3 grid(static_cast<unsigned>((lq + kBQ - 1) / kBQ), static_cast<unsigned>(batch * hq),
                    static_cast<unsigned>(splits));
    hipStream_t s = static_cast<hipStream_t>(stream);
    int kscale_shift = 0;
    while ((kBKey << kscale_shift) < blkk) ++kscale_shift;
    float *part = static_cast<float *>(partial);
#define TU_SPLIT_ARGS                                                                                            \
    q8, q_scale, static_cast<int>(blkq), k8, k_scale, kscale_shift, static_cast<const uint16_t *>(vt_bf16),      \
        static_cast<uint16_t *>(o_bf16), static_cast<int>(hq), static_cast<int>(hq / hkv), lq, lk, lpad, q_sb,    \
        q_sh, q_sl, k_sb, k_sh, k_sl, o_sb, o_sh, o_sl, sm_scale * kLog2e, static_cast<int>(split_tiles), part
    const int64_t rows = batch * hq * lq;
    if (dim == 128) {
        sage_attn_kernel<128, false, true><<<grid, kThreads, 0, s>>>(TU_SPLIT_ARGS);
        sage_combine_kernel<128><<<static_cast<unsigned>((rows + 15) / 16), 256, 0, s>>>(
            part, static_cast<int>(splits), static_cast<int>(hq), batch * hq, lq, static_cast<uint16_t *>(o_bf16),
            o_sb, o_sh, o_sl);
    } else {
        sage_attn_kernel<64, false, true><<<grid, kThreads, 0, s>>>(TU_SPLIT_ARGS);
        sage_combine_kernel<64><<<static_cast<unsigned>((rows + 31) / 32), 256, 0, s>>>(
            part, static_cast<int>(splits), static_cast<int>(hq), batch * hq, lq, static_cast<uint16_t *>(o_bf16),
            o_sb, o_sh, o_sl);
    }
#undef TU_SPLIT_ARGS
    return check_launch("tu_sage_attn_fwd_split");
}
