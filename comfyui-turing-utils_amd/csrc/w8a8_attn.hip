// Dense W8A8 attention forward for gfx950: INT8 QK^T and INT8 PV on MFMA.
//
// Reference semantics: the ForceDense / UseW8A8 specialisation of
// sparse_attention_kernel (kernel/csrc/turing/sage/sol_sparse_cuda_sm75.cu
// :1182-1322) with update_mdo (exp offset), RS_to_u8, accumulate_d,
// compute_int8_sv_permuted and normalize_d (attn_utils.cuh:31-34, :436-568,
// :588-623, :676-703, :791-841, :920-973).  Per query row and key tile of 64:
//   s   = float(q8 . k8), masked keys (k >= Lk; causal k > q) -> -5e6
//   f   = (sm_scale * log2 e) * q_scale * k_scale[tile]
//   m'  = max(m, fma(max s, f, -log2 255));  O, d rescaled by 2^(m - m')
//   p   = 2^(fma(s, f, -m')),  P = cvt.rni.sat.u8(p),  d += p
//   O  += P . v8 (exact integer product)
//   out = O / d * v_scale[channel]
// The masked score is the reference's finite -5e6 in the raw score domain.
//
// MI355X mapping (shared with the Sage kernel: 8 wave64, two groups of 4
// whose MFMA and softmax clusters interleave, 32 query rows a wave, a
// 4-stage LDS ring filled by buffer_load ... lds from group 0):
//   * S^T = K Q^T on v_mfma_i32_16x16x64_i8 as in the Sage kernel, with the
//     K rows permuted so that lane group g holds the 16 consecutive keys
//     16 g .. 16 g + 15 of each query: exactly one 16-byte B operand of the
//     PV MFMA.
//   * O^T = V^T P on v_mfma_i32_16x16x64_i8 (one MFMA covers the whole
//     64-key tile).  CDNA4 multiplies signed x signed only, so P goes in as
//     127 - P (a signed byte for every P in [0, 255]), and one more MFMA per
//     fragment against a constant -127 operand adds -127 * sum_k v8.  The
//     accumulator then holds -(P . v8) exactly, with no V code sums to load.
//     v_cvt_pk_u8_f32 rounds p to an integer half-to-even into its byte of
//     the packed operand, and an XOR with 0x7f per byte turns P into 127 - P.
//   * The PV products stay in int32 accumulators across tiles and are
//     converted to fp32, per 16-row query fragment, only when the maximum
//     of one of its rows moves (the reference
//     rescales O every tile; a rescale by 2^0 is exact) or every 512 tiles
//     (int32 headroom: each key adds at most 255 * 127 in magnitude per
//     product, and 2 * 127 * 127 with the constant MFMA's term).
//   * V^T arrives channel-major as INT8 codes [d][key] (keys padded to a
//     multiple of 64 with zeros) from tu_w8a8_quant_v: the V^T stage is
//     8 KiB, half of the Sage kernel's bf16 stage.
#include <type_traits>

#include "attn_common.h"

namespace tu {
namespace {

constexpr int kThreads = 512;
constexpr int kD = 128;
constexpr int kQT = 2;
constexpr int kWaveQ = 16 * kQT;
constexpr int kBQ = 8 * kWaveQ;
constexpr int kBKey = 64;
constexpr int kKTileBytes = kBKey * kD;   // int8 K tile, 8 KiB
constexpr int kVTileBytes = kD * kBKey;   // int8 V^T tile, 8 KiB
constexpr int kStageBytes = kKTileBytes + kVTileBytes;
constexpr int kStages = 4;
constexpr int kAhead = kStages - 1;
constexpr int kLoadsPerTile = 4;          // per group-0 wave: 2 K + 2 V^T 1 KiB blocks
constexpr float kU8Offset = 7.9943534f;   // log2(255): the largest p is 255
constexpr int kFlushTiles = 512;          // int32 headroom of the PV accumulators
// Biased bit pattern of the masked raw score -5e6: the float kBiasF - 5e6.
constexpr float kMaskedF = kBiasF - 5000000.0f;

// K tile LDS row p = 16 kt + i holds key 16 (i >> 2) + 4 kt + (i & 3): QK
// output row 4 g + r of key block kt is key 16 g + 4 kt + r.
__device__ __forceinline__ int kperm8(int p) {
    const int i = p & 15, kt = p >> 4;
    return 16 * (i >> 2) + 4 * kt + (i & 3);
}

struct LaneGeom8 {
    uint32_t k_src[2];  // byte offset (from key0's row) of this lane's two K source chunks
    uint32_t v_src[2];  // byte offset (from key0's column) of this lane's two V^T source chunks
    uint32_t k_rd[2];   // LDS byte offset of the QK A operand, chunk 4 i + g
    uint32_t v_rd;      // LDS byte offset of the PV A operand (channel lc, keys 16 g ..)
};

// K rows are 128 B with 16-byte chunks XOR-swizzled by row bits 1..3.  A
// V^T block (16 channels x 64 keys) holds chunk (channel c, keys 16 g ..) at
// 16-byte position 16 g + 8 (c & 1) + (g ^ (c >> 1)), so a lane's PV read
// lands on the same position modulo 256 bytes as its K read of chunk column
// g: both reads are spread over the LDS banks alike.  (Plain 64-byte rows
// with a 2-bit XOR swizzle cost 4 bank-conflict cycles per V^T read.)
__device__ __forceinline__ LaneGeom8 lane_geom8(int wave, int lane, int64_t k_sl, int64_t lpad) {
    LaneGeom8 gm;
    const int g = lane >> 4, lc = lane & 15, sw = (lc >> 1) & 7;
    // the chunk that DMA lane `lane` writes to position `lane` of its block
    const int vc = 2 * ((lane & 7) ^ g) + ((lane >> 3) & 1);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int row = (2 * wave + i) * 8 + (lane >> 3);
        gm.k_src[i] = static_cast<uint32_t>(kperm8(row) * k_sl + ((lane & 7) ^ ((row >> 1) & 7)) * 16);
        gm.k_rd[i] = static_cast<uint32_t>(lc * 128 + (((4 * i + g) ^ sw) << 4));
        const int d = 16 * (2 * wave + i) + vc;
        gm.v_src[i] = static_cast<uint32_t>(d * lpad + 16 * g);
    }
    gm.v_rd = static_cast<uint32_t>(kKTileBytes + ((16 * g + 8 * (lc & 1) + (g ^ sw)) << 4));
    return gm;
}

// The K tile's key offset is part of the per-lane offset, which is what the
// buffer range check covers: K rows at or past lk read as zeros (masked
// keys).  V^T is padded to whole tiles, so its key offset stays scalar.
__device__ __forceinline__ void issue_tile8(int8_t *stage, __amdgpu_buffer_rsrc_t krs, __amdgpu_buffer_rsrc_t vrs,
                                            const LaneGeom8 &gm, uint32_t k_sl, uint32_t key0, int wave) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_void *)(stage + (2 * wave + i) * 1024), 16,
                                                 gm.k_src[i] + key0 * k_sl, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_void *)(stage + kKTileBytes + (2 * wave + i) * 1024), 16,
                                                 gm.v_src[i], key0, 0, 0);
}

__device__ __forceinline__ void qk_tile8(const int8_t *stage, const LaneGeom8 &gm, const i32x4 (&qf)[kQT][2],
                                         i32x4 (&s)[4][kQT]) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
        const i32x4 kf0 = *reinterpret_cast<const i32x4 *>(stage + gm.k_rd[0] + kt * 16 * 128);
        const i32x4 kf1 = *reinterpret_cast<const i32x4 *>(stage + gm.k_rd[1] + kt * 16 * 128);
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
            const i32x4 z = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf0, qf[qt][0], i32x4{kBias, kBias, kBias, kBias},
                                                                  0, 0, 0);
            s[kt][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf1, qf[qt][1], z, 0, 0, 0);
        }
    }
}

// Wave softmax state.  acc_i[.][qt] holds -(P . v8) of tiles [seg[qt],
// current) in int32; each 16-row query fragment qt has its own segment.  acc_o and l are kept at a fixed
// exponent base per query, the first one: a segment computed at base m_used
// enters them scaled by beta = 2^(m_used - that base), so a move of the
// running maximum rescales nothing (O / l does not depend on the base).  The
// fixed base moves up to m_used, with acc_o and l rescaled, only when beta
// passes kRebase.
struct W8State {
    float m_used[kQT];
    float beta[kQT];
    float l[kQT];
    f32x4 acc_o[8][kQT];
    i32x4 acc_i[8][kQT];
    int seg[kQT];
};
constexpr float kRebase = 0x1p64f;

template <bool kCausal>
__device__ __forceinline__ void mask_tile8(i32x4 (&s)[4][kQT], int key_lim, int q_rel, int g, int lc) {
    const int masked = __float_as_int(kMaskedF);
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        // key = 16 g + c with c = 4 kt + r; masked iff c > t
        int t = key_lim - 1 - 16 * g;
        if constexpr (kCausal) t = min(t, q_rel + 16 * qt + lc - 16 * g);
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int c = 4 * kt + r;
                const int m = (t - c) >> 31;
                s[kt][qt][r] = (s[kt][qt][r] & ~m) | (masked & m);
            }
    }
}

// Adds fragment qt's int32 segment [st.seg[qt], tile) to acc_o: acc_i holds
// -(P . v8) exactly, so acc_o += float(acc_i) * -beta; then clears acc_i.
template <int qt>
__device__ __forceinline__ void flush_fragment(W8State &st, int tile) {
    if (tile > st.seg[qt]) {
#pragma unroll
        for (int ds = 0; ds < 8; ++ds) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
                st.acc_o[ds][qt][r] =
                    __builtin_fmaf(static_cast<float>(st.acc_i[ds][qt][r]), -st.beta[qt], st.acc_o[ds][qt][r]);
            st.acc_i[ds][qt] = i32x4{0, 0, 0, 0};
        }
    }
    st.seg[qt] = tile;
}

// Flushes both fragments (at the end of the key range).
__device__ __forceinline__ void flush_segment(W8State &st, int tile) {
    flush_fragment<0>(st, tile);
    flush_fragment<1>(st, tile);
}

// The reference's exact running maximum of fragment qt: when some row's
// maximum moves (or the int32 headroom runs out), only this fragment's
// segment is flushed.
template <int qt>
__device__ __forceinline__ void move_max(W8State &st, const float (&mlane)[kQT], int tile) {
    if (__any(mlane[qt] > st.m_used[qt]) || tile - st.seg[qt] >= kFlushTiles) {
        flush_fragment<qt>(st, tile);
        const float mx = xmax_f32(mlane[qt]);
        const float m_new = mx > st.m_used[qt] ? mx : st.m_used[qt];
        // the first tile fixes the base (acc_o and l are still 0)
        st.beta[qt] = st.m_used[qt] == -INFINITY ? 1.0f
                                                 : st.beta[qt] * __builtin_amdgcn_exp2f(m_new - st.m_used[qt]);
        st.m_used[qt] = m_new;
        if (__any(st.beta[qt] > kRebase)) {
            const float alpha = 1.0f / st.beta[qt];
            st.beta[qt] = 1.0f;
            st.l[qt] *= alpha;
#pragma unroll
            for (int ds = 0; ds < 8; ++ds) st.acc_o[ds][qt] *= alpha;
        }
    }
}

// The constant PV operand: -127 in every byte.
__device__ __forceinline__ i32x4 neg127_operand() {
    constexpr int32_t kNeg127x4 = static_cast<int32_t>(0x81818181u);
    return i32x4{kNeg127x4, kNeg127x4, kNeg127x4, kNeg127x4};
}

// Softmax of tile `tile`: new row maxima (with the u8 offset), flush and
// rescale when one moved, then 127 - P packed as the PV B operands p8[qt]
// (dword kt = keys 16 g + 4 kt .. + 3 of query 16 qt + lc) and l += p.
__device__ __forceinline__ void softmax_tile8(const i32x4 (&s)[4][kQT], const float (&f)[kQT], W8State &st,
                                              i32x4 (&p8)[kQT], int tile) {
    float mlane[kQT];
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
        mlane[qt] = __builtin_fmaf(__int_as_float(mi) - kBiasF, f[qt], -kU8Offset);
    }
    move_max<0>(st, mlane, tile);
    move_max<1>(st, mlane, tile);
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
            float lsum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                uint32_t packed = 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float v = __int_as_float(s[kt][qt][r]);
                    const float x = decltype(exact_tag)::value ? __builtin_fmaf(v - kBiasF, f[qt], nm)
                                                               : __builtin_fmaf(v, f[qt], c[qt]);
                    const float p = __builtin_amdgcn_exp2f(x);
                    lsum = kt == 0 && r == 0 ? p : lsum + p;
                    // byte r = rint(p): v_cvt_pk_u8_f32 rounds half to even
                    // (checked against rint on every float in [0, 256]); p
                    // <= 255 since the base sits log2(255) above the maximum
                    packed = __builtin_amdgcn_cvt_pk_u8_f32(p, r, packed);
                }
                // 127 - P as signed bytes for the signed-only MFMA
                p8[qt][kt] = static_cast<int32_t>(packed ^ 0x7f7f7f7fu);
            }
            st.l[qt] = __builtin_fmaf(lsum, st.beta[qt], st.l[qt]);
        }
    };
    if (__any(exact)) make_p(std::true_type{});
    else make_p(std::false_type{});
}

__device__ __forceinline__ void pv_tile8(const int8_t *stage, const LaneGeom8 &gm, const i32x4 (&p8)[kQT],
                                         W8State &st) {
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) {
        const i32x4 vf = *reinterpret_cast<const i32x4 *>(stage + gm.v_rd + ds * 16 * 64);
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
            st.acc_i[ds][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(vf, p8[qt], st.acc_i[ds][qt], 0, 0, 0);
            st.acc_i[ds][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(vf, neg127_operand(), st.acc_i[ds][qt], 0, 0, 0);
        }
    }
}

// Steady-state MFMA cluster: QK^T of the tile in kst, PV of the tile in vst.
__device__ __forceinline__ void mfma_cluster8(const int8_t *kst, const int8_t *vst, const LaneGeom8 &gm,
                                              const i32x4 (&qf)[kQT][2], i32x4 (&s)[4][kQT], const i32x4 (&p8)[kQT],
                                              W8State &st) {
    // PV first: the V^T fragments and P die before the K fragments and the
    // S accumulators come alive, which keeps the two accumulator sets (int32
    // PV, fp32 O) resident without spills.
    i32x4 vf[8];
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) vf[ds] = *reinterpret_cast<const i32x4 *>(vst + gm.v_rd + ds * 16 * 64);
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
            st.acc_i[ds][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(vf[ds], p8[qt], st.acc_i[ds][qt], 0, 0, 0);
            st.acc_i[ds][qt] =
                __builtin_amdgcn_mfma_i32_16x16x64_i8(vf[ds], neg127_operand(), st.acc_i[ds][qt], 0, 0, 0);
        }
    i32x4 kf[4][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) kf[kt][i] = *reinterpret_cast<const i32x4 *>(kst + gm.k_rd[i] + kt * 16 * 128);
    i32x4 z[4][kQT];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
            z[kt][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[kt][0], qf[qt][0], i32x4{kBias, kBias, kBias, kBias},
                                                              0, 0, 0);
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
            s[kt][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf[kt][1], qf[qt][1], z[kt][qt], 0, 0, 0);
    // V^T reads (first half), K reads of the first QK^T half, V^T second
    // half, PV MFMAs, K second half, QK^T MFMAs.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
}

// Schedule of the Sage kernel (see sage_attn.hip): per key tile t an MFMA
// cluster {QK(t+1), PV(t)} and a VALU cluster {softmax(t+1)}, one barrier
// per tile, the two groups' barriers on either side of the softmax.
template <bool kCausal, bool kFp16Out>
__global__ __launch_bounds__(kThreads, 1) void w8a8_attn_kernel(
    const int8_t *__restrict__ q8, const float *__restrict__ q_scale, const int8_t *__restrict__ k8,
    const float *__restrict__ k_scale, const int8_t *__restrict__ vt, const float *__restrict__ v_scale,
    uint16_t *__restrict__ o, int hq, int groups, int64_t lq, int64_t lk,
    int64_t lpad, int64_t nqs, int64_t nks, int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb, int64_t k_sh,
    int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl, float sm_log2) {
    __shared__ __align__(1024) int8_t lds[kStages][kStageBytes];

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
    const int8_t *vtp = vt + (b * hkv + hk) * kD * lpad;
    const float *ks_row = k_scale + (b * hkv + hk) * nks;

    int64_t key_end = lk;
    if constexpr (kCausal) key_end = min(lk, qblock0 + kBQ);
    const int tiles = static_cast<int>((key_end + kBKey - 1) / kBKey);
    int my_tiles = tiles;
    if constexpr (kCausal)
        my_tiles = static_cast<int>(min<int64_t>(tiles, max<int64_t>(1, (min(q0 + kWaveQ, lq) + kBKey - 1) / kBKey)));
    int64_t mask_from = lk / kBKey;
    if constexpr (kCausal) mask_from = min(mask_from, q0 / kBKey);
    const int first_masked = static_cast<int>(min<int64_t>(tiles, mask_from));

    const LaneGeom8 gm = lane_geom8(w4, lane, k_sl, lpad);
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kp, static_cast<uint32_t>(lk * k_sl));
    const __amdgpu_buffer_rsrc_t vrs = make_rsrc(vtp, static_cast<uint32_t>(kD * lpad));
    const uint32_t k_sl32 = static_cast<uint32_t>(k_sl);
    auto tile_key0 = [&](int it) { return static_cast<uint32_t>(min(it, tiles - 1) * kBKey); };

    i32x4 qf[kQT][2];
    float qsc[kQT];
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        const int64_t qi = min(q0 + 16 * qt + lc, lq - 1);
#pragma unroll
        for (int ds = 0; ds < 2; ++ds)
            qf[qt][ds] = *reinterpret_cast<const i32x4 *>(qp + qi * q_sl + 64 * ds + 16 * g);
        qsc[qt] = sm_log2 * q_scale[(b * hq + h) * nqs + qi / 16];
    }
    if (grp == 0) {
#pragma unroll
        for (int j = 0; j < kAhead; ++j) issue_tile8(lds[j], krs, vrs, gm, k_sl32, tile_key0(j), w4);
    }
    W8State st;
    st.seg[0] = st.seg[1] = 0;
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        st.m_used[qt] = -INFINITY;
        st.beta[qt] = 1.0f;
        st.l[qt] = 0.0f;
#pragma unroll
        for (int ds = 0; ds < 8; ++ds) {
            st.acc_o[ds][qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            st.acc_i[ds][qt] = i32x4{0, 0, 0, 0};
        }
    }

    i32x4 s[4][kQT];
    i32x4 p8[kQT];

    auto softmax = [&](int it, auto mask_tag) {
        const float kscale = ks_row[it];
        float f[kQT];
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) f[qt] = qsc[qt] * kscale;
        if (decltype(mask_tag)::value && it >= first_masked) {
            const int64_t key0 = static_cast<int64_t>(it) * kBKey;
            const int key_lim = static_cast<int>(min(lk - key0, static_cast<int64_t>(kBKey)));
            const int q_rel =
                static_cast<int>(max(min(q0 - key0, static_cast<int64_t>(kBKey)), static_cast<int64_t>(-kBQ)));
            mask_tile8<kCausal>(s, key_lim, q_rel, g, lc);
        }
        softmax_tile8(s, f, st, p8, it);
    };

    // The schedule of the Sage kernel (sage_attn.hip): one barrier per key
    // tile; both groups run M_it = {QK(it + 1), PV(it)} then softmax(it + 1),
    // group 0's barrier after the softmax, group 1's before it, so the two
    // groups' MFMA clusters overlap on each SIMD.  Group 0 issues the next
    // tile's loads between its MFMA and softmax clusters, as there.
    if (grp == 0) __builtin_amdgcn_s_waitcnt(vmcnt_imm((kAhead - 1) * kLoadsPerTile));
    wg_barrier();
    qk_tile8(lds[0], gm, qf, s);
    const int main_steps = max(0, min(my_tiles, first_masked) - 1);
    if (grp == 0) {
        softmax(0, std::true_type{});
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((kAhead - 2) * kLoadsPerTile));
    }
    wg_barrier();
    if (grp == 1) softmax(0, std::true_type{});
#pragma clang loop unroll(disable)
    for (int it = 0; it < main_steps; ++it) {
        mfma_cluster8(lds[(it + 1) % kStages], lds[it % kStages], gm, qf, s, p8, st);
        if (grp == 0) issue_tile8(lds[(it + kAhead) % kStages], krs, vrs, gm, k_sl32, tile_key0(it + kAhead), w4);
        if (grp == 1) wg_barrier();
        softmax(it + 1, std::false_type{});
        if (grp == 0) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((kAhead - 2) * kLoadsPerTile));
            wg_barrier();
        }
    }
#pragma clang loop unroll(disable)
    for (int it = main_steps; it < tiles; ++it) {
        if (it + 1 < my_tiles) qk_tile8(lds[(it + 1) % kStages], gm, qf, s);
        if (it < my_tiles) pv_tile8(lds[it % kStages], gm, p8, st);
        if (grp == 0) issue_tile8(lds[(it + kAhead) % kStages], krs, vrs, gm, k_sl32, tile_key0(it + kAhead), w4);
        if (grp == 1) wg_barrier();
        if (it + 1 < my_tiles) softmax(it + 1, std::true_type{});
        if (grp == 0) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((kAhead - 2) * kLoadsPerTile));
            wg_barrier();
        }
    }
    __builtin_amdgcn_s_waitcnt(0);

    // Final segment, then out = O / l * v_scale.  acc_o[ds][qt][r] holds
    // O^T[16 ds + 4 g + r][q0 + 16 qt + lc].
    flush_segment(st, my_tiles);
    const float *vs = v_scale + (b * hkv + hk) * kD + 4 * g;
    uint16_t *op = o + b * o_sb + h * o_sh;
#pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
        const int64_t qi = q0 + 16 * qt + lc;
        const float inv = 1.0f / xsum_f32(st.l[qt]);
        if (qi >= lq) continue;
#pragma unroll
        for (int ds = 0; ds < 8; ++ds) {
            const f32x4 sc = *reinterpret_cast<const f32x4 *>(vs + 16 * ds);
            float y[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) y[r] = (st.acc_o[ds][qt][r] * inv) * sc[r];
            u32x2 packed;
            if constexpr (kFp16Out) {
                packed.x = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(y[0]))) |
                           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(y[1]))) << 16);
                packed.y = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(y[2]))) |
                           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(y[3]))) << 16);
            } else {
                packed.x = pack_bf16x2(y[0], y[1]);
                packed.y = pack_bf16x2(y[2], y[3]);
            }
            *reinterpret_cast<u32x2 *>(op + qi * o_sl + 16 * ds + 4 * g) = packed;
        }
    }
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_w8a8_attn_fwd(const int8_t *q8, const float *q_scale, int64_t nqs, const int8_t *k8,
                                    const float *k_scale, int64_t nks, const int8_t *vt, const float *v_scale,
                                    int64_t lpad, void *out, int32_t out_fp16,
                                    int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk, int64_t dim,
                                    int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb, int64_t k_sh,
                                    int64_t k_sl, int64_t o_sb, int64_t o_sh, int64_t o_sl, float sm_scale,
                                    int32_t causal, void *stream) {
    using namespace tu;
    TU_REQUIRE(dim == kD, "W8A8 attention kernel requires head_dim 128, got %lld", static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "W8A8 attention: hq must be a positive multiple of hkv");
    TU_REQUIRE(lq > 0 && lk > 0, "W8A8 attention requires non-empty sequences");
    TU_REQUIRE(lpad == (lk + kBKey - 1) / kBKey * kBKey, "W8A8 attention: V^T padded length must be ceil(lk/64)*64");
    TU_REQUIRE(nqs >= (lq + 15) / 16 && nks >= (lk + kBKey - 1) / kBKey, "W8A8 attention scale rows too short");
    TU_REQUIRE((lq + kBQ - 1) / kBQ <= 0x7fffffff && batch * hq <= 65535, "W8A8 attention grid too large");
    TU_REQUIRE(lk * k_sl < (int64_t{1} << 32) && kD * lpad < (int64_t{1} << 32),
               "W8A8 attention: one head's K or V^T exceeds 4 GiB of addressable bytes");
    TU_REQUIRE(q8 && q_scale && k8 && k_scale && vt && v_scale && out,
               "W8A8 attention pointers must be non-null");
    TU_REQUIRE(sm_scale > 0.0f, "W8A8 attention sm_scale must be positive");
    TU_REQUIRE(q_sl % 16 == 0 && q_sh % 16 == 0 && q_sb % 16 == 0 && (reinterpret_cast<uintptr_t>(q8) & 15) == 0 &&
                   k_sl % 16 == 0 && k_sh % 16 == 0 && k_sb % 16 == 0 && (reinterpret_cast<uintptr_t>(k8) & 15) == 0,
               "W8A8 attention Q/K rows must be 16-byte aligned");
    TU_REQUIRE((reinterpret_cast<uintptr_t>(vt) & 15) == 0 && (reinterpret_cast<uintptr_t>(v_scale) & 15) == 0 &&
                   o_sl % 4 == 0 && o_sh % 4 == 0 &&
                   o_sb % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0,
               "W8A8 attention V^T/scales/O must be aligned");
    if (require_gfx950()) return -1;
    const dim3 grid(static_cast<unsigned>((lq + kBQ - 1) / kBQ), static_cast<unsigned>(batch * hq));
    const float sm_log2 = sm_scale * kLog2e;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int groups = static_cast<int>(hq / hkv);
#define TU_W8_ARGS                                                                                            \
    q8, q_scale, k8, k_scale, vt, v_scale, static_cast<uint16_t *>(out), static_cast<int>(hq), groups,           \
        lq, lk, lpad, nqs, nks, q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, o_sb, o_sh, o_sl, sm_log2
    if (causal) {
        if (out_fp16) w8a8_attn_kernel<true, true><<<grid, kThreads, 0, s>>>(TU_W8_ARGS);
        else w8a8_attn_kernel<true, false><<<grid, kThreads, 0, s>>>(TU_W8_ARGS);
    } else {
        if (out_fp16) w8a8_attn_kernel<false, true><<<grid, kThreads, 0, s>>>(TU_W8_ARGS);
        else w8a8_attn_kernel<false, false><<<grid, kThreads, 0, s>>>(TU_W8_ARGS);
    }
#undef TU_W8_ARGS
    return check_launch("tu_w8a8_attn_fwd");
}
