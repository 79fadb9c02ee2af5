// Sage INT8 attention forward for gfx950: INT8 QK^T on MFMA, online softmax
// in base 2, P rounded to bf16, PV on bf16 MFMA with fp32 accumulation.
//
// Reference semantics: qk_int_sv_f16_attn_kernel
// (kernel/csrc/turing/sage/qk_int_sv_f16_cuda_sm75.cu:48-830) with
// update_mdo / normalize_d (sage/attn_utils.cuh:464-568, :920-973):
//   s   = float(q8 . k8) * (sm_scale * log2 e) * q_scale * k_scale
//   m   = running row max of s;  p = 2^(s - m);  O = O * 2^(m_old - m) + P V
//   out = O / sum(P)
// The reference rounds P to fp16 for its Turing fp16 MMA; here P is rounded
// to bf16 for the CDNA4 bf16 MFMA, and the row sum adds the rounded values.
//
// MI355X mapping
//   * Workgroup = 4 wave64 = 256 query rows (64 per wave) of one (batch, head);
//     keys are streamed in tiles of 64 through a double-buffered LDS.
//   * S^T = K Q^T with v_mfma_i32_16x16x64_i8 (K tile from LDS as the A
//     operand, the wave's Q rows resident in registers as the B operand), so
//     each lane holds 4 keys x 1 query per 16x16 block: the row max and row
//     sum are in-register reductions plus two cross-lane steps (xor 16, 32).
//   * O^T = V^T P with v_mfma_f32_16x16x32_bf16: P is consumed straight from
//     registers as the B operand (the MFMA's K index runs over the lane's own
//     keys {4g..4g+3, 16+4g..16+4g+3}); V is transposed into LDS as
//     V^T[d][key] while it is staged, so the A operand is two 8-byte reads.
//   * K tile rows are 128 B with 16-byte chunks XOR-swizzled by key bits 1..3;
//     V^T rows are 128 B with 8-byte chunks XOR-swizzled by d bits 0..3.
#include "tu_common.h"

namespace tu {
namespace {

constexpr int kThreads = 256;
constexpr int kD = 128;
constexpr int kBQ = 256;       // query rows per workgroup
constexpr int kWaveQ = 64;     // query rows per wave
constexpr int kBKey = 64;      // keys per tile
constexpr int kKTileBytes = kBKey * kD;       // int8 K tile
constexpr int kVTileBytes = kBKey * kD * 2;   // bf16 V^T tile
constexpr float kLog2e = 1.4426950408889634f;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int k_lds_off(int key, int chunk) { return key * kD + ((chunk ^ ((key >> 1) & 7)) << 4); }
// V^T[d][key]: 64 keys = 16 chunks of 4 keys (8 B) per d row.
__device__ __forceinline__ int v_lds_off(int d, int kchunk) { return d * (kBKey * 2) + ((kchunk ^ (d & 15)) << 3); }

struct KVLoad {
    i32x4 k[2];
    u32x4 v[4];
};

__device__ __forceinline__ void load_kv(KVLoad &t, const int8_t *__restrict__ kp, const uint16_t *__restrict__ vp,
                                        int64_t k_sl, int64_t v_sl, int64_t key0, int64_t lk, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int id = tid + kThreads * i;
        const int key = id >> 3, chunk = id & 7;
        const int64_t kk = min(key0 + key, lk - 1);
        t.k[i] = *reinterpret_cast<const i32x4 *>(kp + kk * k_sl + chunk * 16);
    }
    const int kg = tid & 15, dg = tid >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t key = key0 + 4 * kg + i;
        if (key < lk) t.v[i] = *reinterpret_cast<const u32x4 *>(vp + key * v_sl + dg * 8);
        else t.v[i] = u32x4{0u, 0u, 0u, 0u};
    }
}

__device__ __forceinline__ void store_kv(const KVLoad &t, int8_t *lds_k, uint16_t *lds_v, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int id = tid + kThreads * i;
        const int key = id >> 3, chunk = id & 7;
        *reinterpret_cast<i32x4 *>(lds_k + k_lds_off(key, chunk)) = t.k[i];
    }
    // Transpose 4 keys x 8 channels to 8 channels x 4 keys.
    const int kg = tid & 15, dg = tid >> 4;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t a0 = t.v[0][p], a1 = t.v[1][p], a2 = t.v[2][p], a3 = t.v[3][p];
        u32x2 lo, hi;
        lo.x = (a0 & 0xffffu) | (a1 << 16);
        lo.y = (a2 & 0xffffu) | (a3 << 16);
        hi.x = (a0 >> 16) | (a1 & 0xffff0000u);
        hi.y = (a2 >> 16) | (a3 & 0xffff0000u);
        const int d = dg * 8 + 2 * p;
        *reinterpret_cast<u32x2 *>(reinterpret_cast<int8_t *>(lds_v) + v_lds_off(d, kg)) = lo;
        *reinterpret_cast<u32x2 *>(reinterpret_cast<int8_t *>(lds_v) + v_lds_off(d + 1, kg)) = hi;
    }
}

__device__ __forceinline__ float xmax(float v) {
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}

__device__ __forceinline__ float xsum(float v) {
    v = v + __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

template <bool kCausal>
__global__ __launch_bounds__(kThreads, 1) void sage_attn_kernel(
    const int8_t *__restrict__ q8, const float *__restrict__ q_scale, int blkq, const int8_t *__restrict__ k8,
    const float *__restrict__ k_scale, int blkk, const uint16_t *__restrict__ v, uint16_t *__restrict__ o,
    int hq, int groups, int64_t lq, int64_t lk, int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb,
    int64_t k_sh, int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl, int64_t o_sb, int64_t o_sh,
    int64_t o_sl, float sm_log2) {
    __shared__ __align__(16) int8_t lds_k[2][kKTileBytes];
    __shared__ __align__(16) uint16_t lds_v[2][kVTileBytes / 2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;     // lane group: keys 4g..4g+3 of each 16-key block
    const int lc = lane & 15;    // query column inside a 16-query block

    const int64_t bh = blockIdx.y;  // batch * hq + head
    const int64_t b = bh / hq, h = bh % hq, hk = h / groups;
    const int64_t hkv = hq / groups;
    const int64_t q0 = static_cast<int64_t>(blockIdx.x) * kBQ + wave * kWaveQ;

    const int8_t *qp = q8 + b * q_sb + h * q_sh;
    const int8_t *kp = k8 + b * k_sb + hk * k_sh;
    const uint16_t *vp = v + b * v_sb + hk * v_sh;
    const int64_t nbq = (lq + blkq - 1) / blkq;
    const int64_t nbk = (lk + blkk - 1) / blkk;

    // Q operand: qf[qt][ds], lane -> query q0 + 16 qt + lc, channels 64 ds + 16 g .. +15.
    i32x4 qf[4][2];
    float qsc[4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
        const int64_t qi = min(q0 + 16 * qt + lc, lq - 1);
#pragma unroll
        for (int ds = 0; ds < 2; ++ds)
            qf[qt][ds] = *reinterpret_cast<const i32x4 *>(qp + qi * q_sl + 64 * ds + 16 * g);
        qsc[qt] = q_scale[(b * hq + h) * nbq + qi / blkq] * sm_log2;
    }

    f32x4 acc_o[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc_o[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run[4], l_run[4];
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
        m_run[qt] = -INFINITY;
        l_run[qt] = 0.0f;
    }

    int64_t key_end = lk;
    if constexpr (kCausal) key_end = min(lk, static_cast<int64_t>(blockIdx.x) * kBQ + kBQ);
    const int tiles = static_cast<int>((key_end + kBKey - 1) / kBKey);
    const float *ks_row = k_scale + (b * hkv + hk) * nbk;

    KVLoad t;
    load_kv(t, kp, vp, k_sl, v_sl, 0, lk, tid);
    store_kv(t, lds_k[0], lds_v[0], tid);
    __syncthreads();

    for (int it = 0; it < tiles; ++it) {
        const int cur = it & 1;
        const int64_t key0 = static_cast<int64_t>(it) * kBKey;
        if (it + 1 < tiles) load_kv(t, kp, vp, k_sl, v_sl, key0 + kBKey, lk, tid);

        // S^T = K Q^T: s[kt][qt][r] = S[key0 + 16 kt + 4 g + r][q0 + 16 qt + lc].
        i32x4 s[4][4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            const i32x4 kf0 = *reinterpret_cast<const i32x4 *>(lds_k[cur] + k_lds_off(16 * kt + lc, g));
            const i32x4 kf1 = *reinterpret_cast<const i32x4 *>(lds_k[cur] + k_lds_off(16 * kt + lc, 4 + g));
#pragma unroll
            for (int qt = 0; qt < 4; ++qt) {
                i32x4 z = i32x4{0, 0, 0, 0};
                z = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf0, qf[qt][0], z, 0, 0, 0);
                s[kt][qt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf1, qf[qt][1], z, 0, 0, 0);
            }
        }

        const float kscale = ks_row[key0 / blkk];
        const bool tail = key0 + kBKey > lk;
        // Online softmax per query block; P packed as bf16 B operands.
        bf16x8 pf[2][4];
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) {
            const float f = qsc[qt] * kscale;
            const int64_t qi = q0 + 16 * qt + lc;
            float sf[4][4];
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float x = static_cast<float>(s[kt][qt][r]);
                    const int64_t key = key0 + 16 * kt + 4 * g + r;
                    bool masked = tail && key >= lk;
                    if constexpr (kCausal) masked = masked || key > qi;
                    x = masked ? -INFINITY : x;
                    sf[kt][r] = x;
                    mx = fmaxf(mx, x);
                }
            mx = xmax(mx);
            const float m_new = fmaxf(m_run[qt], mx * f);
            const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
            m_run[qt] = m_new;
            float lsum = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                f32x4 p;
#pragma unroll
                for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sf[kt][r], f, -m_new));
                const f32x2 p01 = f32x2{p[0], p[1]};
                const f32x2 p23 = f32x2{p[2], p[3]};
                const bf16x2_t b01 = __builtin_convertvector(p01, bf16x2_t);
                const bf16x2_t b23 = __builtin_convertvector(p23, bf16x2_t);
                pf[kt >> 1][qt][4 * (kt & 1) + 0] = b01[0];
                pf[kt >> 1][qt][4 * (kt & 1) + 1] = b01[1];
                pf[kt >> 1][qt][4 * (kt & 1) + 2] = b23[0];
                pf[kt >> 1][qt][4 * (kt & 1) + 3] = b23[1];
                lsum += (static_cast<float>(b01[0]) + static_cast<float>(b01[1])) +
                        (static_cast<float>(b23[0]) + static_cast<float>(b23[1]));
            }
            l_run[qt] = l_run[qt] * alpha + lsum;
#pragma unroll
            for (int ds = 0; ds < 8; ++ds) acc_o[ds][qt] *= alpha;
        }

        // O^T += V^T P over the tile's two 32-key halves.
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int ds = 0; ds < 8; ++ds) {
                const int d = 16 * ds + lc;
                const u32x2 lo = *reinterpret_cast<const u32x2 *>(reinterpret_cast<const int8_t *>(lds_v[cur]) +
                                                                  v_lds_off(d, 8 * ks + g));
                const u32x2 hi = *reinterpret_cast<const u32x2 *>(reinterpret_cast<const int8_t *>(lds_v[cur]) +
                                                                  v_lds_off(d, 8 * ks + 4 + g));
                u32x4 raw;
                raw.x = lo.x;
                raw.y = lo.y;
                raw.z = hi.x;
                raw.w = hi.y;
                const bf16x8 vf = __builtin_bit_cast(bf16x8, raw);
#pragma unroll
                for (int qt = 0; qt < 4; ++qt)
                    acc_o[ds][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[ks][qt], acc_o[ds][qt], 0, 0, 0);
            }
        }

        if (it + 1 < tiles) store_kv(t, lds_k[cur ^ 1], lds_v[cur ^ 1], tid);
        __syncthreads();
    }

    // acc_o[ds][qt][r] = O[q0 + 16 qt + lc][16 ds + 4 g + r].
    uint16_t *op = o + b * o_sb + h * o_sh;
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
        const int64_t qi = q0 + 16 * qt + lc;
        const float inv = 1.0f / xsum(l_run[qt]);
        if (qi >= lq) continue;
#pragma unroll
        for (int ds = 0; ds < 8; ++ds) {
            u32x2 packed;
            packed.x = pack_bf16x2(acc_o[ds][qt][0] * inv, acc_o[ds][qt][1] * inv);
            packed.y = pack_bf16x2(acc_o[ds][qt][2] * inv, acc_o[ds][qt][3] * inv);
            *reinterpret_cast<u32x2 *>(op + qi * o_sl + 16 * ds + 4 * g) = packed;
        }
    }
}

}  // namespace
}  // namespace tu

extern "C" int32_t tu_sage_attn_fwd(const int8_t *q8, const float *q_scale, int64_t blkq, const int8_t *k8,
                                    const float *k_scale, int64_t blkk, const void *v_bf16, void *o_bf16,
                                    int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk, int64_t dim,
                                    int64_t q_sb, int64_t q_sh, int64_t q_sl, int64_t k_sb, int64_t k_sh,
                                    int64_t k_sl, int64_t v_sb, int64_t v_sh, int64_t v_sl, int64_t o_sb,
                                    int64_t o_sh, int64_t o_sl, float sm_scale, int32_t causal, void *stream) {
    using namespace tu;
    TU_REQUIRE(dim == kD, "Sage attention kernel requires head_dim 128, got %lld", static_cast<long long>(dim));
    TU_REQUIRE(batch > 0 && hq > 0 && hkv > 0 && hq % hkv == 0, "Sage attention: hq must be a positive multiple of hkv");
    TU_REQUIRE(lq > 0 && lk > 0, "Sage attention requires non-empty sequences");
    TU_REQUIRE(blkq > 0 && blkk > 0 && blkk % kBKey == 0, "Sage attention needs blkq > 0 and blkk %% 64 == 0");
    TU_REQUIRE(blkq <= 0x7fffffff && blkk <= 0x7fffffff, "Sage attention block sizes out of range");
    TU_REQUIRE((lq + kBQ - 1) / kBQ <= 0x7fffffff && batch * hq <= 65535, "Sage attention grid too large");
    TU_REQUIRE(q8 && q_scale && k8 && k_scale && v_bf16 && o_bf16, "Sage attention pointers must be non-null");
    TU_REQUIRE(sm_scale > 0.0f, "Sage attention sm_scale must be positive");
    TU_REQUIRE(q_sl % 16 == 0 && q_sh % 16 == 0 && q_sb % 16 == 0 && (reinterpret_cast<uintptr_t>(q8) & 15) == 0 &&
                   k_sl % 16 == 0 && k_sh % 16 == 0 && k_sb % 16 == 0 && (reinterpret_cast<uintptr_t>(k8) & 15) == 0,
               "Sage attention Q/K rows must be 16-byte aligned");
    TU_REQUIRE(v_sl % 8 == 0 && v_sh % 8 == 0 && v_sb % 8 == 0 && (reinterpret_cast<uintptr_t>(v_bf16) & 15) == 0 &&
                   o_sl % 4 == 0 && o_sh % 4 == 0 && o_sb % 4 == 0 && (reinterpret_cast<uintptr_t>(o_bf16) & 7) == 0,
               "Sage attention V/O rows must be aligned");
    if (require_gfx950()) return -1;
    const dim3 grid(static_cast<unsigned>((lq + kBQ - 1) / kBQ), static_cast<unsigned>(batch * hq));
    const float sm_log2 = sm_scale * kLog2e;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int groups = static_cast<int>(hq / hkv);
#define TU_ATTN_ARGS                                                                                           \
    q8, q_scale, static_cast<int>(blkq), k8, k_scale, static_cast<int>(blkk),                                  \
        static_cast<const uint16_t *>(v_bf16), static_cast<uint16_t *>(o_bf16), static_cast<int>(hq), groups, \
        lq, lk, q_sb, q_sh, q_sl, k_sb, k_sh, k_sl, v_sb, v_sh, v_sl, o_sb, o_sh, o_sl, sm_log2
    if (causal) sage_attn_kernel<true><<<grid, kThreads, 0, s>>>(TU_ATTN_ARGS);
    else sage_attn_kernel<false><<<grid, kThreads, 0, s>>>(TU_ATTN_ARGS);
#undef TU_ATTN_ARGS
    return check_launch("tu_sage_attn_fwd");
}
